// Bit-exact dequantization of one element of a GGUF block, and the
// deterministic block quantizer.
//
// Dequantization follows crates/inferi/src/quantization.rs (Q8_0 :47-55,
// Q6_K :224-257, Q5_K :287-330, Q4_K :358-392, get_scale_min_k4 :394-402,
// decode_f16 :405-422).  Rust evaluates `d1 * q - m1` as three separately
// rounded f32 operations and never contracts them into an FMA, so
// contraction is switched off in every function here.
#pragma once
#include "common.h"

namespace ifr {

IFR_DEV uint32_t rd8(const uint8_t *p) { return *p; }

// Q4_K: d@0 dmin@2 scales[12]@4 qs[128]@16; element e = 64g + 32hi + l.
IFR_DEV float deq_q4k(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    uint32_t g = e >> 6, hi = (e >> 5) & 1u, l = e & 31u;
    float d = f16_to_f32(ld_u16(blk)), dmin = f16_to_f32(ld_u16(blk + 2));
    const uint8_t *s = blk + 4;
    uint32_t w0 = rd8(s) | rd8(s + 1) << 8 | rd8(s + 2) << 16 | rd8(s + 3) << 24;
    uint32_t w1 = rd8(s + 4) | rd8(s + 5) << 8 | rd8(s + 6) << 16 | rd8(s + 7) << 24;
    uint32_t w2 = rd8(s + 8) | rd8(s + 9) << 8 | rd8(s + 10) << 16 | rd8(s + 11) << 24;
    uint32_t sc, m;
    scale_min_k4(2 * g + hi, w0, w1, w2, sc, m);
    float d1 = d * (float)sc, m1 = dmin * (float)m;
    uint32_t q = rd8(blk + 16 + 32 * g + l);
    q = hi ? (q >> 4) : (q & 15u);
    return d1 * (float)q - m1;
}

// Q5_K: d@0 dmin@2 scales[12]@4 qh[32]@16 qs[128]@48.
IFR_DEV float deq_q5k(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    uint32_t g = e >> 6, hi = (e >> 5) & 1u, l = e & 31u;
    float d = f16_to_f32(ld_u16(blk)), dmin = f16_to_f32(ld_u16(blk + 2));
    const uint8_t *s = blk + 4;
    uint32_t w0 = rd8(s) | rd8(s + 1) << 8 | rd8(s + 2) << 16 | rd8(s + 3) << 24;
    uint32_t w1 = rd8(s + 4) | rd8(s + 5) << 8 | rd8(s + 6) << 16 | rd8(s + 7) << 24;
    uint32_t w2 = rd8(s + 8) | rd8(s + 9) << 8 | rd8(s + 10) << 16 | rd8(s + 11) << 24;
    uint32_t sc, m;
    scale_min_k4(2 * g + hi, w0, w1, w2, sc, m);
    float d1 = d * (float)sc, m1 = dmin * (float)m;
    uint32_t q = rd8(blk + 48 + 32 * g + l);
    q = hi ? (q >> 4) : (q & 15u);
    uint32_t h = (rd8(blk + 16 + l) >> (2 * g + hi)) & 1u;
    q += h ? 16u : 0u;
    return d1 * (float)q - m1;
}

// Q6_K: ql[128]@0 qh[64]@128 scales:i8[16]@192 d@208.
// Element e = 128i + 32k + l (k = 0..3, l = 0..31) reads ql[64i + l + 32(k&1)]
// (low nibble for k < 2, high for k >= 2), qh[32i + l] bits 2k..2k+1 and
// scale[8i + l/16 + 2k]; y = (d * scale) * (q - 32).
IFR_DEV float deq_q6k(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    uint32_t i = e >> 7, k = (e >> 5) & 3u, l = e & 31u;
    uint32_t qlb = rd8(blk + 64 * i + l + 32 * (k & 1u));
    uint32_t nib = (k < 2) ? (qlb & 15u) : (qlb >> 4);
    uint32_t h = (rd8(blk + 128 + 32 * i + l) >> (2 * k)) & 3u;
    int q = (int)(nib | (h << 4)) - 32;
    int sc = (int)(int8_t)rd8(blk + 192 + 8 * i + (l >> 4) + 2 * k);
    float d = f16_to_f32(ld_u16(blk + 208));
    return d * (float)sc * (float)q;
}

// Q8_0: d@0 qs:i8[32]@2.
IFR_DEV float deq_q8_0(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    float d = f16_to_f32(ld_u16(blk));
    return (float)(int8_t)rd8(blk + 2 + e) * d;
}

IFR_DEV int fmt_qk(int fmt) { return fmt == Q8_0 ? 32 : (fmt == F32 || fmt == F16) ? 1 : 256; }
IFR_DEV int fmt_bytes(int fmt) {
    switch (fmt) {
    case F32: return 4;
    case F16: return 2;
    case Q8_0: return 34;
    case Q4_K: return 144;
    case Q5_K: return 176;
    default: return 210;
    }
}

// Element `idx` of a tensor stored as consecutive blocks of format `fmt`.
IFR_DEV float deq_elem(int fmt, const uint8_t *base, uint64_t idx) {
    int qk = fmt_qk(fmt), bb = fmt_bytes(fmt);
    uint64_t b = idx / (uint64_t)qk;
    uint32_t e = (uint32_t)(idx % (uint64_t)qk);
    const uint8_t *blk = base + b * (uint64_t)bb;
    switch (fmt) {
    case F32: return *(const float *)blk;
    case F16: return f16_to_f32(ld_u16(blk));
    case Q8_0: return deq_q8_0(blk, e);
    case Q4_K: return deq_q4k(blk, e);
    case Q5_K: return deq_q5k(blk, e);
    default: return deq_q6k(blk, e);
    }
}

// --------------------------------------------------------------- quantizer --
// Deterministic min/max quantizer (the reference has none).  Every step is one
// correctly rounded IEEE operation or exact, so the CPU restatement used by the
// tests produces the same bytes:
//   Q8_0: d = amax/127, q = clamp(rint(x * (1/d)), -127, 127)
//   Q4_K/Q5_K (levels L = 15/31): per 32-element sub-block lo = min(0, min x),
//         s = (max x - lo)/L, n = -lo; d = f16(max s / 63), dmin = f16(max n / 63);
//         sc = clamp(rint(s/d)), m = clamp(rint(n/dmin)) in [0, 63];
//         q = clamp(rint((x + dmin*m) / (d*sc)), 0, L)
//   Q6_K: per 16-element sub-block s = amax/31; d = f16(max s/127);
//         sc = clamp(rint(s/d), 0, 127); q = clamp(rint(x/(d*sc)), -32, 31) + 32
// Comparisons are explicit (no fmin/fmax) so signed zeros resolve identically.

IFR_DEV float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
IFR_DEV int qround(float v, float lo, float hi) { return (int)rintf(clampf(v, lo, hi)); }
IFR_DEV void wr16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

IFR_DEV void quant_q8_0(const float *x, uint8_t *blk) {
#pragma clang fp contract(off)
    float amax = 0.0f;
    for (int l = 0; l < 32; l++) {
        float a = fabsf(x[l]);
        amax = a > amax ? a : amax;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(blk, f32_to_f16(d));
    for (int l = 0; l < 32; l++) blk[2 + l] = (uint8_t)(int8_t)qround(x[l] * id, -127.0f, 127.0f);
}

IFR_DEV void pack_scales_k4(const uint8_t *sc, const uint8_t *mn, uint8_t *q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

IFR_DEV void quant_k_minmax(const float *x, int levels, uint8_t *hdr, uint8_t *q) {
#pragma clang fp contract(off)
    float s[8], n[8], smax = 0.0f, nmax = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = -INFINITY;
        for (int l = 0; l < 32; l++) {
            float v = x[32 * j + l];
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
        }
        if (hi < lo) hi = lo;
        s[j] = (hi - lo) / (float)levels;
        n[j] = -lo;
        smax = s[j] > smax ? s[j] : smax;
        nmax = n[j] > nmax ? n[j] : nmax;
    }
    uint16_t dh = f32_to_f16(smax / 63.0f), mh = f32_to_f16(nmax / 63.0f);
    float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(d > 0.0f ? qround(s[j] / d, 0.0f, 63.0f) : 0);
        mn[j] = (uint8_t)(dmin > 0.0f ? qround(n[j] / dmin, 0.0f, 63.0f) : 0);
    }
    wr16(hdr, dh);
    wr16(hdr + 2, mh);
    pack_scales_k4(sc, mn, hdr + 4);
    for (int j = 0; j < 8; j++) {
        float es = d * (float)sc[j], em = dmin * (float)mn[j];
        for (int l = 0; l < 32; l++) {
            int v = 0;
            if (es > 0.0f) v = qround((x[32 * j + l] + em) / es, 0.0f, (float)levels);
            q[32 * j + l] = (uint8_t)v;
        }
    }
}

IFR_DEV void quant_q4_k(const float *x, uint8_t *blk) {
    uint8_t q[256];
    quant_k_minmax(x, 15, blk, q);
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) blk[16 + 32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

IFR_DEV void quant_q5_k(const float *x, uint8_t *blk) {
    uint8_t q[256];
    quant_k_minmax(x, 31, blk, q);
    uint8_t *qh = blk + 16, *qs = blk + 48;
    for (int l = 0; l < 32; l++) qh[l] = 0;
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) {
            uint8_t a = q[64 * g + l], b = q[64 * g + 32 + l];
            qs[32 * g + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
            qh[l] |= (uint8_t)(((a >> 4) & 1) << (2 * g));
            qh[l] |= (uint8_t)(((b >> 4) & 1) << (2 * g + 1));
        }
}

IFR_DEV void quant_q6_k(const float *x, uint8_t *blk) {
#pragma clang fp contract(off)
    float s[16], smax = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f;
        for (int l = 0; l < 16; l++) {
            float a = fabsf(x[16 * j + l]);
            amax = a > amax ? a : amax;
        }
        s[j] = amax / 31.0f;
        smax = s[j] > smax ? s[j] : smax;
    }
    uint16_t dh = f32_to_f16(smax / 127.0f);
    float d = f16_to_f32(dh);
    uint8_t u[256];
    int8_t sc[16];
    for (int j = 0; j < 16; j++) {
        sc[j] = (int8_t)(d > 0.0f ? qround(s[j] / d, 0.0f, 127.0f) : 0);
        float es = d * (float)sc[j];
        for (int l = 0; l < 16; l++) {
            int v = 0;
            if (es > 0.0f) v = qround(x[16 * j + l] / es, -32.0f, 31.0f);
            u[16 * j + l] = (uint8_t)(v + 32);
        }
    }
    uint8_t *ql = blk, *qh = blk + 128;
    for (int l = 0; l < 64; l++) qh[l] = 0;
    for (int i = 0; i < 2; i++)
        for (int l = 0; l < 32; l++) {
            uint8_t a = u[128 * i + l], b = u[128 * i + l + 32];
            uint8_t c = u[128 * i + l + 64], e = u[128 * i + l + 96];
            ql[64 * i + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
            ql[64 * i + l + 32] = (uint8_t)((b & 15) | ((e & 15) << 4));
            qh[32 * i + l] = (uint8_t)((a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6));
        }
    for (int j = 0; j < 16; j++) blk[192 + j] = (uint8_t)sc[j];
    wr16(blk + 208, dh);
}

} // namespace ifr

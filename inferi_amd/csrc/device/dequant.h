// Bit-exact dequantization of one element of a GGUF block, and the
// deterministic block quantizer.
//
// Dequantization follows crates/inferi/src/quantization.rs (Q8_0 :47-55,
// Q4_0 :66-82, Q4_1 :94-112, Q5_0 :123-143, Q5_1 :155-177, Q8_K :204-212,
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

// Q4_0: d@0 qs[16]@2; byte j holds element j (low nibble) and j+16 (high);
// y = (q - 8) * d.
IFR_DEV float deq_q4_0(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t b = rd8(blk + 2 + (e & 15u));
    const int q = (int)((e < 16) ? (b & 15u) : (b >> 4)) - 8;
    return (float)q * f16_to_f32(ld_u16(blk));
}

// Q4_1: d@0 m@2 qs[16]@4; y = q * d + m (two roundings).
IFR_DEV float deq_q4_1(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t b = rd8(blk + 4 + (e & 15u));
    const uint32_t q = (e < 16) ? (b & 15u) : (b >> 4);
    return (float)q * f16_to_f32(ld_u16(blk)) + f16_to_f32(ld_u16(blk + 2));
}

// Fifth bit of element e of a Q5_0/Q5_1 block: bit e of the little-endian
// word qh (element j and j+16 of byte j read bits j and j+16).
IFR_DEV uint32_t q5_high(const uint8_t *qh, uint32_t e) { return (rd8(qh + (e >> 3)) >> (e & 7u)) & 1u; }

// Q5_0: d@0 qh[4]@2 qs[16]@6; y = (q - 16) * d.
IFR_DEV float deq_q5_0(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t b = rd8(blk + 6 + (e & 15u));
    const uint32_t lo = (e < 16) ? (b & 15u) : (b >> 4);
    const int q = (int)(lo | (q5_high(blk + 2, e) << 4)) - 16;
    return (float)q * f16_to_f32(ld_u16(blk));
}

// Q5_1: d@0 m@2 qh[4]@4 qs[16]@8; y = q * d + m.
IFR_DEV float deq_q5_1(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    const uint32_t b = rd8(blk + 8 + (e & 15u));
    const uint32_t lo = (e < 16) ? (b & 15u) : (b >> 4);
    const uint32_t q = lo | (q5_high(blk + 4, e) << 4);
    return (float)q * f16_to_f32(ld_u16(blk)) + f16_to_f32(ld_u16(blk + 2));
}

// Q8_K: d:f32@0 qs:i8[256]@4 bsums:i16[16]@260; y = d * q.
IFR_DEV float deq_q8_k(const uint8_t *blk, uint32_t e) {
#pragma clang fp contract(off)
    return *(const float *)blk * (float)(int8_t)rd8(blk + 4 + e);
}

IFR_DEV int fmt_qk(int fmt) {
    switch (fmt) {
    case F32: case F16: return 1;
    case Q4_0: case Q4_1: case Q5_0: case Q5_1: case Q8_0: return 32;
    default: return 256;
    }
}
IFR_DEV int fmt_bytes(int fmt) {
    switch (fmt) {
    case F32: return 4;
    case F16: return 2;
    case Q4_0: return 18;
    case Q4_1: return 20;
    case Q5_0: return 22;
    case Q5_1: return 24;
    case Q8_0: return 34;
    case Q4_K: return 144;
    case Q5_K: return 176;
    case Q8_K: return 292;
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
    case Q4_0: return deq_q4_0(blk, e);
    case Q4_1: return deq_q4_1(blk, e);
    case Q5_0: return deq_q5_0(blk, e);
    case Q5_1: return deq_q5_1(blk, e);
    case Q8_0: return deq_q8_0(blk, e);
    case Q4_K: return deq_q4k(blk, e);
    case Q5_K: return deq_q5k(blk, e);
    case Q8_K: return deq_q8_k(blk, e);
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
//   Q4_0/Q5_0 (H = 8/16): v = the element of largest magnitude (first one),
//         d = f16(v / -H) (+0 when v = 0); q = clamp(rint(x * (1/d)), -H, H-1) + H
//   Q4_1/Q5_1 (L = 15/31): lo = min x, hi = max x; d = f16((hi-lo)/L),
//         m = f16(lo); q = clamp(rint((x - m) / d), 0, L)
//   Q8_K: d = amax/127 (f32); q = clamp(rint(x * (1/d)), -127, 127),
//         bsums = the sums of q over each 16 elements
// (d and m above are the decoded f16 values wherever codes are formed.)
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

// Q4_0 / Q5_0: symmetric codes around H with the block's extreme at -H.
IFR_DEV void quant_sym32(const float *x, int H, uint16_t *dh_out, int *q) {
#pragma clang fp contract(off)
    float amax = 0.0f, v = 0.0f;
    for (int l = 0; l < 32; l++) {
        const float a = fabsf(x[l]);
        if (a > amax) {
            amax = a;
            v = x[l];
        }
    }
    // an all-zero block gets d = +0 (stated, not left to how 0/-H is folded)
    const uint16_t dh = f32_to_f16(v == 0.0f ? 0.0f : v / -(float)H);
    const float d = f16_to_f32(dh);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int l = 0; l < 32; l++) q[l] = qround(x[l] * id, -(float)H, (float)(H - 1)) + H;
    *dh_out = dh;
}

// Q4_1 / Q5_1: affine codes from the block's min.
IFR_DEV void quant_aff32(const float *x, int L, uint16_t *dh_out, uint16_t *mh_out, int *q) {
#pragma clang fp contract(off)
    float lo = x[0], hi = x[0];
    for (int l = 1; l < 32; l++) {
        lo = x[l] < lo ? x[l] : lo;
        hi = x[l] > hi ? x[l] : hi;
    }
    const uint16_t dh = f32_to_f16((hi - lo) / (float)L), mh = f32_to_f16(lo);
    const float d = f16_to_f32(dh), m = f16_to_f32(mh);
    for (int l = 0; l < 32; l++) q[l] = d > 0.0f ? qround((x[l] - m) / d, 0.0f, (float)L) : 0;
    *dh_out = dh;
    *mh_out = mh;
}

IFR_DEV void pack_nibbles16(const int *q, uint8_t *qs) {
    for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}
IFR_DEV void pack_high32(const int *q, uint8_t *qh) {
    uint32_t h = 0;
    for (int j = 0; j < 32; j++) h |= (uint32_t)((q[j] >> 4) & 1) << j;
    for (int b = 0; b < 4; b++) qh[b] = (uint8_t)(h >> (8 * b));
}

IFR_DEV void quant_q4_0(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh;
    quant_sym32(x, 8, &dh, q);
    wr16(blk, dh);
    pack_nibbles16(q, blk + 2);
}
IFR_DEV void quant_q5_0(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh;
    quant_sym32(x, 16, &dh, q);
    wr16(blk, dh);
    pack_high32(q, blk + 2);
    pack_nibbles16(q, blk + 6);
}
IFR_DEV void quant_q4_1(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh, mh;
    quant_aff32(x, 15, &dh, &mh, q);
    wr16(blk, dh);
    wr16(blk + 2, mh);
    pack_nibbles16(q, blk + 4);
}
IFR_DEV void quant_q5_1(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh, mh;
    quant_aff32(x, 31, &dh, &mh, q);
    wr16(blk, dh);
    wr16(blk + 2, mh);
    pack_high32(q, blk + 4);
    pack_nibbles16(q, blk + 8);
}
IFR_DEV void quant_q8_k(const float *x, uint8_t *blk) {
#pragma clang fp contract(off)
    float amax = 0.0f;
    for (int l = 0; l < 256; l++) {
        const float a = fabsf(x[l]);
        amax = a > amax ? a : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint32_t db = __float_as_uint(d);
    for (int b = 0; b < 4; b++) blk[b] = (uint8_t)(db >> (8 * b));
    for (int j = 0; j < 16; j++) {
        int sum = 0;
        for (int l = 0; l < 16; l++) {
            const int v = qround(x[16 * j + l] * id, -127.0f, 127.0f);
            blk[4 + 16 * j + l] = (uint8_t)(int8_t)v;
            sum += v;
        }
        wr16(blk + 260 + 2 * j, (uint16_t)(int16_t)sum);
    }
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

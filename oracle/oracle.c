/*
 * CPU oracle for the inferi batch-1 GGUF decode token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with -ffp-contract=off so
 * that every f32 multiply and subtract rounds separately, exactly as the
 * reference's Rust dequantizers evaluate them (Rust never contracts to FMA).
 *
 * Citations are relative to the reference root (dimforge/inferi).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define QK_K 256

int ifo_block_elems(int dtype) {
    switch (dtype) {
    case IFO_F32: case IFO_F16: return 1;
    case IFO_Q4_0: case IFO_Q4_1: case IFO_Q5_0: case IFO_Q5_1: case IFO_Q8_0: return 32;
    case IFO_Q4_K: case IFO_Q5_K: case IFO_Q6_K: case IFO_Q8_K: return QK_K;
    default: return 0;
    }
}

int ifo_block_bytes(int dtype) {
    switch (dtype) {
    case IFO_F32: return 4;
    case IFO_F16: return 2;
    case IFO_Q4_0: return 18;   /* quantization.rs:60-63 */
    case IFO_Q4_1: return 20;   /* quantization.rs:87-91 */
    case IFO_Q5_0: return 22;   /* quantization.rs:116-120 */
    case IFO_Q5_1: return 24;   /* quantization.rs:147-152 */
    case IFO_Q8_0: return 34;   /* quantization.rs:42-45 */
    case IFO_Q8_K: return 292;  /* quantization.rs:183-187 */
    case IFO_Q4_K: return 144;  /* quantization.rs:335-340 */
    case IFO_Q5_K: return 176;  /* quantization.rs:262-268 */
    case IFO_Q6_K: return 210;  /* quantization.rs:217-222 */
    default: return 0;
    }
}

/* ------------------------------------------------------------------ f16 -- */

/* quantization.rs:405-422.  Exact: subnormals are mant * 2^-24, normals
 * (mant + 1024) * 2^(exp-25); exponent 31 gives inf or a canonical NaN. */
float ifo_decode_f16(uint16_t half) {
    uint16_t exp = (half >> 10) & 0x1f;
    uint16_t mant = half & 0x3ff;
    float val;
    if (exp == 0)
        val = (float)mant * ldexpf(1.0f, -24);
    else if (exp != 31)
        val = ((float)mant + 1024.0f) * ldexpf(1.0f, (int)exp - 25);
    else if (mant == 0)
        val = INFINITY;
    else
        val = NAN;
    return (half & 0x8000) ? -val : val;
}

/* binary32 -> binary16, round to nearest, ties to even, with subnormals,
 * overflow to infinity and NaN kept NaN. */
uint16_t ifo_encode_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) /* inf or NaN */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    if (absx >= 0x477ff000u) /* rounds to >= 65520: overflow */
        return (uint16_t)(sign | 0x7c00u);
    if (absx < 0x38800000u) { /* result is subnormal or zero: |f| < 2^-14 */
        if (absx < 0x33000000u) /* < 2^-25: rounds to zero */
            return (uint16_t)sign;
        uint32_t e = absx >> 23;            /* biased f32 exponent */
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;           /* 14 + (127 - e) - 1 ... value = m * 2^(e-150) */
        /* half subnormal unit is 2^-24: q = m * 2^(e-150+24) = m >> (126 - e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1)))
            q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112;        /* rebias 127 -> 15 */
    uint32_t m = absx & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1)))
        q++;                                /* may carry into the exponent: correct */
    return (uint16_t)(sign | q);
}

void ifo_decode_f16_array(const uint16_t *h, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = ifo_decode_f16(h[i]);
}

void ifo_encode_f16_array(const float *f, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = ifo_encode_f16(f[i]);
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------- dequant -- */

/* quantization.rs:394-402 */
void ifo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quantization.rs:47-55.  Layout: d:f16 @0, qs:i8[32] @2. */
void ifo_dequant_q8_0(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk));
    for (int l = 0; l < 32; l++) y[l] = (float)(int8_t)blk[2 + l] * d;
}

/* quantization.rs:358-392.  Layout: d @0, dmin @2, scales[12] @4, qs[128] @16. */
void ifo_dequant_q4_k(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk));
    float min = ifo_decode_f16(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t sc, m;
        ifo_get_scale_min_k4(is, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = min * (float)m;
        ifo_get_scale_min_k4(is + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++) y[j + l] = d1 * (float)(qs[l] & 0xf) - m1;
        for (int l = 0; l < 32; l++) y[j + l + 32] = d2 * (float)(qs[l] >> 4) - m2;
        qs += 32;
        is += 2;
    }
}

/* quantization.rs:287-330.  Layout: d @0, dmin @2, scales[12] @4, qh[32] @16,
 * qs[128] @48. */
void ifo_dequant_q5_k(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk));
    float min = ifo_decode_f16(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t sc, m;
        ifo_get_scale_min_k4(is, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = min * (float)m;
        ifo_get_scale_min_k4(is + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++)
            y[j + l] = d1 * (float)((qs[l] & 0xf) + ((qh[l] & u1) ? 16 : 0)) - m1;
        for (int l = 0; l < 32; l++)
            y[j + l + 32] = d2 * (float)((qs[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - m2;
        qs += 32;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* quantization.rs:224-257.  Layout: ql[128] @0, qh[64] @128, scales:i8[16] @192,
 * d @208.  Each output is (d * scale) * q, two roundings, left to right. */
void ifo_dequant_q6_k(const uint8_t *blk, float *y) {
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    float d = ifo_decode_f16(rd16(blk + 208));
    for (int i = 0; i < 2; i++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            uint8_t ql0 = ql[i * 64 + l], ql32 = ql[i * 64 + l + 32], h = qh[i * 32 + l];
            int q1 = (int8_t)((ql0 & 0xf) | (((h >> 0) & 3) << 4)) - 32;
            int q2 = (int8_t)((ql32 & 0xf) | (((h >> 2) & 3) << 4)) - 32;
            int q3 = (int8_t)((ql0 >> 4) | (((h >> 4) & 3) << 4)) - 32;
            int q4 = (int8_t)((ql32 >> 4) | (((h >> 6) & 3) << 4)) - 32;
            y[i * 128 + l + 0] = d * (float)sc[i * 8 + is + 0] * (float)q1;
            y[i * 128 + l + 32] = d * (float)sc[i * 8 + is + 2] * (float)q2;
            y[i * 128 + l + 64] = d * (float)sc[i * 8 + is + 4] * (float)q3;
            y[i * 128 + l + 96] = d * (float)sc[i * 8 + is + 6] * (float)q4;
        }
    }
}

/* quantization.rs:66-82.  Layout: d @0, qs[16] @2; byte j holds element j
 * (low nibble) and j+16 (high); y = (q - 8) * d. */
void ifo_dequant_q4_0(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk));
    for (int j = 0; j < 16; j++) {
        int x0 = (blk[2 + j] & 0x0F) - 8, x1 = (blk[2 + j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}

/* quantization.rs:94-112.  Layout: d @0, m @2, qs[16] @4; y = q * d + m. */
void ifo_dequant_q4_1(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk)), m = ifo_decode_f16(rd16(blk + 2));
    for (int j = 0; j < 16; j++) {
        y[j] = (float)(blk[4 + j] & 0x0F) * d + m;
        y[j + 16] = (float)(blk[4 + j] >> 4) * d + m;
    }
}

static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

/* quantization.rs:123-143.  Layout: d @0, qh[4] @2 (read as a little-endian
 * u32), qs[16] @6; y = (q - 16) * d. */
void ifo_dequant_q5_0(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk));
    uint32_t qh = rd32(blk + 2);
    for (uint32_t j = 0; j < 16; j++) {
        uint32_t xh_0 = ((qh >> j) << 4) & 0x10, xh_1 = (qh >> (j + 12)) & 0x10;
        int x0 = (int)(((uint32_t)blk[6 + j] & 0x0F) | xh_0) - 16;
        int x1 = (int)(((uint32_t)blk[6 + j] >> 4) | xh_1) - 16;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}

/* quantization.rs:155-177.  Layout: d @0, m @2, qh[4] @4, qs[16] @8;
 * y = q * d + m. */
void ifo_dequant_q5_1(const uint8_t *blk, float *y) {
    float d = ifo_decode_f16(rd16(blk)), m = ifo_decode_f16(rd16(blk + 2));
    uint32_t qh = rd32(blk + 4);
    for (uint32_t j = 0; j < 16; j++) {
        uint32_t xh_0 = ((qh >> j) << 4) & 0x10, xh_1 = (qh >> (j + 12)) & 0x10;
        uint32_t x0 = ((uint32_t)blk[8 + j] & 0x0F) | xh_0, x1 = ((uint32_t)blk[8 + j] >> 4) | xh_1;
        y[j] = (float)x0 * d + m;
        y[j + 16] = (float)x1 * d + m;
    }
}

/* quantization.rs:204-212.  Layout: d:f32 @0, qs:i8[256] @4, bsums:i16[16]
 * @260 (not read by dequantize); y = d * q. */
void ifo_dequant_q8_k(const uint8_t *blk, float *y) {
    float d;
    memcpy(&d, blk, 4);
    for (int j = 0; j < QK_K; j++) y[j] = d * (float)(int8_t)blk[4 + j];
}

int ifo_dequant(int dtype, const void *data, size_t n_elems, float *y) {
    const uint8_t *p = (const uint8_t *)data;
    int qk = ifo_block_elems(dtype), bb = ifo_block_bytes(dtype);
    if (qk == 0 || n_elems % (size_t)qk) return -1;
    size_t nb = n_elems / (size_t)qk;
    for (size_t b = 0; b < nb; b++, p += bb, y += qk) {
        switch (dtype) {
        case IFO_F32: memcpy(y, p, 4); break;
        case IFO_F16: y[0] = ifo_decode_f16(rd16(p)); break;
        case IFO_Q4_0: ifo_dequant_q4_0(p, y); break;
        case IFO_Q4_1: ifo_dequant_q4_1(p, y); break;
        case IFO_Q5_0: ifo_dequant_q5_0(p, y); break;
        case IFO_Q5_1: ifo_dequant_q5_1(p, y); break;
        case IFO_Q8_0: ifo_dequant_q8_0(p, y); break;
        case IFO_Q4_K: ifo_dequant_q4_k(p, y); break;
        case IFO_Q5_K: ifo_dequant_q5_k(p, y); break;
        case IFO_Q6_K: ifo_dequant_q6_k(p, y); break;
        case IFO_Q8_K: ifo_dequant_q8_k(p, y); break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------ quantize -- */
/*
 * The reference has no quantizer (quantization.rs only dequantizes), so this
 * is our own deterministic min/max quantizer, written so that a GPU port of it
 * produces the same bytes: every step is a single correctly rounded IEEE
 * operation (division, multiply, add) or exact (min, max, integer), rounding
 * to integers clamps to the code range in float and then rounds half to even
 * (rintf), comparisons are explicit (no fminf/fmaxf, so signed zeros resolve
 * the same everywhere), and there is no FMA contraction.
 *
 *   Q8_0: d = amax/127; q = clamp(rint(x * (1/d)), -127, 127).
 *   Q4_K: per 32-element sub-block j, lo_j = min(0, min x), hi_j = max x,
 *         s_j = (hi_j - lo_j)/15, n_j = -lo_j.  Super scales d = max s/63 and
 *         dmin = max n/63 are stored as f16 (RNE); the 6-bit codes are
 *         sc_j = clamp(rint(s_j/d'), 0, 63), m_j = clamp(rint(n_j/dmin'), 0, 63)
 *         with d', dmin' the decoded f16 values; the 4-bit codes are
 *         q = clamp(rint((x + dmin'*m_j) / (d'*sc_j)), 0, 15).
 *   Q5_K: as Q4_K with 31 levels and the 5th bit in qh.
 *   Q6_K: per 16-element sub-block, s_j = amax_j/31; d = max s/127 as f16;
 *         sc_j = clamp(rint(s_j/d'), 0, 127);
 *         q = clamp(rint(x/(d'*sc_j)), -32, 31) + 32.
 *   Q4_0/Q5_0 (H = 8/16): v = the first element of largest magnitude;
 *         d = v/-H as f16 (+0 when v = 0); q = clamp(rint(x * (1/d')), -H, H-1) + H.
 *   Q4_1/Q5_1 (L = 15/31): lo = min x, hi = max x; d = (hi-lo)/L and
 *         m = lo as f16; q = clamp(rint((x - m') / d'), 0, L) (0 when d' = 0).
 *   Q8_K: d = amax/127 kept in f32; q = clamp(rint(x * (1/d)), -127, 127);
 *         bsums_j = the sum of q over elements 16j..16j+15.
 */
static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* clamp in the float domain first, then round half to even: defined for every
 * finite input and identical to rounding first and clamping after. */
static inline int qround(float v, float lo, float hi) { return (int)rintf(clampf(v, lo, hi)); }

static void quant_q8_0(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int l = 0; l < 32; l++) {
        float a = fabsf(x[l]);
        amax = a > amax ? a : amax;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = ifo_encode_f16(d);
    wr16(blk, dh);
    for (int l = 0; l < 32; l++) blk[2 + l] = (uint8_t)(int8_t)qround(x[l] * id, -127.0f, 127.0f);
}

static void quant_sym32(const float *x, int H, uint16_t *dh_out, int *q) {
    float amax = 0.0f, v = 0.0f;
    for (int l = 0; l < 32; l++) {
        float a = fabsf(x[l]);
        if (a > amax) {
            amax = a;
            v = x[l];
        }
    }
    uint16_t dh = ifo_encode_f16(v == 0.0f ? 0.0f : v / -(float)H); /* +0 for an all-zero block */
    float d = ifo_decode_f16(dh);
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int l = 0; l < 32; l++) q[l] = qround(x[l] * id, -(float)H, (float)(H - 1)) + H;
    *dh_out = dh;
}

static void quant_aff32(const float *x, int L, uint16_t *dh_out, uint16_t *mh_out, int *q) {
    float lo = x[0], hi = x[0];
    for (int l = 1; l < 32; l++) {
        lo = x[l] < lo ? x[l] : lo;
        hi = x[l] > hi ? x[l] : hi;
    }
    uint16_t dh = ifo_encode_f16((hi - lo) / (float)L), mh = ifo_encode_f16(lo);
    float d = ifo_decode_f16(dh), m = ifo_decode_f16(mh);
    for (int l = 0; l < 32; l++) q[l] = d > 0.0f ? qround((x[l] - m) / d, 0.0f, (float)L) : 0;
    *dh_out = dh;
    *mh_out = mh;
}

static void pack_nibbles16(const int *q, uint8_t *qs) {
    for (int j = 0; j < 16; j++) qs[j] = (uint8_t)((q[j] & 15) | ((q[j + 16] & 15) << 4));
}

static void pack_high32(const int *q, uint8_t *qh) {
    uint32_t h = 0;
    for (int j = 0; j < 32; j++) h |= (uint32_t)((q[j] >> 4) & 1) << j;
    for (int b = 0; b < 4; b++) qh[b] = (uint8_t)(h >> (8 * b));
}

static void quant_q4_0(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh;
    quant_sym32(x, 8, &dh, q);
    wr16(blk, dh);
    pack_nibbles16(q, blk + 2);
}

static void quant_q5_0(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh;
    quant_sym32(x, 16, &dh, q);
    wr16(blk, dh);
    pack_high32(q, blk + 2);
    pack_nibbles16(q, blk + 6);
}

static void quant_q4_1(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh, mh;
    quant_aff32(x, 15, &dh, &mh, q);
    wr16(blk, dh);
    wr16(blk + 2, mh);
    pack_nibbles16(q, blk + 4);
}

static void quant_q5_1(const float *x, uint8_t *blk) {
    int q[32];
    uint16_t dh, mh;
    quant_aff32(x, 31, &dh, &mh, q);
    wr16(blk, dh);
    wr16(blk + 2, mh);
    pack_high32(q, blk + 4);
    pack_nibbles16(q, blk + 8);
}

static void quant_q8_k(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int l = 0; l < QK_K; l++) {
        float a = fabsf(x[l]);
        amax = a > amax ? a : amax;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    memcpy(blk, &d, 4);
    for (int j = 0; j < 16; j++) {
        int sum = 0;
        for (int l = 0; l < 16; l++) {
            int v = qround(x[16 * j + l] * id, -127.0f, 127.0f);
            blk[4 + 16 * j + l] = (uint8_t)(int8_t)v;
            sum += v;
        }
        wr16(blk + 260 + 2 * j, (uint16_t)(int16_t)sum);
    }
}

/* Pack 8 six-bit scales and mins into the 12-byte K-quant layout read by
 * get_scale_min_k4 (quantization.rs:394-402). */
static void pack_scales_k4(const uint8_t *sc, const uint8_t *mn, uint8_t *q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

/* Shared by Q4_K (levels 15) and Q5_K (levels 31): fills d/dmin/scales and the
 * integer codes q[256]. */
static void quant_k_minmax(const float *x, int levels, uint8_t *hdr, uint8_t *q) {
    float s[8], n[8];
    float smax = 0.0f, nmax = 0.0f;
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
    uint16_t dh = ifo_encode_f16(smax / 63.0f), mh = ifo_encode_f16(nmax / 63.0f);
    float d = ifo_decode_f16(dh), dmin = ifo_decode_f16(mh);
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

static void quant_q4_k(const float *x, uint8_t *blk) {
    uint8_t q[QK_K];
    quant_k_minmax(x, 15, blk, q);
    uint8_t *qs = blk + 16;
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++)
            qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

static void quant_q5_k(const float *x, uint8_t *blk) {
    uint8_t q[QK_K];
    quant_k_minmax(x, 31, blk, q);
    uint8_t *qh = blk + 16, *qs = blk + 48;
    memset(qh, 0, 32);
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) {
            uint8_t a = q[64 * g + l], b = q[64 * g + 32 + l];
            qs[32 * g + l] = (uint8_t)((a & 15) | ((b & 15) << 4));
            qh[l] |= (uint8_t)(((a >> 4) & 1) << (2 * g));
            qh[l] |= (uint8_t)(((b >> 4) & 1) << (2 * g + 1));
        }
}

static void quant_q6_k(const float *x, uint8_t *blk) {
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
    uint16_t dh = ifo_encode_f16(smax / 127.0f);
    float d = ifo_decode_f16(dh);
    int8_t sc[16];
    uint8_t u[QK_K];
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
    memset(qh, 0, 64);
    for (int i = 0; i < 2; i++)
        for (int l = 0; l < 32; l++) {
            uint8_t a = u[128 * i + l], b = u[128 * i + l + 32];
            uint8_t c = u[128 * i + l + 64], e = u[128 * i + l + 96];
            ql[64 * i + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
            ql[64 * i + l + 32] = (uint8_t)((b & 15) | ((e & 15) << 4));
            qh[32 * i + l] = (uint8_t)((a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6));
        }
    memcpy(blk + 192, sc, 16);
    wr16(blk + 208, dh);
}

int ifo_quantize(int dtype, const float *x, size_t n_elems, void *out) {
    uint8_t *p = (uint8_t *)out;
    int qk = ifo_block_elems(dtype), bb = ifo_block_bytes(dtype);
    if (qk == 0 || n_elems % (size_t)qk) return -1;
    for (size_t b = 0; b < n_elems / (size_t)qk; b++, x += qk, p += bb) {
        switch (dtype) {
        case IFO_F32: memcpy(p, x, 4); break;
        case IFO_F16: wr16(p, ifo_encode_f16(x[0])); break;
        case IFO_Q4_0: quant_q4_0(x, p); break;
        case IFO_Q4_1: quant_q4_1(x, p); break;
        case IFO_Q5_0: quant_q5_0(x, p); break;
        case IFO_Q5_1: quant_q5_1(x, p); break;
        case IFO_Q8_0: quant_q8_0(x, p); break;
        case IFO_Q4_K: quant_q4_k(x, p); break;
        case IFO_Q5_K: quant_q5_k(x, p); break;
        case IFO_Q6_K: quant_q6_k(x, p); break;
        case IFO_Q8_K: quant_q8_k(x, p); break;
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- GEMV -- */

/* gemv_quant.rs:444-456: f64 accumulation of f32 products, rounded once. */
void ifo_gemv_f64(const float *w, int rows, int cols, const float *x, float *y) {
    for (int r = 0; r < rows; r++) {
        double sum = 0.0;
        const float *wr = w + (size_t)r * cols;
        for (int c = 0; c < cols; c++) sum += (double)wr[c] * (double)x[c];
        y[r] = (float)sum;
    }
}

typedef struct {
    int dtype, rows, cols, r0, r1;
    const uint8_t *w;
    const float *x;
    float *y;
} gemv_job;

/* Accumulation of the quantized GEMVs: 0 (default) in f64, rounded once;
 * 1 in f32, left to right, each product and sum rounded (nalgebra's gemv,
 * cpu.rs:375-381), to measure what plain f32 arithmetic costs a model. */
static int g_f32_accum = 0;
void ifo_set_f32_accum(int on) { g_f32_accum = on; }

static void *gemv_worker(void *arg) {
    gemv_job *j = (gemv_job *)arg;
    int qk = ifo_block_elems(j->dtype), bb = ifo_block_bytes(j->dtype);
    int nb = j->cols / qk;
    float buf[QK_K];
    for (int r = j->r0; r < j->r1; r++) {
        const uint8_t *row = j->w + (size_t)r * nb * bb;
        double sum = 0.0;
        float sum32 = 0.0f;
        for (int b = 0; b < nb; b++) {
            ifo_dequant(j->dtype, row + (size_t)b * bb, (size_t)qk, buf);
            const float *xb = j->x + (size_t)b * qk;
            if (g_f32_accum)
                for (int l = 0; l < qk; l++) sum32 += buf[l] * xb[l];
            else
                for (int l = 0; l < qk; l++) sum += (double)buf[l] * (double)xb[l];
        }
        j->y[r] = g_f32_accum ? sum32 : (float)sum;
    }
    return NULL;
}

static int default_threads(void) {
    const char *e = getenv("IFO_THREADS");
    if (e && atoi(e) > 0) return atoi(e);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)(n > 64 ? 64 : n) : 1;
}

int ifo_gemv_quant(int dtype, const void *w, int rows, int cols, const float *x,
                   float *y, int nthreads) {
    int qk = ifo_block_elems(dtype);
    if (qk == 0 || cols % qk || rows <= 0) return -1;
    if (nthreads <= 0) nthreads = default_threads();
    if (nthreads > rows) nthreads = rows;
    if ((size_t)rows * (size_t)cols < (1u << 16)) nthreads = 1;
    gemv_job jobs[64];
    pthread_t th[64];
    if (nthreads > 64) nthreads = 64;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (gemv_job){dtype, rows, cols, (int)((long)rows * t / nthreads),
                             (int)((long)rows * (t + 1) / nthreads), (const uint8_t *)w, x, y};
    }
    if (nthreads == 1) {
        gemv_worker(&jobs[0]);
        return 0;
    }
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, gemv_worker, &jobs[t]);
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    return 0;
}

/* ------------------------------------------------------- elementwise ops -- */

/* inferi-shaders/src/rms_norm.rs:112-120:
 * rms = 1/sqrt(sum(x^2)/n + eps); out = (x * rms) * w. */
void ifo_rms_norm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    double rms = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (int i = 0; i < n; i++) out[i] = (float)(((double)x[i] * rms) * (double)w[i]);
}

/* inferi-shaders/src/rope.rs:51-92 (Original) and :97-141 (NeoX).  theta and
 * the angle are f32 values, as the shader computes them: the exponent
 * -((2i) mod hs)/hs is an f32 division, theta = base^exponent rounded to f32
 * (evaluated in f64, so it is the correctly rounded f32 power, where the
 * shader's powf may be off by an ulp), angle = (f32)pos * theta; the rotation
 * itself is evaluated in f64 and rounded once. */
void ifo_rope(int neox, float *q, int q_len, float *k, int k_len, int head_size,
              int pos, float base_freq) {
    for (int i = 0; i < q_len / 2; i++) {
        float head_dim = (float)((i * 2) % head_size);
        float theta = (float)pow((double)base_freq, (double)(-head_dim / (float)head_size));
        float m_theta = (float)pos * theta;
        double c = cos((double)m_theta), s = sin((double)m_theta);
        int iq, shift;
        if (neox) {
            int head_id = (i * 2) / head_size;
            iq = i + head_id * head_size / 2;
            shift = head_size / 2;
        } else {
            iq = 2 * i;
            shift = 1;
        }
        double a = q[iq], b = q[iq + shift];
        q[iq] = (float)(c * a - s * b);
        q[iq + shift] = (float)(s * a + c * b);
        if (i * 2 < k_len) {
            double ka = k[iq], kb = k[iq + shift];
            k[iq] = (float)(c * ka - s * kb);
            k[iq + shift] = (float)(s * ka + c * kb);
        }
    }
}

/* inferi-shaders/src/silu.rs:24-53: h1 <- h2 * (h1 / (1 + exp(-h1))). */
void ifo_silu_mul(float *h1, const float *h2, int n) {
    for (int i = 0; i < n; i++) {
        double h = h1[i];
        h1[i] = (float)((double)h2[i] * (h / (1.0 + exp(-h))));
    }
}

void ifo_add(float *x, const float *b, int n) {
    for (int i = 0; i < n; i++) x[i] = x[i] + b[i];
}

/* ----------------------------------------------------------- attention -- */

static inline float kv_at(const void *cache, int kv_f16, size_t idx) {
    return kv_f16 ? ifo_decode_f16(((const uint16_t *)cache)[idx]) : ((const float *)cache)[idx];
}

/* ops/batched_multiquery_attention.rs:191-245 with the fused kernel's
 * semantics (fused_attention.rs:66-241): for query head h and kv head
 * h / kv_mul, s_t = (q_h . k_t) / sqrt(head_size) for t in [0, pos];
 * p = softmax(s); out_h = sum_t p_t v_t. */
void ifo_attention(const ifo_attn_params *p, const float *q, const void *k_cache,
                   const void *v_cache, int kv_f16, float *out) {
    int hs = (int)p->head_size, T = (int)p->pos + 1;
    double *s = (double *)malloc(sizeof(double) * (size_t)T);
    double *acc = (double *)malloc(sizeof(double) * (size_t)hs);
    double scale = sqrt((double)hs);
    for (int h = 0; h < (int)p->n_heads; h++) {
        int kvh = h / (int)p->kv_mul;
        const float *qh = q + (size_t)h * hs;
        double mx = -INFINITY;
        for (int t = 0; t < T; t++) {
            size_t base = (size_t)t * p->kv_dim + (size_t)kvh * hs;
            double dot = 0.0;
            for (int d = 0; d < hs; d++) dot += (double)qh[d] * (double)kv_at(k_cache, kv_f16, base + d);
            s[t] = dot / scale;
            if (s[t] > mx) mx = s[t];
        }
        double sum = 0.0;
        for (int t = 0; t < T; t++) {
            s[t] = exp(s[t] - mx);
            sum += s[t];
        }
        for (int d = 0; d < hs; d++) acc[d] = 0.0;
        for (int t = 0; t < T; t++) {
            size_t base = (size_t)t * p->kv_dim + (size_t)kvh * hs;
            double pt = s[t] / sum;
            for (int d = 0; d < hs; d++) acc[d] += pt * (double)kv_at(v_cache, kv_f16, base + d);
        }
        for (int d = 0; d < hs; d++) out[(size_t)h * hs + d] = (float)acc[d];
    }
    free(s);
    free(acc);
}

/* models/sampler.rs:54-56 (nalgebra imax): first index of the maximum. */
int ifo_argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ops/softmax.rs:130-143: max, then exp(x - max) accumulated left to right
 * into an f32 sum, then every element divided by the sum. */
void ifo_softmax(float *v, int n) {
    float mx = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    for (int i = 0; i < n; i++) v[i] /= sum;
}

/* models/sampler.rs:60-76: f32 running CDF, first index with coin < cdf. */
int ifo_sample_mult(const float *p, int n, float coin) {
    float cdf = 0.0f;
    for (int i = 0; i < n; i++) {
        cdf += p[i];
        if (coin < cdf) return i;
    }
    return n - 1;
}

typedef struct {
    float prob;
    int index;
} ifo_prob_index;

/* The reference sorts with a stable sort keyed on -prob (sampler.rs:101);
 * the candidates are gathered in index order, so "probability descending,
 * then index ascending" is the same order. */
static int cmp_prob_desc(const void *a, const void *b) {
    const ifo_prob_index *x = (const ifo_prob_index *)a, *y = (const ifo_prob_index *)b;
    if (x->prob > y->prob) return -1;
    if (x->prob < y->prob) return 1;
    return (x->index > y->index) - (x->index < y->index);
}

/* models/sampler.rs:83-131. */
int ifo_sample_topp(const float *p, int n, float topp, float coin, int *last, float *cum) {
    const float cutoff = (1.0f - topp) / ((float)n - 1.0f);
    ifo_prob_index *pi = (ifo_prob_index *)malloc((size_t)n * sizeof *pi);
    int n0 = 0;
    for (int i = 0; i < n; i++)
        if (p[i] >= cutoff) {
            pi[n0].index = i;
            pi[n0].prob = p[i];
            n0++;
        }
    if (n0 == 0) {
        free(pi);
        return -1;
    }
    qsort(pi, (size_t)n0, sizeof *pi, cmp_prob_desc);
    float cumulative = 0.0f;
    int last_idx = n0 - 1;
    for (int i = 0; i < n0; i++) {
        cumulative += pi[i].prob;
        if (cumulative > topp) {
            last_idx = i;
            break;
        }
    }
    if (last) *last = last_idx;
    if (cum) *cum = cumulative;
    const float r = coin * cumulative;
    float cdf = 0.0f;
    int out = pi[last_idx].index;
    for (int i = 0; i <= last_idx; i++) {
        cdf += pi[i].prob;
        if (r < cdf) {
            out = pi[i].index;
            break;
        }
    }
    free(pi);
    return out;
}

/* models/sampler.rs:32-52. */
int ifo_sample(float *logits, int n, float temperature, float topp, float coin) {
    if (temperature == 0.0f) return ifo_argmax(logits, n);
    for (int i = 0; i < n; i++) logits[i] /= temperature;
    ifo_softmax(logits, n);
    if (topp <= 0.0f || topp >= 1.0f) return ifo_sample_mult(logits, n, coin);
    return ifo_sample_topp(logits, n, topp, coin, NULL, NULL);
}

/* --------------------------------------------------------------- model -- */

struct ifo_state {
    ifo_config cfg;
    float *x, *xb, *xb2, *q, *hb, *hb2, *att_out;
    void **k_cache, **v_cache;
};

ifo_state *ifo_state_new(const ifo_config *cfg) {
    ifo_state *s = (ifo_state *)calloc(1, sizeof(ifo_state));
    int kv_dim = cfg->hidden * cfg->n_kv_heads / cfg->n_heads;
    size_t esz = cfg->kv_f16 ? 2 : 4;
    s->cfg = *cfg;
    s->x = (float *)calloc((size_t)cfg->hidden, 4);
    s->xb = (float *)calloc((size_t)cfg->hidden, 4);
    s->xb2 = (float *)calloc((size_t)cfg->hidden, 4);
    s->q = (float *)calloc((size_t)cfg->hidden, 4);
    s->att_out = (float *)calloc((size_t)cfg->hidden, 4);
    s->hb = (float *)calloc((size_t)cfg->ffn, 4);
    s->hb2 = (float *)calloc((size_t)cfg->ffn, 4);
    s->k_cache = (void **)calloc((size_t)cfg->n_layers, sizeof(void *));
    s->v_cache = (void **)calloc((size_t)cfg->n_layers, sizeof(void *));
    for (int l = 0; l < cfg->n_layers; l++) {
        s->k_cache[l] = calloc((size_t)cfg->max_pos * kv_dim, esz);
        s->v_cache[l] = calloc((size_t)cfg->max_pos * kv_dim, esz);
    }
    return s;
}

void ifo_state_free(ifo_state *s) {
    if (!s) return;
    for (int l = 0; l < s->cfg.n_layers; l++) {
        free(s->k_cache[l]);
        free(s->v_cache[l]);
    }
    free(s->k_cache); free(s->v_cache);
    free(s->x); free(s->xb); free(s->xb2); free(s->q); free(s->att_out);
    free(s->hb); free(s->hb2);
    free(s);
}

const void *ifo_state_buffer(const ifo_state *s, int which, int layer) {
    switch (which) {
    case 0: return s->x;
    case 1: return s->k_cache[layer];
    case 2: return s->v_cache[layer];
    default: return NULL;
    }
}

static int tensor_gemv(const ifo_tensor *t, const float *x, float *y, int nthreads) {
    return ifo_gemv_quant(t->dtype, t->data, t->rows, t->cols, x, y, nthreads);
}

/* Llama2::launch (models/llama2/transformer.rs:409-481) with the token
 * embedding copy of chat_llama2.rs:217-219 and the state of
 * transformer.rs:46-137.  K/V are produced in f32, RoPE rotates q and k in
 * f32, and only then is the row stored (rounded to binary16 when kv_f16). */
int ifo_forward(const ifo_model *m, ifo_state *s, int token, int pos, float *logits,
                int nthreads) {
    const ifo_config *c = &m->cfg;
    int dim = c->hidden, hs = dim / c->n_heads;
    int kv_dim = dim * c->n_kv_heads / c->n_heads;
    if (token < 0 || token >= c->vocab || pos < 0 || pos >= c->max_pos) return -1;

    /* x <- dequant(token_embd)[token, :] (transformer.rs:366-374) */
    {
        int qk = ifo_block_elems(m->token_embd.dtype), bb = ifo_block_bytes(m->token_embd.dtype);
        const uint8_t *row = (const uint8_t *)m->token_embd.data + (size_t)token * (dim / qk) * bb;
        ifo_dequant(m->token_embd.dtype, row, (size_t)dim, s->x);
    }
    float *k = (float *)malloc((size_t)kv_dim * 4), *v = (float *)malloc((size_t)kv_dim * 4);
    ifo_attn_params ap = {(uint32_t)c->max_pos, (uint32_t)kv_dim,
                          (uint32_t)(c->n_heads / c->n_kv_heads), (uint32_t)c->n_heads,
                          (uint32_t)hs, (uint32_t)pos};
    for (int l = 0; l < c->n_layers; l++) {
        const ifo_layer *wl = &m->layers[l];
        ifo_rms_norm(s->xb, s->x, wl->attn_norm, dim, c->rms_eps);
        tensor_gemv(&wl->attn_q, s->xb, s->q, nthreads);
        tensor_gemv(&wl->attn_k, s->xb, k, nthreads);
        tensor_gemv(&wl->attn_v, s->xb, v, nthreads);
        /* transformer.rs:434-442: the biases are added before RoPE */
        if (wl->q_bias) ifo_add(s->q, wl->q_bias, dim);
        if (wl->k_bias) ifo_add(k, wl->k_bias, kv_dim);
        if (wl->v_bias) ifo_add(v, wl->v_bias, kv_dim);
        ifo_rope(c->rope_neox, s->q, dim, k, kv_dim, hs, pos, c->rope_theta);
        size_t off = (size_t)pos * kv_dim;
        if (c->kv_f16) {
            ifo_encode_f16_array(k, (uint16_t *)s->k_cache[l] + off, (size_t)kv_dim);
            ifo_encode_f16_array(v, (uint16_t *)s->v_cache[l] + off, (size_t)kv_dim);
        } else {
            memcpy((float *)s->k_cache[l] + off, k, (size_t)kv_dim * 4);
            memcpy((float *)s->v_cache[l] + off, v, (size_t)kv_dim * 4);
        }
        ifo_attention(&ap, s->q, s->k_cache[l], s->v_cache[l], c->kv_f16, s->att_out);
        tensor_gemv(&wl->attn_output, s->att_out, s->xb2, nthreads);
        ifo_add(s->x, s->xb2, dim);
        ifo_rms_norm(s->xb, s->x, wl->ffn_norm, dim, c->rms_eps);
        tensor_gemv(&wl->ffn_gate, s->xb, s->hb, nthreads);
        tensor_gemv(&wl->ffn_up, s->xb, s->hb2, nthreads);
        ifo_silu_mul(s->hb, s->hb2, c->ffn);
        tensor_gemv(&wl->ffn_down, s->hb, s->xb2, nthreads);
        ifo_add(s->x, s->xb2, dim);
    }
    ifo_rms_norm(s->xb, s->x, m->output_norm, dim, c->rms_eps);
    tensor_gemv(&m->output, s->xb, logits, nthreads);
    free(k);
    free(v);
    return 0;
}

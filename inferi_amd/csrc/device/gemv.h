// Dequant-fused GEMV for GGUF blocks on gfx950 (HBM-bound; no MFMA).
//
// Work mapping.  A workgroup is W waves of 64 lanes; each wave owns R
// consecutive rows of a W*R-row tile and walks the K range of those rows in
// steps: a block is split over LPB lanes (4 for the 256-element K-quants, so a
// lane owns 64 elements of a block; 2 for Q8_0) and a step covers 64/LPB
// consecutive blocks.  A wave's work is one flat stream of (tile, step) pairs
// (tiles with a grid stride), and the next step's weight loads, possibly in
// the next tile, are always issued before the current step computes; the
// first step's loads go out before x is staged.  Row results are combined
// with a DPP butterfly.
//
// Arithmetic: two paths.
//  - integer (default): x arrives quantized by the kernel that produced it
//    (16-element groups of 22-bit fixed point as three int8 digit planes,
//    see quant16 below); the quant codes are multiplied with v_dot4_i32_i8
//    and the block and group scales applied in fp32;
//  - exact fp32: x staged as f32 (times the RMSNorm weight), codes converted
//    and multiplied with fp32 FMAs.
// Both use the reference kernels' refactoring of the block affine map
// (inferi-shaders/src/gemv_quant_q4_k.rs:47-93):
//   sum_e (d1*q_e - m1) x_e = d1 * sum_e q_e x_e - m1 * sum_e x_e.
#pragma once
#include "dequant.h"

namespace ifr {

// Geometry of each mode's launch: the quantized-output modes need a tile of
// exactly 16 output values (one activation group).
template <int MODE>
struct GemvGeom {
    static constexpr int R = gemv_geom(MODE).R, W = gemv_geom(MODE).W;
    static constexpr bool PIPE = false;
};

// Scale/min pair for sub-blocks 2g and 2g+1 of a Q4_K/Q5_K block
// (get_scale_min_k4, crates/inferi/src/quantization.rs:394-402), branch-free:
// both encodings are computed and selected, since g differs between the
// lanes of a wave.
IFR_DEV void scale_min_pair(uint32_t g, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t &sc0, uint32_t &m0,
                            uint32_t &sc1, uint32_t &m1) {
    const uint32_t sh = 16u * (g & 1u);
    const uint32_t a0 = w0 >> sh, a1 = w1 >> sh, a2 = w2 >> sh;
    // j < 4: sc = q[j] & 63, m = q[j+4] & 63
    // j >= 4: sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4
    const uint32_t hs0 = ((a0 >> 6) & 3u) << 4, hm0 = ((a1 >> 6) & 3u) << 4;
    const uint32_t hs1 = ((a0 >> 14) & 3u) << 4, hm1 = ((a1 >> 14) & 3u) << 4;
    // all ones for g >= 2: a bit select, so the compiler emits no branch
    const uint32_t mk = 0u - (g >> 1);
    sc0 = ((a0 & 63u) & ~mk) | (((a2 & 15u) | hs0) & mk);
    m0 = ((a1 & 63u) & ~mk) | ((((a2 >> 4) & 15u) | hm0) & mk);
    sc1 = (((a0 >> 8) & 63u) & ~mk) | ((((a2 >> 8) & 15u) | hs1) & mk);
    m1 = (((a1 >> 8) & 63u) & ~mk) | ((((a2 >> 12) & 15u) | hm1) & mk);
}

IFR_DEV void lds16(const float *p, float *x) {
    const float4 *p4 = (const float4 *)__builtin_assume_aligned(p, 16);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 t = p4[i];
        x[4 * i] = t.x;
        x[4 * i + 1] = t.y;
        x[4 * i + 2] = t.z;
        x[4 * i + 3] = t.w;
    }
}

IFR_DEV float sum16v(const float *x) {
    float s0 = (x[0] + x[1]) + (x[2] + x[3]);
    float s1 = (x[4] + x[5]) + (x[6] + x[7]);
    float s2 = (x[8] + x[9]) + (x[10] + x[11]);
    float s3 = (x[12] + x[13]) + (x[14] + x[15]);
    return (s0 + s1) + (s2 + s3);
}

// Dot of 16 unsigned byte codes (four words) with x[0..15].
IFR_DEV float dot16u(uint32_t a, uint32_t b, uint32_t c, uint32_t d, const float *x) {
    float s = 0.0f;
    s = dot4u(a, x, s);
    s = dot4u(b, x + 4, s);
    s = dot4u(c, x + 8, s);
    s = dot4u(d, x + 12, s);
    return s;
}

template <int FMT>
struct QFmt;
template <>
struct QFmt<Q4_K> { static constexpr int QK = 256, BB = 144, LPB = 8; };
template <>
struct QFmt<Q5_K> { static constexpr int QK = 256, BB = 176, LPB = 8; };
template <>
struct QFmt<Q6_K> { static constexpr int QK = 256, BB = 210, LPB = 8; };
template <>
struct QFmt<Q8_0> { static constexpr int QK = 32, BB = 34, LPB = 2; };
template <>
struct QFmt<Q4_0> { static constexpr int QK = 32, BB = 18, LPB = 2; };
template <>
struct QFmt<Q4_1> { static constexpr int QK = 32, BB = 20, LPB = 2; };
template <>
struct QFmt<Q5_0> { static constexpr int QK = 32, BB = 22, LPB = 2; };
template <>
struct QFmt<Q5_1> { static constexpr int QK = 32, BB = 24, LPB = 2; };
template <>
struct QFmt<Q8_K> { static constexpr int QK = 256, BB = 292, LPB = 16; };
// unquantized matrices (GpuQuantTensor::F32 and the F16 tensors the
// reference converts to it, gemv_quant.rs:203-208, gguf.rs:113-128): a
// 32-element virtual block per two lanes, as the 32-element formats
template <>
struct QFmt<F16> { static constexpr int QK = 32, BB = 64, LPB = 2; };
template <>
struct QFmt<F32> { static constexpr int QK = 32, BB = 128, LPB = 2; };

// Codes of lane half c (elements 16c..16c+15) of a 32-element block whose
// qs byte j holds element j (low nibble) and j+16 (high), with the fifth bits
// (Q5_0/Q5_1: bit e of the word qh) when `qh` is given.
IFR_DEV uint4 codes32(uint4 qs, uint32_t c, bool five, uint32_t qh) {
    const uint32_t M = 0x0F0F0F0Fu, sh = 4u * c;
    uint4 r = make_uint4((qs.x >> sh) & M, (qs.y >> sh) & M, (qs.z >> sh) & M, (qs.w >> sh) & M);
    if (five) {
        const uint32_t h = qh >> (16u * c);
        r.x |= spread4_b4(h & 15u);
        r.y |= spread4_b4((h >> 4) & 15u);
        r.z |= spread4_b4((h >> 8) & 15u);
        r.w |= spread4_b4((h >> 12) & 15u);
    }
    return r;
}

// Header and codes of the 32-element formats (Q4_0 :66-82, Q4_1 :94-112,
// Q5_0 :123-143, Q5_1 :155-177 of crates/inferi/src/quantization.rs):
// d (and m) as f32, the 16 qs bytes and the 32 fifth bits.  Field offsets:
// Q4_0 d@0 qs@2; Q4_1 d@0 m@2 qs@4; Q5_0 d@0 qh@2 qs@6; Q5_1 d@0 m@2 qh@4 qs@8.
template <int FMT>
struct Blk32 {
    static constexpr bool FIVE = FMT == Q5_0 || FMT == Q5_1;  // a fifth bit per code
    static constexpr bool AFF = FMT == Q4_1 || FMT == Q5_1;   // y = q d + m, else (q - H) d
    static constexpr float H = FMT == Q4_0 ? 8.0f : 16.0f;    // the symmetric formats' offset
    static constexpr int QS = FMT == Q4_0 ? 2 : FMT == Q4_1 ? 4 : FMT == Q5_0 ? 6 : 8;
    uint4 qs;
    uint32_t dm, qh; // dm: d | m << 16
    IFR_DEV void load(const uint8_t *b) {
        if constexpr (QS % 4 == 0) qs = ld16_a4(b + QS);
        else qs = ld16_a2(b + QS);
        dm = AFF ? (ld_u16(b) | ld_u16(b + 2) << 16) : ld_u16(b);
        if constexpr (FMT == Q5_0) qh = ld_u16(b + 2) | ld_u16(b + 4) << 16;
        else if constexpr (FMT == Q5_1) qh = *(const uint32_t *)(b + 4);
        else qh = 0;
    }
    IFR_DEV float d() const { return f16_to_f32(dm & 0xFFFFu); }
    IFR_DEV float m() const { return f16_to_f32(dm >> 16); }
    IFR_DEV uint4 codes(uint32_t c) const { return codes32(qs, c, FIVE, qh); }
    // sum over the lane's 16 elements of y * x, from dq = sum q x and sx = sum x
    IFR_DEV float apply(float dq, float sx) const { return AFF ? d() * dq + m() * sx : d() * (dq - H * sx); }
};

// One lane's share of one block step for R rows: the raw bytes (load) and
// their dot with x (compute), split so the next step's loads can be in
// flight while this step computes.
template <int FMT, int R>
struct Chunk;

// Q4_K lane chunk c: qs bytes [16c, 16c+16) = elements 64g+16h+t (low
// nibbles) and 64g+32+16h+t (high nibbles), g = c/2, h = c%2.
template <int R>
struct Chunk<Q4_K, R> {
    uint4 hv[R], qv[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 144;
            hv[r] = ld16(b);
            qv[r] = ld16(b + 16 + 16 * c);
        }
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        const uint32_t g = c >> 1, h = c & 1u;
        float xl[16], xh[16];
        const float *xp = xs + kb * 256 + 64 * g + 16 * h;
        lds16(xp, xl);
        lds16(xp + 32, xh);
        const float sl = sum16v(xl), sh = sum16v(xh);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, m0, sc1, m1;
            scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
            const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
            const uint4 q = qv[r];
            const uint32_t M = 0x0F0F0F0Fu;
            const float dl = dot16u(q.x & M, q.y & M, q.z & M, q.w & M, xl);
            const float dh = dot16u((q.x >> 4) & M, (q.y >> 4) & M, (q.z >> 4) & M, (q.w >> 4) & M, xh);
            acc[r] += (d * (float)sc0) * dl - (dm * (float)m0) * sl + (d * (float)sc1) * dh - (dm * (float)m1) * sh;
        }
    }
};

// Q5_K: as Q4_K plus the fifth bit from qh[16h + t], bit 2g (low) / 2g+1 (high).
template <int R>
struct Chunk<Q5_K, R> {
    uint4 hv[R], qv[R], qhv[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
        const uint32_t h = c & 1u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 176;
            hv[r] = ld16(b);
            qhv[r] = ld16(b + 16 + 16 * h);
            qv[r] = ld16(b + 48 + 16 * c);
        }
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        const uint32_t g = c >> 1, h = c & 1u;
        float xl[16], xh[16];
        const float *xp = xs + kb * 256 + 64 * g + 16 * h;
        lds16(xp, xl);
        lds16(xp + 32, xh);
        const float sl = sum16v(xl), sh = sum16v(xh);
        const uint32_t s0 = 2 * g, s1 = 2 * g + 1;
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, m0, sc1, m1;
            scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
            const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
            const uint4 q = qv[r], e = qhv[r];
            const uint32_t M = 0x0F0F0F0Fu, B = 0x01010101u;
            const float dl = dot16u((q.x & M) | (((e.x >> s0) & B) << 4), (q.y & M) | (((e.y >> s0) & B) << 4),
                                    (q.z & M) | (((e.z >> s0) & B) << 4), (q.w & M) | (((e.w >> s0) & B) << 4), xl);
            const float dh = dot16u(((q.x >> 4) & M) | (((e.x >> s1) & B) << 4),
                                    ((q.y >> 4) & M) | (((e.y >> s1) & B) << 4),
                                    ((q.z >> 4) & M) | (((e.z >> s1) & B) << 4),
                                    ((q.w >> 4) & M) | (((e.w >> s1) & B) << 4), xh);
            acc[r] += (d * (float)sc0) * dl - (dm * (float)m0) * sl + (d * (float)sc1) * dh - (dm * (float)m1) * sh;
        }
    }
};

// Q6_K lane chunk c: i = c/4 (half), cp = c%4, s = cp%2, u = cp/2.  ql bytes
// [64i+16cp, +16): low nibbles are elements 128i+32u+16s+t, high nibbles +64;
// qh bytes [32i+16s, +16) give bits 2u..2u+1 (low) and 2u+4..2u+5 (high);
// scales 8i+s+2u and +4.  Blocks are 210 bytes, so fields are 2-byte aligned.
template <int R>
struct Chunk<Q6_K, R> {
    uint4 qlv[R], qhv[R];
    uint32_t dsc[R], scl[R], sch[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
        const uint32_t i = c >> 2, cp = c & 3u, s = cp & 1u, u = cp >> 1;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 210;
            qlv[r] = ld16_a2(b + 64 * i + 16 * cp);
            qhv[r] = ld16_a2(b + 128 + 32 * i + 16 * s);
            scl[r] = b[192 + 8 * i + s + 2 * u];
            sch[r] = b[192 + 8 * i + s + 2 * u + 4];
            dsc[r] = ld_u16(b + 208);
        }
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        const uint32_t i = c >> 2, cp = c & 3u, s = cp & 1u, u = cp >> 1;
        float xl[16], xh[16];
        const float *xp = xs + kb * 256 + 128 * i + 32 * u + 16 * s;
        lds16(xp, xl);
        lds16(xp + 64, xh);
        const float sl = sum16v(xl), sh = sum16v(xh);
        const uint32_t s0 = 2 * u, s1 = 2 * u + 4;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 q = qlv[r], e = qhv[r];
            const uint32_t M = 0x0F0F0F0Fu, B = 0x03030303u;
            const float dl = dot16u((q.x & M) | (((e.x >> s0) & B) << 4), (q.y & M) | (((e.y >> s0) & B) << 4),
                                    (q.z & M) | (((e.z >> s0) & B) << 4), (q.w & M) | (((e.w >> s0) & B) << 4), xl);
            const float dh = dot16u(((q.x >> 4) & M) | (((e.x >> s1) & B) << 4),
                                    ((q.y >> 4) & M) | (((e.y >> s1) & B) << 4),
                                    ((q.z >> 4) & M) | (((e.z >> s1) & B) << 4),
                                    ((q.w >> 4) & M) | (((e.w >> s1) & B) << 4), xh);
            const float d = f16_to_f32(dsc[r]);
            const float fl = (float)(int)(int8_t)scl[r], fh = (float)(int)(int8_t)sch[r];
            // codes are stored +32: sum (q-32) x = sum q x - 32 sum x
            acc[r] += (d * fl) * (dl - 32.0f * sl) + (d * fh) * (dh - 32.0f * sh);
        }
    }
};

// Q8_0 lane half c of block kb: qs bytes [16c, 16c+16).
template <int R>
struct Chunk<Q8_0, R> {
    uint4 qv[R];
    uint32_t dsc[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 34;
            dsc[r] = ld_u16(b);
            qv[r] = ld16_a2(b + 2 + 16 * c);
        }
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        float xv[16];
        lds16(xs + kb * 32 + 16 * c, xv);
        const float sx = sum16v(xv);
#pragma unroll
        for (int r = 0; r < R; r++) {
            // signed codes: (q ^ 0x80) = q + 128 as an unsigned byte
            const uint4 q = qv[r];
            const uint32_t F = 0x80808080u;
            const float dq = dot16u(q.x ^ F, q.y ^ F, q.z ^ F, q.w ^ F, xv);
            acc[r] += f16_to_f32(dsc[r]) * (dq - 128.0f * sx);
        }
    }
};

// F16 / F32 rows: lane c owns elements 16c..16c+15 of the 32-element
// virtual block kb, multiplied in fp32.
template <int R>
struct Chunk<F16, R> {
    uint4 h0[R], h1[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 64 + 32 * c;
            h0[r] = ld16(b);
            h1[r] = ld16(b + 16);
        }
    }
    // row r's 16 weights times x[0..15]
    IFR_DEV float dot(int r, const float *xv) const {
        const uint32_t w[8] = {h0[r].x, h0[r].y, h0[r].z, h0[r].w, h1[r].x, h1[r].y, h1[r].z, h1[r].w};
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) t = fmaf(f16_to_f32((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu), xv[i], t);
        return t;
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        float xv[16];
        lds16(xs + kb * 32 + 16 * c, xv);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += dot(r, xv);
    }
};
template <int R>
struct Chunk<F32, R> {
    uint4 v[R][4];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int k = 0; k < 4; k++) v[r][k] = ld16(rowp[r] + (size_t)kb * 128 + 64 * c + 16 * k);
    }
    IFR_DEV float dot(int r, const float *xv) const {
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            t = fmaf(__uint_as_float(v[r][k].x), xv[4 * k], t);
            t = fmaf(__uint_as_float(v[r][k].y), xv[4 * k + 1], t);
            t = fmaf(__uint_as_float(v[r][k].z), xv[4 * k + 2], t);
            t = fmaf(__uint_as_float(v[r][k].w), xv[4 * k + 3], t);
        }
        return t;
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        float xv[16];
        lds16(xs + kb * 32 + 16 * c, xv);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += dot(r, xv);
    }
};

// 32-element formats, lane half c of block kb (elements 16c..16c+15).
template <int FMT, int R>
struct Chunk32 {
    Blk32<FMT> b[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t) {
#pragma unroll
        for (int r = 0; r < R; r++) b[r].load(rowp[r] + (size_t)kb * QFmt<FMT>::BB);
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        float xv[16];
        lds16(xs + kb * 32 + 16 * c, xv);
        const float sx = sum16v(xv);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 q = b[r].codes(c);
            acc[r] += b[r].apply(dot16u(q.x, q.y, q.z, q.w, xv), sx);
        }
    }
};
template <int R>
struct Chunk<Q4_0, R> : Chunk32<Q4_0, R> {};
template <int R>
struct Chunk<Q4_1, R> : Chunk32<Q4_1, R> {};
template <int R>
struct Chunk<Q5_0, R> : Chunk32<Q5_0, R> {};
template <int R>
struct Chunk<Q5_1, R> : Chunk32<Q5_1, R> {};

// Q8_K (quantization.rs:204-212): d:f32@0 qs:i8[256]@4; lane c of 16 reads
// qs[16c, 16c+16).
template <int R>
struct Chunk<Q8_K, R> {
    uint4 qv[R];
    float dv[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 292;
            dv[r] = *(const float *)b;
            qv[r] = ld16_a4(b + 4 + 16 * c);
        }
    }
    IFR_DEV void compute(uint32_t kb, uint32_t c, const float *xs, float *acc) const {
        float xv[16];
        lds16(xs + kb * 256 + 16 * c, xv);
        const float sx = sum16v(xv);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 q = qv[r];
            const uint32_t F = 0x80808080u;
            const float dq = dot16u(q.x ^ F, q.y ^ F, q.z ^ F, q.w ^ F, xv);
            acc[r] += dv[r] * (dq - 128.0f * sx);
        }
    }
};

// ------------------------------------------------------------------------
// Integer path.  An activation vector of K values is kept as XQ (K % 16 == 0):
//   XA, XB, XC int8[K] @0, @K, @2K;  XS f32[K/16] @3K;  XSUM f32[K/16] @3K+K/4.
// Element i of group J = i/16 is x~_i = XS[J] * v_i, v_i = 65536*XA[i] +
// 256*XB[i] + XC[i] (balanced base-256 digits of a 22-bit code, |v| <=
// 2^21 - 1), XS[J] = max|x|_J / (2^21 - 1) and XSUM[J] = sum of x~ over the
// group: |x~ - x| <= max|x|_J * 2.4e-7.  A group's dot with the unsigned
// codes q of a K-quant is one exact int32, built by chaining three
// v_dot4_i32_i8 sums (sum q*XA, shifted left 8, plus sum q*XB, shifted left 8,
// plus sum q*XC); 16 codes of at most 63 times 2^21 stay below 2^31.  The
// group scale and the block scales are then applied in fp32.

IFR_DEV uint32_t xq_bytes(uint32_t K) { return 3 * K + K / 2; }

struct XQ {
    const int8_t *xa, *xb, *xc;
    const float *xs, *xsum;
    IFR_DEV XQ(const uint8_t *base, uint32_t K)
        : xa((const int8_t *)base), xb((const int8_t *)base + K), xc((const int8_t *)base + 2 * K),
          xs((const float *)(base + 3 * K)), xsum((const float *)(base + 3 * K + K / 4)) {}
};


constexpr float XQ_MAXCODE = 2097151.0f; // 2^21 - 1
// clamp to the code range in one v_med3_f32 (v * inv only overshoots it by
// rounding; the same value as a compare-and-select clamp for any non-NaN)
IFR_DEV float xq_clamp(float v) { return __builtin_amdgcn_fmed3f(v, -XQ_MAXCODE, XQ_MAXCODE); }

// Quantizes one value per lane into XQ at element i; the 16 lanes of a DPP
// row form one group (i % 16 == lane % 16).  Every lane of the wave must call
// it (the reductions read neighbours); `ok` gates the stores.
template <bool COH = false>
IFR_DEV void quant16(float v, bool ok, uint8_t *xq, uint32_t K, uint32_t i, int lane) {
    const float am = max16(fabsf(v));
    const float sc = am / XQ_MAXCODE;
    const float inv = am > 0.0f ? XQ_MAXCODE / am : 0.0f;
    const int q = (int)rintf(xq_clamp(v * inv));
    // balanced base-256 digits: dc, db in [-128, 127], da in [-32, 32]
    const int dc = ((q + 128) & 0xFF) - 128;
    const int q1 = (q - dc) >> 8;
    const int db = ((q1 + 128) & 0xFF) - 128;
    const int da = (q1 - db) >> 8;
    const float sq = sum16((float)q);
    if (ok) {
        st_out<COH>(xq + i, (uint8_t)(int8_t)da);
        st_out<COH>(xq + K + i, (uint8_t)(int8_t)db);
        st_out<COH>(xq + 2 * K + i, (uint8_t)(int8_t)dc);
        if ((lane & 15) == 0) {
            st_out<COH>((float *)(xq + 3 * K) + i / 16, sc);
            st_out<COH>((float *)(xq + 3 * K + K / 4) + i / 16, sc * sq);
        }
    }
}

// The same quantization with one whole 16-value group per lane (elements
// 16g .. 16g+15, as the bits of four uint4): the maximum, the two divisions
// and the sum of codes are issued once per 16 values instead of once per 4.
// Bytes are quant16's: the same scale, codes and digits, and the sum of
// codes formed from two exact 8-value halves with one final rounding.  The
// maximum uses the NaN-propagating v_maximum3 (no canonicalising moves);
// it equals quant16's for every non-NaN input.  Writes 16 bytes of each
// digit plane and the group's two floats through a generic pointer.
IFR_DEV void quant1x16(const uint4 (&u)[4], bool ok, uint8_t *xq, uint32_t K, uint32_t g) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        v[4 * k] = __uint_as_float(u[k].x);
        v[4 * k + 1] = __uint_as_float(u[k].y);
        v[4 * k + 2] = __uint_as_float(u[k].z);
        v[4 * k + 3] = __uint_as_float(u[k].w);
    }
    float am = fabsf(v[0]);
#pragma unroll
    for (int e = 1; e < 16; e++) am = __builtin_elementwise_maximum(am, fabsf(v[e]));
    const float sc = am / XQ_MAXCODE;
    const float inv = am > 0.0f ? XQ_MAXCODE / am : 0.0f;
    uint32_t wa[4] = {0, 0, 0, 0}, wb[4] = {0, 0, 0, 0}, wc[4] = {0, 0, 0, 0};
    float s0 = 0.0f, s1 = 0.0f; // exact: |code| <= 2^21, eight of them
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const float qf = rintf(xq_clamp(v[e] * inv));
        const int q = (int)qf;
        const int dc = ((q + 128) & 0xFF) - 128;
        const int q1 = (q - dc) >> 8;
        const int db = ((q1 + 128) & 0xFF) - 128;
        const int da = (q1 - db) >> 8;
        wa[e / 4] |= ((uint32_t)da & 0xFFu) << (8 * (e % 4));
        wb[e / 4] |= ((uint32_t)db & 0xFFu) << (8 * (e % 4));
        wc[e / 4] |= ((uint32_t)dc & 0xFFu) << (8 * (e % 4));
        if (e < 8) s0 += qf;
        else s1 += qf;
    }
    const float sq = s0 + s1;
    if (ok) {
        *(uint4 *)(xq + 16 * g) = make_uint4(wa[0], wa[1], wa[2], wa[3]);
        *(uint4 *)(xq + K + 16 * g) = make_uint4(wb[0], wb[1], wb[2], wb[3]);
        *(uint4 *)(xq + 2 * K + 16 * g) = make_uint4(wc[0], wc[1], wc[2], wc[3]);
        ((float *)(xq + 3 * K))[g] = sc;
        ((float *)(xq + 3 * K + K / 4))[g] = sc * sq;
    }
}

IFR_DEV uint4 ld_u4(const int8_t *p) { return *(const uint4 *)__builtin_assume_aligned(p, 16); }
IFR_DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
// c + sum over four words of codes q and x digits
IFR_DEV int sdot16(uint4 q, uint4 x, int c) {
    c = sdot4(q.x, x.x, c);
    c = sdot4(q.y, x.y, c);
    c = sdot4(q.z, x.z, c);
    return sdot4(q.w, x.w, c);
}
IFR_DEV uint4 and4(uint4 q, uint32_t m) { return make_uint4(q.x & m, q.y & m, q.z & m, q.w & m); }
IFR_DEV uint4 shr4(uint4 q, uint32_t s) { return make_uint4(q.x >> s, q.y >> s, q.z >> s, q.w >> s); }

// x digits of one 16-element group
struct XG {
    uint4 a, b, c;
};
IFR_DEV XG xg_load(const XQ &x, uint32_t e) { return XG{ld_u4(x.xa + e), ld_u4(x.xb + e), ld_u4(x.xc + e)}; }
// sum_e q_e v_e of one group for codes 0 <= q <= 63: exact in int32
IFR_DEV int gdot_u(uint4 q, const XG &x) {
    return sdot16(q, x.c, sdot16(q, x.b, sdot16(q, x.a, 0) << 8) << 8);
}
// the same for signed codes |q| <= 127, as a float (two exact int parts)
IFR_DEV float gdot_s(uint4 q, const XG &x) {
    const int hi = sdot16(q, x.a, 0);
    const int lo = sdot16(q, x.c, sdot16(q, x.b, 0) << 8);
    return fmaf((float)hi, 65536.0f, (float)lo);
}

// The integer chunks give the GEMV body four operations for the step of one
// lane: xscales (the scales and sums of the lane's four activation groups),
// xgroup (the x digits of group q), gdot (the exact int32 dot of row r's
// codes in group q with those digits) and combine (block and group scales
// applied in fp32, added to acc[r]).  The body feeds one group at a time so
// only one group of x digits is live in registers.
struct XS4 {
    float4 s, S;
};

template <int FMT, int R>
struct ChunkI;

// Q4_K, 4 lanes per block: lane g owns sub-blocks 2g (low nibbles, elements
// 64g+l) and 2g+1 (high nibbles, 64g+32+l), l = 0..31: qs bytes [32g, 32g+32).
// Group q = 0..3 holds elements 64g + 16q + (0..15).
template <int R>
struct ChunkI<Q4_K, R> {
    static constexpr int LPB = 4;
    static constexpr bool DIRECT = false;
    uint4 hv[R], q0[R], q1[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t g) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 144;
            hv[r] = ld16(b);
            q0[r] = ld16(b + 16 + 32 * g);
            q1[r] = ld16(b + 32 + 32 * g);
        }
    }
    static IFR_DEV XS4 xscales(const XQ &x, uint32_t kb, uint32_t g) {
        const uint32_t e = kb * 256 + 64 * g;
        return XS4{*(const float4 *)__builtin_assume_aligned(x.xs + e / 16, 16),
                   *(const float4 *)__builtin_assume_aligned(x.xsum + e / 16, 16)};
    }
    static IFR_DEV XG xgroup(const XQ &x, uint32_t kb, uint32_t g, int q) { return xg_load(x, kb * 256 + 64 * g + 16 * q); }
    IFR_DEV int gdot(uint32_t, int q, int r, const XG &xg) const {
        const uint32_t M = 0x0F0F0F0Fu;
        const uint4 c = q == 0 ? and4(q0[r], M) : q == 1 ? and4(q1[r], M) : q == 2 ? and4(shr4(q0[r], 4), M) : and4(shr4(q1[r], 4), M);
        return gdot_u(c, xg);
    }
    IFR_DEV void combine(uint32_t g, const int (&iv)[4][R], const XS4 &f, bool valid, float *acc) const {
        const float S_lo = f.S.x + f.S.y, S_hi = f.S.z + f.S.w;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float t_lo = fmaf((float)iv[0][r], f.s.x, (float)iv[1][r] * f.s.y);
            const float t_hi = fmaf((float)iv[2][r], f.s.z, (float)iv[3][r] * f.s.w);
            uint32_t sc0, m0, sc1, m1;
            scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
            const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
            const float v = (d * (float)sc0) * t_lo - (dm * (float)m0) * S_lo + (d * (float)sc1) * t_hi - (dm * (float)m1) * S_hi;
            acc[r] += valid ? v : 0.0f;
        }
    }
};

// Q5_K: as Q4_K, fifth bit of element l from qh[l], bit 2g (low) / 2g+1 (high).
template <int R>
struct ChunkI<Q5_K, R> {
    static constexpr int LPB = 4;
    static constexpr bool DIRECT = false;
    uint4 hv[R], q0[R], q1[R], e0[R], e1[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t g) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 176;
            hv[r] = ld16(b);
            e0[r] = ld16(b + 16);
            e1[r] = ld16(b + 32);
            q0[r] = ld16(b + 48 + 32 * g);
            q1[r] = ld16(b + 64 + 32 * g);
        }
    }
    static IFR_DEV XS4 xscales(const XQ &x, uint32_t kb, uint32_t g) { return ChunkI<Q4_K, R>::xscales(x, kb, g); }
    static IFR_DEV XG xgroup(const XQ &x, uint32_t kb, uint32_t g, int q) { return ChunkI<Q4_K, R>::xgroup(x, kb, g, q); }
    IFR_DEV int gdot(uint32_t g, int q, int r, const XG &xg) const {
        const uint32_t M = 0x0F0F0F0Fu, B = 0x10101010u;
        const bool hi = q >= 2;
        const uint32_t sh = 2 * g + (hi ? 1u : 0u); // qh bit of this sub-block
        const uint4 a = (q & 1) ? q1[r] : q0[r], h = (q & 1) ? e1[r] : e0[r];
        const uint4 n = hi ? shr4(a, 4) : a;
        // 4-bit code | fifth bit at bit 4 of each byte
        const uint4 c = make_uint4((n.x & M) | (((h.x >> sh) << 4) & B), (n.y & M) | (((h.y >> sh) << 4) & B),
                                   (n.z & M) | (((h.z >> sh) << 4) & B), (n.w & M) | (((h.w >> sh) << 4) & B));
        return gdot_u(c, xg);
    }
    IFR_DEV void combine(uint32_t g, const int (&iv)[4][R], const XS4 &f, bool valid, float *acc) const {
        const float S_lo = f.S.x + f.S.y, S_hi = f.S.z + f.S.w;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float t_lo = fmaf((float)iv[0][r], f.s.x, (float)iv[1][r] * f.s.y);
            const float t_hi = fmaf((float)iv[2][r], f.s.z, (float)iv[3][r] * f.s.w);
            uint32_t sc0, m0, sc1, m1;
            scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
            const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
            const float v = (d * (float)sc0) * t_lo - (dm * (float)m0) * S_lo + (d * (float)sc1) * t_hi - (dm * (float)m1) * S_hi;
            acc[r] += valid ? v : 0.0f;
        }
    }
};

// Q6_K, 4 lanes per block: lane c = 2i + u owns ql bytes [64i+32u, +32): low
// nibbles are elements 128i+32u+l, high nibbles 128i+64+32u+l (l = 0..31),
// with qh[32i+l] bits 2u..2u+1 / 2u+4..2u+5 and scales sc[8i+2u+l/16] /
// sc[8i+2u+4+l/16].  Codes are stored +32: sum (q-32) x = sum q x - 32 sum x.
// Groups q = 0..3 start at e, e+16 (low nibbles), e+64, e+80 (high), with
// e = 128i + 32u.
template <int R>
struct ChunkI<Q6_K, R> {
    static constexpr int LPB = 4;
    static constexpr bool DIRECT = false;
    uint4 l0[R], l1[R], h0[R], h1[R];
    uint32_t sc_lo[R], sc_hi[R], dd[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
        const uint32_t i = c >> 1, u = c & 1u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 210;
            l0[r] = ld16_a2(b + 64 * i + 32 * u);
            l1[r] = ld16_a2(b + 64 * i + 32 * u + 16);
            h0[r] = ld16_a2(b + 128 + 32 * i);
            h1[r] = ld16_a2(b + 144 + 32 * i);
            sc_lo[r] = ld_u16(b + 192 + 8 * i + 2 * u);
            sc_hi[r] = ld_u16(b + 196 + 8 * i + 2 * u);
            dd[r] = ld_u16(b + 208);
        }
    }
    static IFR_DEV uint32_t e0(uint32_t kb, uint32_t c) { return kb * 256 + 128 * (c >> 1) + 32 * (c & 1u); }
    static IFR_DEV XS4 xscales(const XQ &x, uint32_t kb, uint32_t c) {
        const uint32_t e = e0(kb, c);
        const float2 sl = *(const float2 *)(x.xs + e / 16), sh = *(const float2 *)(x.xs + e / 16 + 4);
        const float2 Sl = *(const float2 *)(x.xsum + e / 16), Sh = *(const float2 *)(x.xsum + e / 16 + 4);
        return XS4{make_float4(sl.x, sl.y, sh.x, sh.y), make_float4(Sl.x, Sl.y, Sh.x, Sh.y)};
    }
    static IFR_DEV XG xgroup(const XQ &x, uint32_t kb, uint32_t c, int q) {
        return xg_load(x, e0(kb, c) + (q >= 2 ? 64u : 0u) + 16u * (uint32_t)(q & 1));
    }
    IFR_DEV int gdot(uint32_t c, int q, int r, const XG &xg) const {
        const uint32_t M = 0x0F0F0F0Fu, B = 0x30303030u;
        const bool hi = q >= 2;
        const uint32_t sh = 2 * (c & 1u) + (hi ? 4u : 0u); // this lane's qh bit pair
        const uint4 a = (q & 1) ? l1[r] : l0[r], h = (q & 1) ? h1[r] : h0[r];
        const uint4 n = hi ? shr4(a, 4) : a;
        // 6-bit codes: ql nibble | (qh pair << 4)
        const uint4 cd = make_uint4((n.x & M) | (((h.x >> sh) << 4) & B), (n.y & M) | (((h.y >> sh) << 4) & B),
                                    (n.z & M) | (((h.z >> sh) << 4) & B), (n.w & M) | (((h.w >> sh) << 4) & B));
        return gdot_u(cd, xg);
    }
    IFR_DEV void combine(uint32_t, const int (&iv)[4][R], const XS4 &f, bool valid, float *acc) const {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float t0 = fmaf((float)iv[0][r], f.s.x, -32.0f * f.S.x);
            const float t1 = fmaf((float)iv[1][r], f.s.y, -32.0f * f.S.y);
            const float t2 = fmaf((float)iv[2][r], f.s.z, -32.0f * f.S.z);
            const float t3 = fmaf((float)iv[3][r], f.s.w, -32.0f * f.S.w);
            const float d = f16_to_f32(dd[r]);
            const float c0 = (float)(int)(int8_t)(sc_lo[r] & 0xFFu), c1 = (float)(int)(int8_t)(sc_lo[r] >> 8);
            const float c2 = (float)(int)(int8_t)(sc_hi[r] & 0xFFu), c3 = (float)(int)(int8_t)(sc_hi[r] >> 8);
            const float v = d * (c0 * t0 + c1 * t1 + c2 * t2 + c3 * t3);
            acc[r] += valid ? v : 0.0f;
        }
    }
};

// Q8_0, 2 lanes per block: lane c owns qs bytes [16c, 16c+16) (signed codes),
// which is exactly one activation group.
template <int R>
struct ChunkI<Q8_0, R> {
    static constexpr int LPB = 2;
    static constexpr bool DIRECT = true; // compute() does the whole step
    uint4 qv[R];
    uint32_t dd[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 34;
            dd[r] = ld_u16(b);
            qv[r] = ld16_a2(b + 2 + 16 * c);
        }
    }
    IFR_DEV void compute(const XQ &x, uint32_t kb, uint32_t c, bool valid, float *acc) const {
        const uint32_t e = kb * 32 + 16 * c;
        const XG xg = xg_load(x, e);
        const float s = x.xs[e / 16];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = f16_to_f32(dd[r]) * (gdot_s(qv[r], xg) * s);
            acc[r] += valid ? v : 0.0f;
        }
    }
};

// 32-element formats, 2 lanes per block: lane c owns elements 16c..16c+15,
// exactly one activation group.  The codes (at most 31) times the x digits
// form one exact int32 (gdot_u); the block affine map is applied in fp32:
//   sum (q - H) x = s*sum q v - H*S,  sum (q d + m) x = d*(s*sum q v) + m*S
// with s, S the group's scale and sum of x.
template <int FMT, int R>
struct ChunkI32 {
    static constexpr int LPB = 2;
    static constexpr bool DIRECT = true;
    Blk32<FMT> b[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t) {
#pragma unroll
        for (int r = 0; r < R; r++) b[r].load(rowp[r] + (size_t)kb * QFmt<FMT>::BB);
    }
    IFR_DEV void compute(const XQ &x, uint32_t kb, uint32_t c, bool valid, float *acc) const {
        const uint32_t e = kb * 32 + 16 * c;
        const XG xg = xg_load(x, e);
        const float s = x.xs[e / 16], S = x.xsum[e / 16];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = b[r].apply((float)gdot_u(b[r].codes(c), xg) * s, S);
            acc[r] += valid ? v : 0.0f;
        }
    }
};
template <int R>
struct ChunkI<Q4_0, R> : ChunkI32<Q4_0, R> {};
template <int R>
struct ChunkI<Q4_1, R> : ChunkI32<Q4_1, R> {};
template <int R>
struct ChunkI<Q5_0, R> : ChunkI32<Q5_0, R> {};
template <int R>
struct ChunkI<Q5_1, R> : ChunkI32<Q5_1, R> {};

// Q8_K, 4 lanes per block: lane c owns elements 64c..64c+63 (four groups),
// signed codes times the x digits as two exact int parts (gdot_s), times the
// group scale, then d.
template <int R>
struct ChunkI<Q8_K, R> {
    static constexpr int LPB = 4;
    static constexpr bool DIRECT = true;
    uint4 q[R][4];
    float dv[R];
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *b = rowp[r] + (size_t)kb * 292;
            dv[r] = *(const float *)b;
#pragma unroll
            for (int k = 0; k < 4; k++) q[r][k] = ld16_a4(b + 4 + 64 * c + 16 * k);
        }
    }
    IFR_DEV void compute(const XQ &x, uint32_t kb, uint32_t c, bool valid, float *acc) const {
        const uint32_t e0 = kb * 256 + 64 * c;
        const float4 s4 = *(const float4 *)__builtin_assume_aligned(x.xs + e0 / 16, 16);
        const float s[4] = {s4.x, s4.y, s4.z, s4.w};
        float t[R];
#pragma unroll
        for (int r = 0; r < R; r++) t[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const XG xg = xg_load(x, e0 + 16 * k);
#pragma unroll
            for (int r = 0; r < R; r++) t[r] = fmaf(gdot_s(q[r][k], xg), s[k], t[r]);
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += valid ? dv[r] * t[r] : 0.0f;
    }
};

// F16 / F32 rows on the integer path: lane c owns elements 16c..16c+15 of
// the 32-element virtual block, exactly one activation group; the group's
// 22-bit codes v (exact in f32) are rebuilt from the digit planes once and
// multiplied by the weights in fp32, then by the group scale.
IFR_DEV void xg_codes(const XG &g, float *v) {
    const uint32_t a[4] = {g.a.x, g.a.y, g.a.z, g.a.w}, b[4] = {g.b.x, g.b.y, g.b.z, g.b.w},
                   c[4] = {g.c.x, g.c.y, g.c.z, g.c.w};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int sh = 24 - 8 * (i & 3);
        const int da = (int32_t)(a[i >> 2] << sh) >> 24, db = (int32_t)(b[i >> 2] << sh) >> 24,
                  dc = (int32_t)(c[i >> 2] << sh) >> 24;
        v[i] = (float)(da * 65536 + db * 256 + dc);
    }
}
template <int FMT, int R>
struct ChunkIF {
    static constexpr int LPB = 2;
    static constexpr bool DIRECT = true;
    Chunk<FMT, R> w;
    IFR_DEV void load(const uint8_t *const *rowp, uint32_t kb, uint32_t c) { w.load(rowp, kb, c); }
    IFR_DEV void compute(const XQ &x, uint32_t kb, uint32_t c, bool valid, float *acc) const {
        const uint32_t e = kb * 32 + 16 * c;
        float v[16];
        xg_codes(xg_load(x, e), v);
        const float s = x.xs[e / 16];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += valid ? w.dot(r, v) * s : 0.0f;
    }
};
template <int R>
struct ChunkI<F16, R> : ChunkIF<F16, R> {};
template <int R>
struct ChunkI<F32, R> : ChunkIF<F32, R> {};

// One step of a lane for R rows (K-quants group by group), added to acc
// when `valid` (a select, not a branch).
template <int FMT, int R>
IFR_DEV void chunk_step(const ChunkI<FMT, R> &w, const XQ &x, uint32_t kb, uint32_t c, bool valid, float *acc) {
    if constexpr (ChunkI<FMT, R>::DIRECT) {
        w.compute(x, kb, c, valid, acc);
    } else {
        const XS4 sc = ChunkI<FMT, R>::xscales(x, kb, c);
        int iv[4][R];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const XG xg = ChunkI<FMT, R>::xgroup(x, kb, c, q);
#pragma unroll
            for (int r = 0; r < R; r++) {
                iv[q][r] = w.gdot(c, q, r, xg);
                // this group's sums are formed before the next group's x is
                // read (a compiler-only fence, no instruction is emitted):
                // one group of x digits is live at a time
                asm volatile("" : "+v"(iv[q][r])::"memory");
            }
        }
        w.combine(c, iv, sc, valid, acc);
    }
}

// QKV with NeoX RoPE (rope.rs:97-141): virtual rows 2j and 2j+1 of a q or
// k head are its rows j and j + hs/2, so that the two outputs one lane
// rotates together stay adjacent in the launch; v rows keep their order.
IFR_DEV uint32_t qkv_phys(const GemvArgs &a, uint32_t v) {
    if (!a.neox || v >= a.rows0 + a.rows1) return v;
    const uint32_t base = v < a.rows0 ? 0u : a.rows0, u = v - base, hs = a.head_size;
    const uint32_t r = u % hs;
    return base + (u - r) + (r >> 1) + (r & 1u) * (hs / 2);
}

template <int MODE>
IFR_DEV const uint8_t *gemv_row_ptr(const GemvArgs &a, uint32_t v) {
    if constexpr (MODE == GEMV_QKV) {
        v = qkv_phys(a, v);
        if (v < a.rows0) return a.w0 + (size_t)v * a.row_bytes;
        v -= a.rows0;
        if (v < a.rows1) return a.w1 + (size_t)v * a.row_bytes;
        return a.w2 + (size_t)(v - a.rows1) * a.row_bytes;
    } else if constexpr (MODE == GEMV_GATEUP) {
        return ((v & 1u) ? a.w1 : a.w0) + (size_t)(v >> 1) * a.row_bytes;
    } else {
        return a.w0 + (size_t)v * a.row_bytes;
    }
}

// One RoPE rotation of the adjacent pair at even index idx of a head-strided
// vector (inferi-shaders/src/rope.rs:51-92): theta = base^(-(idx mod hs)/hs)
// read from the state's table (rope_theta_f32 of every pair), angle =
// pos * theta.
IFR_DEV void rope_pair_theta(float &a, float &b, float theta, uint32_t pos) {
    const float ang = (float)pos * theta;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float x = a, y = b;
    a = cs * x - sn * y;
    b = sn * x + cs * y;
}
// The rotation of the prompt path, given the angle's cosine and sine (the
// prefill's per-pass table), written out so that the separate RoPE kernel
// and the GEMM epilogue that fuses it round alike: a' = cos a - sin b, b' =
// sin a + cos b, each one fused multiply-add over a rounded product.
IFR_DEV void rope_rotate(float &a, float &b, float cs, float sn) {
#pragma clang fp contract(off)
    const float x = a, y = b;
    a = fmaf(cs, x, -(sn * y));
    b = fmaf(sn, x, cs * y);
}
IFR_DEV void rope_pair(float &a, float &b, uint32_t idx, uint32_t hs, uint32_t pos, const float *theta_tab) {
    rope_pair_theta(a, b, theta_tab[(idx % hs) >> 1], pos);
}

// QKV epilogue of virtual rows v, v+1 (v even, one pair of one head): the
// Qwen2 biases added first, then RoPE on q and k (transformer.rs:434-445),
// q to a.y, k and v to this position's cache row.  Physical indices follow
// qkv_phys; the theta index of the pair is (v mod hs) / 2 in both variants.
IFR_DEV void qkv_store_pair(const GemvArgs &a, uint32_t v, float x0, float x1, uint32_t pos, const float *theta) {
    const bool is_q = v < a.rows0, is_k = !is_q && v < a.rows0 + a.rows1;
    const uint32_t base = is_q ? 0u : is_k ? a.rows0 : a.rows0 + a.rows1;
    const uint32_t idx = v - base;
    uint32_t i0 = idx, i1 = idx + 1;
    if (a.neox && (is_q || is_k)) {
        const uint32_t hs = a.head_size, r = idx % hs;
        i0 = idx - r + (r >> 1);
        i1 = i0 + hs / 2;
    }
    const float *bias = is_q ? a.q_bias : is_k ? a.k_bias : a.v_bias;
    if (bias) {
        x0 = x0 + bias[i0];
        x1 = x1 + bias[i1];
    }
    if (is_q || is_k) rope_pair(x0, x1, idx, a.head_size, pos, theta);
    if (is_q) {
        a.y[i0] = x0;
        a.y[i1] = x1;
        return;
    }
    const size_t off = (size_t)pos * a.kv_dim;
    void *cache = is_k ? a.k_cache : a.v_cache;
    if (a.kv_f16) {
        uint16_t *c16 = (uint16_t *)cache + off;
        if (i1 == i0 + 1) {
            *(uint32_t *)(c16 + i0) = (uint32_t)f32_to_f16(x0) | ((uint32_t)f32_to_f16(x1) << 16);
        } else {
            c16[i0] = f32_to_f16(x0);
            c16[i1] = f32_to_f16(x1);
        }
    } else {
        ((float *)cache)[off + i0] = x0;
        ((float *)cache)[off + i1] = x1;
    }
}

// Stages x (times gamma for the normalising modes) into LDS as f32 and
// returns this thread's share of sum(x^2).
template <bool NORM, int W>
IFR_DEV float gemv_stage_f32(const GemvArgs &a, float *xs) {
    float ss = 0.0f;
    for (uint32_t i = (uint32_t)threadIdx.x * 4; i < a.cols; i += 64 * W * 4) {
        float4 v = *(const float4 *)(a.x + i);
        if constexpr (NORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            const float4 g = *(const float4 *)(a.gamma + i);
            v.x *= g.x;
            v.y *= g.y;
            v.z *= g.z;
            v.w *= g.w;
        }
        *(float4 *)(xs + i) = v;
    }
    return ss;
}

// Exact fp32 path: W waves of R rows, tiles of W*R rows with a grid stride.
template <int FMT, int MODE, int R = GemvGeom<MODE>::R, int W = GemvGeom<MODE>::W, bool PIPE = GemvGeom<MODE>::PIPE>
__device__ void gemv_f32_body(const GemvArgs &a) {
    using CH = Chunk<FMT, R>;
    constexpr int LPB = QFmt<FMT>::LPB, BPI = 64 / LPB;
    constexpr bool NORM = (MODE == GEMV_QKV || MODE == GEMV_GATEUP || MODE == GEMV_HEAD);
    // RESID and GATEUP also quantize their output for the next GEMV: a tile
    // must then hold exactly one 16-value activation group
    constexpr bool QOUT = (MODE == GEMV_RESID || MODE == GEMV_GATEUP);
    static_assert(!QOUT || (MODE == GEMV_RESID ? W * R == 16 : W * R == 32), "tile must be one activation group");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float red[W];
    __shared__ uint64_t kred[W];
    __shared__ float tvals[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
    const uint32_t steps = (a.nb + BPI - 1) / BPI;
    const uint32_t ntiles = (a.total_rows + W * R - 1) / (W * R);

    const uint8_t *rowp[R];
    auto set_rows = [&](uint32_t t, const uint8_t **rp) {
        const uint32_t v0 = (t * W + (uint32_t)wave) * R;
#pragma unroll
        for (int r = 0; r < R; r++) rp[r] = gemv_row_ptr<MODE>(a, min(v0 + r, a.total_rows - 1));
    };
    CH A, B;
    uint32_t tile = blockIdx.x, step = 0;
    // the first step's weights do not depend on x: in flight before staging
    if (tile < ntiles) {
        set_rows(tile, rowp);
        if (bsub < a.nb) A.load(rowp, bsub, c);
    }

    float ss = gemv_stage_f32<NORM, W>(a, (float *)lds);
    float rs = 1.0f;
    if constexpr (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    if constexpr (NORM) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) t += red[w];
        rs = 1.0f / sqrtf(t / (float)a.cols + a.eps); // rms_norm.rs:115
    }
    const float *xf = (const float *)lds;
    uint32_t pos = 0;
    if constexpr (MODE == GEMV_QKV) pos = a.ctl->pos;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    uint64_t best = 0;

    // Row results of tile t: reduce, then the mode's epilogue.  Every wave of
    // the workgroup calls this for the same tile (barriers inside for QOUT).
    auto finish = [&](uint32_t t) {
        const uint32_t v0 = (t * W + (uint32_t)wave) * R;
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]) * rs;
        if constexpr (MODE == GEMV_PLAIN || MODE == GEMV_HEAD) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (lane == r && v0 + r < a.total_rows) a.y[v0 + r] = acc[r];
            if constexpr (MODE == GEMV_HEAD) {
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (v0 + r < a.total_rows) {
                        const uint64_t k = argmax_key(acc[r], v0 + r);
                        best = k > best ? k : best;
                    }
            }
        } else if constexpr (MODE == GEMV_RESID) {
            // x += W v, then x * gamma_next quantized for the next GEMV
#pragma unroll
            for (int r = 0; r < R; r++)
                if (lane == r && v0 + r < a.total_rows) {
                    const float xn = a.y[v0 + r] + acc[r];
                    a.y[v0 + r] = xn;
                    tvals[wave * R + r] = xn;
                }
            __syncthreads();
            if (wave == 0 && a.xq_out) {
                const uint32_t i = t * 16 + (uint32_t)(lane & 15);
                const bool ok = lane < 16 && i < a.total_rows;
                const float xn = ok ? tvals[lane & 15] : 0.0f;
                const float g = (ok && a.gamma_next) ? a.gamma_next[i] : 1.0f;
                quant16(xn * g, ok, a.xq_out, a.total_rows, i, lane);
                const float sq = sum16(xn * xn);
                if (lane == 0) a.ss_out[t] = sq;
            }
            __syncthreads();
        } else if constexpr (MODE == GEMV_GATEUP) {
            // virtual rows 2j (gate j) and 2j+1 (up j): h[j] = up * silu(gate)
#pragma unroll
            for (int p = 0; p < R / 2; p++)
                if (lane == p && v0 + 2 * p + 1 < a.total_rows) {
                    const float gt = acc[2 * p], up = acc[2 * p + 1];
                    const float h = up * (gt / (1.0f + expf(-gt)));
                    a.y[(v0 >> 1) + p] = h;
                    tvals[wave * (R / 2) + p] = h;
                }
            __syncthreads();
            if (wave == 0 && a.xq_out) {
                const uint32_t K = a.total_rows / 2;
                const uint32_t i = t * 16 + (uint32_t)(lane & 15);
                const bool ok = lane < 16 && i < K;
                quant16(ok ? tvals[lane & 15] : 0.0f, ok, a.xq_out, K, i, lane);
            }
            __syncthreads();
        } else if constexpr (MODE == GEMV_QKV) {
#pragma unroll
            for (int p = 0; p < R / 2; p++) {
                const uint32_t v = v0 + 2 * p;
                if (lane == p && v + 1 < a.total_rows) qkv_store_pair(a, v, acc[2 * p], acc[2 * p + 1], pos, a.rope_tab);
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
    };

    // One step of the flat (tile, step) stream: issue the next step's loads
    // into `nxt`, compute `cur`, finish the tile after its last step.
    auto advance = [&](CH &cur, CH &nxt) -> bool {
        uint32_t nt = tile, ns = step + 1;
        if (ns == steps) {
            nt = tile + gridDim.x;
            ns = 0;
        }
        const uint8_t *rown[R];
        if (nt < ntiles) {
            if (nt != tile) set_rows(nt, rown);
            const uint32_t kn = ns * BPI + bsub;
            if (kn < a.nb) nxt.load(nt != tile ? rown : rowp, kn, c);
        }
        const uint32_t kb = step * BPI + bsub;
        if (kb < a.nb) cur.compute(kb, c, xf, acc);
        if (ns == 0) {
            finish(tile);
            if (nt < ntiles) {
#pragma unroll
                for (int r = 0; r < R; r++) rowp[r] = rown[r];
            }
        }
        tile = nt;
        step = ns;
        return tile < ntiles;
    };
    if (tile < ntiles) {
        if constexpr (PIPE) {
            while (true) {
                if (!advance(A, B)) break;
                if (!advance(B, A)) break;
            }
        } else {
            // one stage: the step's loads are issued right before its compute
            // (latency hidden by the other waves of the CU instead)
            while (true) {
                const uint32_t kb = step * BPI + bsub;
                if (step != 0 || tile != blockIdx.x)
                    if (kb < a.nb) A.load(rowp, kb, c);
                if (kb < a.nb) A.compute(kb, c, xf, acc);
                if (++step == steps) {
                    finish(tile);
                    step = 0;
                    tile += gridDim.x;
                    if (tile >= ntiles) break;
                    set_rows(tile, rowp);
                }
            }
        }
    }

    if constexpr (MODE == GEMV_HEAD) {
        if (a.part_keys) {
            if (lane == 0) kred[wave] = best;
            __syncthreads();
            if (tid == 0) {
                uint64_t b = kred[0];
                for (int w = 1; w < W; w++) b = kred[w] > b ? kred[w] : b;
                a.part_keys[blockIdx.x] = b;
            }
        }
    }
}

// Epilogue arithmetic of the integer path's fused norms and activations, on
// the hardware's reciprocal, reciprocal square root and exp2 (each within
// about 1 ulp) instead of the correctly rounded library sequences (about 35
// instructions each, issued by every wave for its one or two outputs).
// RMSNorm scale 1 / sqrt(t / n + eps) (rms_norm.rs:115):
IFR_DEV float rms_scale(float t, uint32_t n, float eps) {
    return __builtin_amdgcn_rsqf(fmaf(t, __builtin_amdgcn_rcpf((float)n), eps));
}
// silu(g) = g / (1 + e^-g) (silu.rs:59): e^-g as 2^(-g log2 e); a large
// negative g gives 2^+inf = inf and g * 0 = -0, the function's limit.
IFR_DEV float silu_fast(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}

// ------------------------------------------------------------------------
// Integer path.  A workgroup of W waves (W = blockDim.x / 64) copies the
// input XQ into LDS once and then works through output groups of GR virtual
// rows (16; 32 for GATEUP, whose virtual rows 2j, 2j+1 are gate j and up j),
// groups with a grid stride.  Its waves form KS K-slices times RW = W / KS
// row waves: wave (rw, ks) takes R rows of each RW*R-row sub-tile of the
// group and the steps ks, ks + KS, ... of their K range.  The next item's
// weights are loaded before the current item computes (PIPE).
//  - KS = 1 and no quantized output (PLAIN, QKV, HEAD): each wave finishes
//    its own rows (store, RoPE and KV-cache store, argmax keys);
//  - otherwise each wave's row sums go to LDS, the workgroup synchronises
//    once per group and wave 0 adds the K-slices and runs the epilogue on the
//    group's 16 outputs (residual add and quantization of x * gamma_next for
//    the next GEMV, or silu(gate) * up and its quantization).
template <int FMT, int MODE, bool PIPE, int NI = 1, bool XF = false>
__device__ void gemv_int_body(const GemvArgs &a) {
    constexpr int R = 2;
    using CH = ChunkI<FMT, R>;
    constexpr int LPB = CH::LPB, BPI = 64 / LPB;
    constexpr bool NORM = (MODE == GEMV_QKV || MODE == GEMV_GATEUP || MODE == GEMV_HEAD);
    constexpr bool QOUT = (MODE == GEMV_RESID || MODE == GEMV_GATEUP);
    // output group: 16 values (32 virtual rows for GATEUP) where a group is
    // quantized or its K-slices are added; where waves finish their own rows
    // (one K-slice, no quantized output) a group is just the workgroup's rows
    constexpr uint32_t GRQ = MODE == GEMV_GATEUP ? 32 : 16;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float part[2][GEMV_KS_MAX][32];

    // the wave index is uniform across the wave: row addresses stay scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Every argument the prologue needs, read in one batch: left to itself
    // the compiler loads each field next to its first use and waits each
    // time, three dependent round trips before the first weight load.  (An
    // empty asm that takes them in scalar registers; it emits nothing.)
    asm volatile("" ::"s"(a.w0), "s"(a.w1), "s"(a.w2), "s"(a.rows0), "s"(a.rows1), "s"(a.total_rows), "s"(a.cols),
                 "s"(a.nb), "s"(a.row_bytes), "s"(a.n_ss), "s"(a.xq), "s"(a.ss_part), "s"(a.ks), "s"(a.y),
                 "s"(a.gamma_next), "s"(a.rope_tab), "s"(a.ctl), "s"(a.head_size), "s"(a.nwaves));
    // the launch shape comes from the arguments: reading blockDim costs a
    // vector load of the dispatch packet and a full wait at kernel entry
    const uint32_t W = a.nwaves, NT = W * 64, KS = a.ks, RW = W / KS;
    const uint32_t ks = (uint32_t)wave % KS, rw = (uint32_t)wave / KS;
    // a geometry that does not tile the group would never advance: the host
    // never launches one, and the workgroup exits as a whole if it did
    const bool local_rows = !QOUT && KS == 1;
    const uint32_t GR = local_rows ? RW * R : GRQ;
    if (KS == 0 || KS > GEMV_KS_MAX || RW == 0 || RW * KS != W || GR % (RW * R) != 0) return;
    const uint32_t SUBR = RW * R, SUB = GR / SUBR;
    const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
    const uint32_t steps = (a.nb + BPI - 1) / BPI;
    const uint32_t ngroups = (a.total_rows + GR - 1) / GR;
    const bool local = !QOUT && KS == 1; // waves finish their own rows

    // one work item: sub-tile j of group g, step st (st >= steps: none)
    struct Item {
        uint32_t g, j, st;
    };
    auto next = [&](Item it) {
        it.st += KS;
        if (it.st >= steps) {
            it.st = ks;
            if (++it.j == SUB) {
                it.j = 0;
                it.g += gridDim.x;
            }
        }
        return it;
    };
    // Loads are unconditional: an item past the end (or a lane past the
    // row's last block) reads a clamped, valid address and its data is not
    // used.  A load behind a branch would leave the compiler unsure which
    // buffer's loads are the newest at the join, and it would then wait for
    // the prefetched ones too before computing.
    auto load = [&](CH &w, const Item &it) {
        const uint32_t kb = min(min(it.st, steps - 1) * BPI + bsub, a.nb - 1);
        const uint32_t v0 = min(it.g, ngroups - 1) * GR + it.j * SUBR + rw * R;
        const uint8_t *rowp[R];
#pragma unroll
        for (int r = 0; r < R; r++) rowp[r] = gemv_row_ptr<MODE>(a, min(v0 + r, a.total_rows - 1));
        w.load(rowp, kb, c);
    };

    Item cur{blockIdx.x, 0, ks};
    CH A, B;
    if (cur.g >= ngroups) { // no work for this workgroup (the host never launches one)
        if constexpr (MODE == GEMV_HEAD)
            if (tid == 0 && a.part_keys) a.part_keys[blockIdx.x] = 0;
        return;
    }
    // Prologue order.  Loads complete in issue order, so every small input
    // (x's XQ copy, the RMSNorm partial sums, the RoPE thetas, the first
    // group's residual) is requested before the first item's weights: staging
    // x then waits for those few loads only, while the weights stream in.
    // The first XC chunks per thread and SC partial sums per lane are
    // straight-line loads of clamped (valid) addresses; loops cover larger
    // inputs.
    // XF: x arrives in f32 and this kernel quantizes it into LDS itself,
    // one 16-value group per thread (quant1x16, quant16's bytes): the four
    // chunks are the four 16-byte quarters of the thread's first group
    constexpr uint32_t XC = 4, SC = 4;
    const uint32_t n16 = XF ? a.cols / 4 : xq_bytes(a.cols) / 16;
    const uint32_t ngrp = a.cols / 16, gq = min((uint32_t)tid, ngrp - 1);
    const uint4 *xsrc = XF ? (const uint4 *)a.x : (const uint4 *)a.xq;
    static_assert(XC == 4, "four named chunks");
    const uint32_t xi0 = XF ? gq * 4 : min((uint32_t)tid, n16 - 1);
    const uint32_t xi1 = XF ? gq * 4 + 1 : min((uint32_t)tid + NT, n16 - 1);
    const uint32_t xi2 = XF ? gq * 4 + 2 : min((uint32_t)tid + 2 * NT, n16 - 1);
    const uint32_t xi3 = XF ? gq * 4 + 3 : min((uint32_t)tid + 3 * NT, n16 - 1);
    const uint4 xv0 = xsrc[xi0], xv1 = xsrc[xi1], xv2 = xsrc[xi2], xv3 = xsrc[xi3];
    float sv[SC];
    if constexpr (NORM) {
        // with no partial sums, a harmless read of x instead (never added)
        const float *ssp = a.n_ss ? a.ss_part : (const float *)a.xq;
        const uint32_t last = a.n_ss ? a.n_ss - 1 : 0;
#pragma unroll
        for (uint32_t j = 0; j < SC; j++) sv[j] = ssp[min((uint32_t)lane + 64 * j, last)];
    }
    uint32_t pos = 0;
    // QKV: the RoPE theta table (head_size/2 <= 64 values) read once into LDS
    __shared__ float theta_lds[64];
    float th = 0.0f;
    if constexpr (MODE == GEMV_QKV) {
        pos = a.ctl->pos;
        th = a.rope_tab[min((uint32_t)tid & 63u, a.head_size / 2 - 1)];
    }
    // RESID: wave 0 reads the group's residual and next RMSNorm weight before
    // the weights, so the epilogue waits for no load of its own
    float y_pre = 0.0f, g_pre = 1.0f;
    auto preload = [&](uint32_t g) {
        if constexpr (MODE == GEMV_RESID) {
            const uint32_t v = g * 16 + ((uint32_t)lane & 15u);
            if (wave == 0 && lane < 16 && v < a.total_rows) {
                y_pre = a.y[v];
                if (a.gamma_next) g_pre = a.gamma_next[v];
            }
        }
    };
    preload(cur.g);
    // keeps the small loads ahead of the weights (a scheduling fence only)
    __builtin_amdgcn_sched_barrier(0);
    load(A, cur);
    // NI = 2: the second item's weights are requested up front as well (a
    // workgroup whose second item lies past the end re-reads its first one)
    Item c2 = next(cur);
    if constexpr (NI >= 2) load(B, c2.g < ngroups ? c2 : cur);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XF) {
        // a wave with no group skips (uniform); in a wave that has some, a
        // thread past the last group quantizes it again with the stores off
        if ((uint32_t)wave * 64 < ngrp) {
            const uint4 u[4] = {xv0, xv1, xv2, xv3};
            quant1x16(u, (uint32_t)tid < ngrp, lds, a.cols, gq);
        }
        for (uint32_t g = (uint32_t)tid + NT; g < ngrp; g += NT) {
            const uint4 u[4] = {xsrc[4 * g], xsrc[4 * g + 1], xsrc[4 * g + 2], xsrc[4 * g + 3]};
            quant1x16(u, true, lds, a.cols, g);
        }
    } else {
        uint4 *dst = (uint4 *)lds;
        // unconditional stores (a thread past the end rewrites the last
        // chunk with its own value), so no load is moved behind a branch
        dst[xi0] = xv0;
        dst[xi1] = xv1;
        dst[xi2] = xv2;
        dst[xi3] = xv3;
        for (uint32_t i = (uint32_t)tid + XC * NT; i < n16; i += NT) dst[i] = xsrc[i];
    }
    float rs = 1.0f;
    if constexpr (NORM) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < SC; j++) t += (uint32_t)lane + 64 * j < a.n_ss ? sv[j] : 0.0f;
        for (uint32_t i = (uint32_t)lane + 64 * SC; i < a.n_ss; i += 64) t += a.ss_part[i];
        t = wave_sum(t);
        rs = rms_scale(t, a.cols, a.eps);
    }
    if constexpr (MODE == GEMV_QKV)
        if (tid < 64 && (uint32_t)tid < a.head_size / 2) theta_lds[tid] = th;
    __syncthreads();
    const XQ xq(lds, a.cols);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    uint64_t best = 0;
    uint32_t buf = 0;

    // outputs v, v+1 of a QKV launch (an even pair of one head): q, or RoPE'd
    // k / v into the cache row of this position
    auto qkv_store = [&](uint32_t v, float x0, float x1) { qkv_store_pair(a, v, x0, x1, pos, theta_lds); };

    // wave 0, after the group's barrier: the group's outputs
    auto epilogue = [&](uint32_t g) {
        auto val = [&](uint32_t i) {
            float t = part[buf][0][i];
            for (uint32_t k = 1; k < KS; k++) t += part[buf][k][i];
            return t * rs;
        };
        const uint32_t l = (uint32_t)lane & 15u;
        if constexpr (MODE == GEMV_PLAIN || MODE == GEMV_HEAD) {
            const uint32_t v = g * 16 + l;
            if (lane < 16 && v < a.total_rows) {
                const float y = val(l);
                a.y[v] = y;
                if constexpr (MODE == GEMV_HEAD) {
                    const uint64_t k = argmax_key(y, v);
                    best = k > best ? k : best;
                }
            }
        } else if constexpr (MODE == GEMV_RESID) {
            // x += W v, then x * gamma_next quantized for the next GEMV
            const uint32_t v = g * 16 + l;
            const bool ok = lane < 16 && v < a.total_rows;
            float xn = 0.0f;
            if (ok) {
                xn = y_pre + val(l);
                a.y[v] = xn;
            }
            if (a.xq_out) {
                quant16(xn * g_pre, ok, a.xq_out, a.total_rows, v, lane);
                const float sq = sum16(xn * xn);
                if (lane == 0) a.ss_out[g] = sq;
            }
        } else if constexpr (MODE == GEMV_GATEUP) {
            // h[j] = up * silu(gate), quantized for the down GEMV
            const uint32_t K = a.total_rows / 2, v = g * 16 + l;
            const bool ok = lane < 16 && v < K;
            float h = 0.0f;
            if (ok) {
                const float gt = val(2 * l), up = val(2 * l + 1);
                h = up * silu_fast(gt);
                a.y[v] = h;
            }
            if (a.xq_out) quant16(h, ok, a.xq_out, K, v, lane);
        } else if constexpr (MODE == GEMV_QKV) {
            const uint32_t v = g * 16 + 2 * (uint32_t)lane;
            if (lane < 8 && v + 1 < a.total_rows) qkv_store(v, val(2 * lane), val(2 * lane + 1));
        }
    };

    // every lane computes every item (on the clamped block for a lane past
    // the row's end or an item past the last step, which is then not added):
    // the loaded data is consumed on every path
    auto compute = [&](const CH &w, const Item &it) {
        const uint32_t kb = it.st * BPI + bsub;
        const bool valid = it.st < steps && kb < a.nb;
        chunk_step<FMT, R>(w, xq, min(min(it.st, steps - 1) * BPI + bsub, a.nb - 1), c, valid, acc);
        if (it.st + KS < steps) return; // more steps of this sub-tile
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
        if constexpr (!QOUT) {
            if (local) {
                const uint32_t v0 = it.g * GR + it.j * SUBR + rw * R;
                if constexpr (MODE == GEMV_QKV) {
                    if (lane == 0 && v0 + 1 < a.total_rows) qkv_store(v0, acc[0] * rs, acc[1] * rs);
                } else {
#pragma unroll
                    for (int r = 0; r < R; r++)
                        if (v0 + r < a.total_rows) {
                            const float y = acc[r] * rs;
                            if (lane == r) a.y[v0 + r] = y;
                            if constexpr (MODE == GEMV_HEAD) {
                                const uint64_t k = argmax_key(y, v0 + r);
                                best = k > best ? k : best;
                            }
                        }
                }
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] = 0.0f;
                return;
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) part[buf][ks][it.j * SUBR + rw * R + r] = acc[r];
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        if (it.j + 1 == SUB) {
            lds_barrier();
            if (wave == 0) {
                epilogue(it.g);
                preload(it.g + gridDim.x);
            }
            buf ^= 1u;
        }
    };

    if constexpr (PIPE) {
        // the scheduling barriers keep each prefetch ahead of the compute
        while (cur.g < ngroups) {
            Item nx = next(cur);
            load(B, nx);
            __builtin_amdgcn_sched_barrier(0);
            compute(A, cur);
            cur = nx;
            if (cur.g >= ngroups) break;
            nx = next(cur);
            load(A, nx);
            __builtin_amdgcn_sched_barrier(0);
            compute(B, cur);
            cur = nx;
        }
    } else {
        bool first = true;
        if constexpr (NI >= 2) {
            compute(A, cur);
            cur = c2;
            if (cur.g < ngroups) {
                compute(B, cur);
                cur = next(cur);
            }
            first = false;
        }
        while (cur.g < ngroups) {
            if (!first) load(A, cur);
            first = false;
            compute(A, cur);
            cur = next(cur);
        }
    }

    if constexpr (MODE == GEMV_HEAD) {
        if (a.part_keys) {
            // every wave holds keys when waves finish their own rows, else wave 0
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint64_t o = __shfl_xor((unsigned long long)best, off, 64);
                best = o > best ? o : best;
            }
            __shared__ uint64_t kred[GEMV_INT_MAX_WAVES];
            if (lane == 0) kred[wave] = best;
            __syncthreads();
            if (tid == 0) {
                uint64_t b = kred[0];
                for (uint32_t w = 1; w < W; w++) b = kred[w] > b ? kred[w] : b;
                a.part_keys[blockIdx.x] = b;
            }
        }
    }
}

// ------------------------------------------------------------------------
// One-item form of the integer path for the modes whose waves finish their
// own rows (PLAIN, QKV, HEAD, GATEUP) when a row is one 64-lane step (K <=
// 64/LPB blocks): workgroups of GEMV_ONE_WAVES waves of R rows each (R = 2
// or 4), one workgroup per R*GEMV_ONE_WAVES rows, launched all at once.
// Each wave requests x, then its rows' weights, then stages x and computes:
// no item loop, no buffers carried between items.  With R = 4 a wave's fixed
// work (staging, the RMSNorm scale, the reductions, the epilogue, which
// lanes 0 and 1 run side by side for two outputs) serves twice the rows.
// Same arithmetic and order as gemv_int_body for every R.
template <int FMT, int MODE, int R = 2, bool XF = false>
__device__ void gemv_one_body(const GemvArgs &a) {
    static_assert(R == 2 || R == 4, "two or four rows per wave");
    static_assert(!XF || MODE == GEMV_PLAIN, "f32 input only for the plain GEMV");
    using CH = ChunkI<FMT, R>;
    constexpr int LPB = CH::LPB;
    constexpr bool NORM = MODE == GEMV_QKV || MODE == GEMV_HEAD || MODE == GEMV_GATEUP;
    static_assert(MODE == GEMV_PLAIN || MODE == GEMV_QKV || MODE == GEMV_HEAD || MODE == GEMV_GATEUP,
                  "modes whose waves finish their own rows");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float theta_lds[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr uint32_t NT = GEMV_ONE_WAVES * 64;
    const uint32_t v0 = (blockIdx.x * GEMV_ONE_WAVES + (uint32_t)wave) * R;
    const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
    // x first (loads complete in issue order: staging waits for these only).
    // XF: x arrives in f32 (ifr_matmul_quant's caller) and is quantized into
    // LDS here, one 16-value group per thread (quant1x16: quant16's bytes),
    // instead of by a launch of its own: the four chunks are the four
    // 16-byte quarters of the thread's first group
    const uint32_t n16 = XF ? a.cols / 4 : xq_bytes(a.cols) / 16;
    const uint32_t ngrp = a.cols / 16, gq = min((uint32_t)tid, ngrp - 1);
    const uint4 *xsrc = XF ? (const uint4 *)a.x : (const uint4 *)a.xq;
    // four named chunks (an array here ends up in scratch memory)
    constexpr uint32_t XC = 4;
    const uint32_t xi0 = XF ? 4 * gq : min((uint32_t)tid, n16 - 1);
    const uint32_t xi1 = XF ? 4 * gq + 1 : min((uint32_t)tid + NT, n16 - 1);
    const uint32_t xi2 = XF ? 4 * gq + 2 : min((uint32_t)tid + 2 * NT, n16 - 1);
    const uint32_t xi3 = XF ? 4 * gq + 3 : min((uint32_t)tid + 3 * NT, n16 - 1);
    const uint4 xv0 = xsrc[xi0], xv1 = xsrc[xi1], xv2 = xsrc[xi2], xv3 = xsrc[xi3];
    float sv[4];
    uint32_t pos = 0;
    float th = 0.0f;
    if constexpr (NORM) {
        const float *ssp = a.n_ss ? a.ss_part : (const float *)a.xq;
        const uint32_t last = a.n_ss ? a.n_ss - 1 : 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) sv[j] = ssp[min((uint32_t)lane + 64 * j, last)];
        if constexpr (MODE == GEMV_QKV) {
            pos = a.ctl->pos;
            th = a.rope_tab[min((uint32_t)tid & 63u, a.head_size / 2 - 1)];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    CH w;
    {
        const uint8_t *rowp[R];
#pragma unroll
        for (int r = 0; r < R; r++) rowp[r] = gemv_row_ptr<MODE>(a, min(v0 + r, a.total_rows - 1));
        w.load(rowp, min(bsub, a.nb - 1), c);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XF) {
        // a wave with no group skips (uniform); in a wave that has some, a
        // thread past the last group quantizes it again with the stores off
        if ((uint32_t)wave * 64 < ngrp) {
            const uint4 u[4] = {xv0, xv1, xv2, xv3};
            quant1x16(u, (uint32_t)tid < ngrp, lds, a.cols, gq);
        }
        for (uint32_t g = (uint32_t)tid + NT; g < ngrp; g += NT) {
            const uint4 u[4] = {xsrc[4 * g], xsrc[4 * g + 1], xsrc[4 * g + 2], xsrc[4 * g + 3]};
            quant1x16(u, true, lds, a.cols, g);
        }
    } else {
        uint4 *dst = (uint4 *)lds;
        dst[xi0] = xv0;
        dst[xi1] = xv1;
        dst[xi2] = xv2;
        dst[xi3] = xv3;
        for (uint32_t i = (uint32_t)tid + XC * NT; i < n16; i += NT) dst[i] = xsrc[i];
    }
    float rs = 1.0f;
    if constexpr (NORM) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) t += (uint32_t)lane + 64 * j < a.n_ss ? sv[j] : 0.0f;
        for (uint32_t i = (uint32_t)lane + 256; i < a.n_ss; i += 64) t += a.ss_part[i];
        t = wave_sum(t);
        rs = rms_scale(t, a.cols, a.eps);
        if (MODE == GEMV_QKV && tid < 64 && (uint32_t)tid < a.head_size / 2) theta_lds[tid] = th;
    }
    __syncthreads();
    const XQ xq(lds, a.cols);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    chunk_step<FMT, R>(w, xq, min(bsub, a.nb - 1), c, bsub < a.nb, acc);
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    // lane p < R/2 takes the row pair (v0 + 2p, v0 + 2p + 1); with R = 2 the
    // pair index is the constant 0, so its row arithmetic stays scalar
    const uint32_t p = R == 2 ? 0u : (uint32_t)lane;
    const bool pl = R == 2 ? lane == 0 : (uint32_t)lane < R / 2;
    float pr0 = acc[0], pr1 = acc[1];
#pragma unroll
    for (int k = 1; k < R / 2; k++)
        if (p == (uint32_t)k) {
            pr0 = acc[2 * k];
            pr1 = acc[2 * k + 1];
        }
    if constexpr (MODE == GEMV_GATEUP) {
        // virtual rows v0 + 2p (gate j), v0 + 2p + 1 (up j): h[j] = up *
        // silu(gate), in f32 (the down GEMV quantizes it)
        if (pl && v0 + 2 * p + 1 < a.total_rows) {
            const float gt = pr0 * rs, up = pr1 * rs;
            a.y[(v0 >> 1) + p] = up * silu_fast(gt);
        }
    } else if constexpr (MODE == GEMV_QKV) {
        if (pl && v0 + 2 * p + 1 < a.total_rows)
            qkv_store_pair(a, v0 + 2 * p, pr0 * rs, pr1 * rs, pos, theta_lds);
    } else {
        uint64_t best = 0;
#pragma unroll
        for (int r = 0; r < R; r++)
            if (v0 + r < a.total_rows) {
                const float y = acc[r] * rs;
                if (lane == r) a.y[v0 + r] = y;
                if constexpr (MODE == GEMV_HEAD) {
                    const uint64_t k = argmax_key(y, v0 + r);
                    best = k > best ? k : best;
                }
            }
        if constexpr (MODE == GEMV_HEAD) {
            // the workgroup's key (every lane of a wave holds its wave's)
            __shared__ uint64_t kred[GEMV_ONE_WAVES];
            if (lane == 0) kred[wave] = best;
            __syncthreads();
            if (tid == 0 && a.part_keys) {
                uint64_t b = kred[0];
#pragma unroll
                for (uint32_t w2 = 1; w2 < GEMV_ONE_WAVES; w2++) b = kred[w2] > b ? kred[w2] : b;
                a.part_keys[blockIdx.x] = b;
            }
        }
    }
}

// One-item form of the grouped modes (RESID, GATEUP): a workgroup owns one
// output group (16 values: RESID 16 rows, GATEUP 16 gate/up pairs) with RW
// row waves of R rows times KS K-slices; every wave computes one item (its R
// rows over one 64-lane K step), the slices are added in LDS in slice
// order, and wave 0 runs gemv_int_body's epilogue.  Same arithmetic and
// order as gemv_int_body.
template <int FMT, int MODE, int R, int RW, int KS>
__device__ void gemv_grp_body(const GemvArgs &a) {
    static_assert(MODE == GEMV_RESID || MODE == GEMV_GATEUP, "grouped modes only");
    constexpr uint32_t GR = RW * R;
    static_assert(GR == (MODE == GEMV_GATEUP ? 32u : 16u), "one output group per workgroup");
    constexpr bool NORM = MODE == GEMV_GATEUP;
    using CH = ChunkI<FMT, R>;
    constexpr int LPB = CH::LPB, BPI = 64 / LPB;
    constexpr uint32_t NT = RW * KS * 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float part[KS][GR];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ks = (uint32_t)wave % KS, rw = (uint32_t)wave / KS, g = blockIdx.x;
    const uint32_t v0 = g * GR + rw * R;
    const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
    // x first (four named chunks: an array ends up in scratch memory)
    const uint32_t n16 = xq_bytes(a.cols) / 16;
    const uint4 *xsrc = (const uint4 *)a.xq;
    constexpr uint32_t XC = 4;
    const uint32_t xi0 = min((uint32_t)tid, n16 - 1), xi1 = min((uint32_t)tid + NT, n16 - 1);
    const uint32_t xi2 = min((uint32_t)tid + 2 * NT, n16 - 1), xi3 = min((uint32_t)tid + 3 * NT, n16 - 1);
    const uint4 xv0 = xsrc[xi0], xv1 = xsrc[xi1], xv2 = xsrc[xi2], xv3 = xsrc[xi3];
    float sv[4];
    if constexpr (NORM) {
        const float *ssp = a.n_ss ? a.ss_part : (const float *)a.xq;
        const uint32_t last = a.n_ss ? a.n_ss - 1 : 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) sv[j] = ssp[min((uint32_t)lane + 64 * j, last)];
    }
    // RESID: wave 0 reads the group's residual and next RMSNorm weight
    float y_pre = 0.0f, g_pre = 1.0f;
    if constexpr (MODE == GEMV_RESID) {
        const uint32_t v = g * 16 + ((uint32_t)lane & 15u);
        if (wave == 0 && lane < 16 && v < a.total_rows) {
            y_pre = a.y[v];
            if (a.gamma_next) g_pre = a.gamma_next[v];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    CH w;
    const uint32_t kb = ks * BPI + bsub;
    {
        const uint8_t *rowp[R];
#pragma unroll
        for (int r = 0; r < R; r++) rowp[r] = gemv_row_ptr<MODE>(a, min(v0 + r, a.total_rows - 1));
        w.load(rowp, min(kb, a.nb - 1), c);
    }
    __builtin_amdgcn_sched_barrier(0);
    {
        uint4 *dst = (uint4 *)lds;
        dst[xi0] = xv0;
        dst[xi1] = xv1;
        dst[xi2] = xv2;
        dst[xi3] = xv3;
        for (uint32_t i = (uint32_t)tid + XC * NT; i < n16; i += NT) dst[i] = xsrc[i];
    }
    float rs = 1.0f;
    if constexpr (NORM) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) t += (uint32_t)lane + 64 * j < a.n_ss ? sv[j] : 0.0f;
        for (uint32_t i = (uint32_t)lane + 256; i < a.n_ss; i += 64) t += a.ss_part[i];
        t = wave_sum(t);
        rs = rms_scale(t, a.cols, a.eps);
    }
    __syncthreads();
    const XQ xq(lds, a.cols);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    chunk_step<FMT, R>(w, xq, min(kb, a.nb - 1), c, kb < a.nb, acc);
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) part[ks][rw * R + r] = acc[r];
    }
    lds_barrier();
    if (wave != 0) return;
    auto val = [&](uint32_t i) {
        float t = part[0][i];
#pragma unroll
        for (uint32_t k = 1; k < KS; k++) t += part[k][i];
        return t * rs;
    };
    const uint32_t l = (uint32_t)lane & 15u;
    if constexpr (MODE == GEMV_RESID) {
        // x += W v, then x * gamma_next quantized for the next GEMV
        const uint32_t v = g * 16 + l;
        const bool ok = lane < 16 && v < a.total_rows;
        float xn = 0.0f;
        if (ok) {
            xn = y_pre + val(l);
            a.y[v] = xn;
        }
        if (a.xq_out) {
            quant16(xn * g_pre, ok, a.xq_out, a.total_rows, v, lane);
            const float sq = sum16(xn * xn);
            if (lane == 0) a.ss_out[g] = sq;
        }
    } else {
        // h[j] = up * silu(gate), quantized for the down GEMV
        const uint32_t K = a.total_rows / 2, v = g * 16 + l;
        const bool ok = lane < 16 && v < K;
        float h = 0.0f;
        if (ok) {
            const float gt = val(2 * l), up = val(2 * l + 1);
            h = up * silu_fast(gt);
            a.y[v] = h;
        }
        if (a.xq_out) quant16(h, ok, a.xq_out, K, v, lane);
    }
}

} // namespace ifr

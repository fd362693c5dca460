// Weight-tile loaders of the prefill GEMMs: a row's 32 elements of one K
// step read as GGUF block bytes and dequantized to f16 with the reference's
// f32 arithmetic (crates/inferi/src/quantization.rs:47-392).
#pragma once
#include "gemv.h"

namespace ifr {

// Weight tiles by format: row r's elements [k0 + 32*hs, +32) (k0 a multiple
// of 64, hs 0 or 1), loaded as raw bytes (load) and dequantized with the
// reference's f32 arithmetic, contraction off, then rounded to f16 (deq,
// through f16_run, whose conversion instruction is fixed so that the
// rounding is always f32 value -> f16).
// Runtime offsets select among loaded registers; nothing is indexed by a
// runtime value, so the staging stays in registers.
IFR_DEV uint32_t pick4(const uint4 &v, uint32_t i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
// byte l (0..31) of two 16-byte registers, l known at compile time after unrolling
IFR_DEV uint32_t byte32(const uint4 &a, const uint4 &b, int l) {
    const uint32_t w = l < 16 ? pick4(a, (uint32_t)(l >> 2)) : pick4(b, (uint32_t)((l - 16) >> 2));
    return (w >> (8 * (l & 3))) & 0xFFu;
}

// f16 pair of two f32 values, each rounded to nearest from its f32 value
// (v_cvt_pk_f16_f32 written out, so the compiler cannot fuse the producing
// multiply or FMA into one rounding straight to f16, v_fma_mix)
IFR_DEV uint32_t pack_f16x2(float a, float b) {
    uint32_t u;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(u) : "v"(a), "v"(b));
    return u;
}
// f16 of one f32 value (v_cvt_f16_f32 written out, for the same reason)
IFR_DEV _Float16 f16_of(float a) {
    uint32_t u;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(u) : "v"(a));
    const uint16_t b = (uint16_t)u;
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return h;
}
// h[l] = f16(y[l]) for the 32 values of a run, rounded from f32 by pack_f16x2
IFR_DEV void f16_run(const float *y, _Float16 *h) {
#pragma unroll
    for (int l = 0; l < 32; l += 2) {
        const uint32_t u = pack_f16x2(y[l], y[l + 1]);
        __builtin_memcpy(&h[l], &u, 4);
    }
}

template <int FMT>
struct PfTile;

// Q4_K (quantization.rs:358-392): sub-block 2g + hs of block k0/256.
template <>
struct PfTile<Q4_K> {
    static constexpr int QK = 256, BB = 144;
    uint4 hv, q0, q1;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t) {
        const uint32_t kb = k0 / 256, g = (k0 % 256) / 64;
        const uint8_t *b = wrow + (size_t)kb * 144;
        hv = ld16(b);
        q0 = ld16(b + 16 + 32 * g);
        q1 = ld16(b + 32 + 32 * g);
    }
    IFR_DEV void deq(uint32_t k0, uint32_t hs, _Float16 *h) const {
#pragma clang fp contract(off)
        const uint32_t g = (k0 % 256) / 64;
        uint32_t sc0, m0s, sc1, m1s;
        scale_min_pair(g, hv.y, hv.z, hv.w, sc0, m0s, sc1, m1s);
        const float d = f16_to_f32(hv.x & 0xFFFFu), dm = f16_to_f32(hv.x >> 16);
        const float d1 = d * (float)(hs ? sc1 : sc0), mm = dm * (float)(hs ? m1s : m0s);
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(q0, q1, l);
            const float q = (float)(hs ? (b >> 4) : (b & 15u));
            y[l] = d1 * q - mm;
        }
        f16_run(y, h);
    }
};

// Q5_K (quantization.rs:287-330): as Q4_K plus qh[l] bit 2g + hs.
template <>
struct PfTile<Q5_K> {
    static constexpr int QK = 256, BB = 176;
    uint4 hv, e0, e1, q0, q1;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t) {
        const uint32_t kb = k0 / 256, g = (k0 % 256) / 64;
        const uint8_t *b = wrow + (size_t)kb * 176;
        hv = ld16(b);
        e0 = ld16(b + 16);
        e1 = ld16(b + 32);
        q0 = ld16(b + 48 + 32 * g);
        q1 = ld16(b + 64 + 32 * g);
    }
    IFR_DEV void deq(uint32_t k0, uint32_t hs, _Float16 *h) const {
#pragma clang fp contract(off)
        const uint32_t g = (k0 % 256) / 64, sh = 2 * g + hs;
        uint32_t sc0, m0s, sc1, m1s;
        scale_min_pair(g, hv.y, hv.z, hv.w, sc0, m0s, sc1, m1s);
        const float d = f16_to_f32(hv.x & 0xFFFFu), dm = f16_to_f32(hv.x >> 16);
        const float d1 = d * (float)(hs ? sc1 : sc0), mm = dm * (float)(hs ? m1s : m0s);
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(q0, q1, l);
            const uint32_t q = (hs ? (b >> 4) : (b & 15u)) + (((byte32(e0, e1, l) >> sh) & 1u) ? 16u : 0u);
            y[l] = d1 * (float)q - mm;
        }
        f16_run(y, h);
    }
};

// Q6_K (quantization.rs:224-257): run j = 2*((k0%256)/64) + hs of 32
// elements 128i + 32k + l (i = j/4, k = j%4): ql[64i + 32(k&1) + l] (low
// nibble for k < 2), qh[32i + l] bits 2k..2k+1, scale[8i + 2k + l/16].
template <>
struct PfTile<Q6_K> {
    static constexpr int QK = 256, BB = 210;
    uint4 l0, l1, h0, h1;
    uint32_t sc, dd;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        const uint32_t kb = k0 / 256, j = 2 * ((k0 % 256) / 64) + hs, i = j >> 2, k = j & 3u;
        const uint8_t *b = wrow + (size_t)kb * 210;
        l0 = ld16_a2(b + 64 * i + 32 * (k & 1u));
        l1 = ld16_a2(b + 64 * i + 32 * (k & 1u) + 16);
        h0 = ld16_a2(b + 128 + 32 * i);
        h1 = ld16_a2(b + 144 + 32 * i);
        sc = ld_u16(b + 192 + 8 * i + 2 * k);
        dd = ld_u16(b + 208);
    }
    IFR_DEV void deq(uint32_t k0, uint32_t hs, _Float16 *h) const {
#pragma clang fp contract(off)
        const uint32_t k = (2 * ((k0 % 256) / 64) + hs) & 3u;
        const float d = f16_to_f32(dd);
        const float s_lo = (float)(int)(int8_t)(sc & 0xFFu), s_hi = (float)(int)(int8_t)(sc >> 8);
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t qlb = byte32(l0, l1, l);
            const uint32_t nib = k < 2 ? (qlb & 15u) : (qlb >> 4);
            const uint32_t hb = (byte32(h0, h1, l) >> (2 * k)) & 3u;
            const int q = (int)(nib | (hb << 4)) - 32;
            y[l] = d * (l < 16 ? s_lo : s_hi) * (float)q;
        }
        f16_run(y, h);
    }
};

// Q8_K (quantization.rs:204-212): d:f32, qs[(k0%256) + 32hs, +32).
template <>
struct PfTile<Q8_K> {
    static constexpr int QK = 256, BB = 292;
    uint4 q0, q1;
    uint32_t db;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        const uint8_t *b = wrow + (size_t)(k0 / 256) * 292;
        db = *(const uint32_t *)b;
        q0 = ld16_a4(b + 4 + (k0 % 256) + 32 * hs);
        q1 = ld16_a4(b + 20 + (k0 % 256) + 32 * hs);
    }
    IFR_DEV void deq(uint32_t, uint32_t, _Float16 *h) const {
#pragma clang fp contract(off)
        const float d = __uint_as_float(db);
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d * (float)(int)(int8_t)byte32(q0, q1, l);
        f16_run(y, h);
    }
};

// Unquantized rows (GpuQuantTensor::F32, and F16 which the reference
// converts to F32 at load, gguf.rs:113-128): elements k0 + 32hs .. +32 taken
// as they are (F16) or rounded to f16 (F32) for the matrix cores.
template <>
struct PfTile<F16> {
    static constexpr int QK = 1, BB = 2;
    uint4 v[4];
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        const uint8_t *b = wrow + 2 * (size_t)(k0 + 32 * hs);
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = ld16(b + 16 * k);
    }
    IFR_DEV void deq(uint32_t, uint32_t, _Float16 *h) const {
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t w = pick4(v[l >> 3], (uint32_t)((l >> 1) & 3));
            const uint16_t b = (uint16_t)((l & 1) ? (w >> 16) : (w & 0xFFFFu));
            __builtin_memcpy(&h[l], &b, 2);
        }
    }
};
template <>
struct PfTile<F32> {
    static constexpr int QK = 1, BB = 4;
    uint4 v[8];
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        const uint8_t *b = wrow + 4 * (size_t)(k0 + 32 * hs);
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = ld16(b + 16 * k);
    }
    IFR_DEV void deq(uint32_t, uint32_t, _Float16 *h) const {
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = __uint_as_float(pick4(v[l >> 2], (uint32_t)(l & 3)));
        f16_run(y, h);
    }
};

// The 32-element formats: the run is exactly block (k0 + 32hs)/32.
// Q8_0 (quantization.rs:47-55): d@0 qs:i8[32]@2, y = q * d.
template <>
struct PfTile<Q8_0> {
    static constexpr int QK = 32, BB = 34;
    uint4 q0, q1;
    uint32_t dd;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        const uint8_t *b = wrow + (size_t)((k0 + 32 * hs) / 32) * 34;
        dd = ld_u16(b);
        q0 = ld16_a2(b + 2);
        q1 = ld16_a2(b + 18);
    }
    IFR_DEV void deq(uint32_t, uint32_t, _Float16 *h) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(dd);
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = (float)(int)(int8_t)byte32(q0, q1, l) * d;
        f16_run(y, h);
    }
};

// Q4_0/Q4_1/Q5_0/Q5_1 (quantization.rs:66-177) through Blk32 (device/gemv.h):
// element l < 16 is the low nibble of qs byte l, element l >= 16 the high
// nibble of byte l - 16; the fifth bit is bit l of qh.
template <int FMT>
struct PfTile32 {
    static constexpr int QK = 32, BB = QFmt<FMT>::BB;
    Blk32<FMT> blk;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t hs) {
        blk.load(wrow + (size_t)((k0 + 32 * hs) / 32) * BB);
    }
    IFR_DEV void deq(uint32_t, uint32_t, _Float16 *h) const {
#pragma clang fp contract(off)
        const float d = blk.d(), m = Blk32<FMT>::AFF ? blk.m() : 0.0f;
        float y[32];
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(blk.qs, blk.qs, l & 15);
            uint32_t q = l < 16 ? (b & 15u) : (b >> 4);
            if constexpr (Blk32<FMT>::FIVE) q |= ((blk.qh >> l) & 1u) << 4;
            if constexpr (Blk32<FMT>::AFF) y[l] = (float)q * d + m;
            else y[l] = (float)((int)q - (int)Blk32<FMT>::H) * d;
        }
        f16_run(y, h);
    }
};
template <>
struct PfTile<Q4_0> : PfTile32<Q4_0> {};
template <>
struct PfTile<Q4_1> : PfTile32<Q4_1> {};
template <>
struct PfTile<Q5_0> : PfTile32<Q5_0> {};
template <>
struct PfTile<Q5_1> : PfTile32<Q5_1> {};

} // namespace ifr

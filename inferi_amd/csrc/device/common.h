// Device helpers for the gfx950 kernels: binary16 decode, 64-lane wave
// reductions over DPP, and loads of GGUF fields at the alignments the block
// formats give them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../kargs.h"

#define IFR_DEV __device__ __forceinline__

namespace ifr {

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
// matrix-core operand and accumulator vectors (v_mfma_f32_32x32x16_f16)
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_a16 __attribute__((ext_vector_type(4), aligned(16)));

// binary16 -> binary32.  v_cvt_f32_f16 is exact for every finite code,
// subnormals included (f16 denormals are not flushed in the default mode);
// exponent 31 decodes to +-inf or a NaN.
IFR_DEV float f16_to_f32(uint32_t h16) {
    _Float16 h;
    uint16_t b = (uint16_t)h16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// binary32 -> binary16, round to nearest even.
IFR_DEV uint16_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// DPP row-local butterfly steps (lanes exchange within a row of 16).
template <int CTRL>
IFR_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
#define DPP_QUAD_XOR1 0xB1   // quad_perm [1,0,3,2]
#define DPP_QUAD_XOR2 0x4E   // quad_perm [2,3,0,1]
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_MIRROR 0x140

// Sum over groups of 16 consecutive lanes; every lane of the group gets it.
IFR_DEV float sum16(float v) {
    v += dpp_f<DPP_QUAD_XOR1>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f<DPP_ROW_MIRROR>(v);
    return v;
}
// Sum over groups of 8 consecutive lanes.
IFR_DEV float sum8(float v) {
    v += dpp_f<DPP_QUAD_XOR1>(v);
    v += dpp_f<DPP_QUAD_XOR2>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    return v;
}
IFR_DEV float max16(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return v;
}
// Full 64-lane sum, result in every lane.
IFR_DEV float wave_sum(float v) {
    v = sum16(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}
IFR_DEV float wave_max(float v) {
    v = max16(v);
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Workgroup barrier that orders LDS only: this wave's LDS operations are
// complete (lgkmcnt 0) before it arrives, and no memory access is moved
// across it by the compiler.  Unlike __syncthreads it does not wait for the
// wave's outstanding global loads, so weights prefetched for the next item
// stay in flight.  Use only where the waves exchange data through LDS.
IFR_DEV void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Stores that another workgroup of the same launch reads after a grid
// barrier (COH): agent-scope atomic stores, which are written through to the
// device-coherent level instead of staying in this XCD's L2.  Plain stores
// otherwise (the kernel boundary makes them visible).
template <bool COH, typename T>
IFR_DEV void st_out(T *p, T v) {
    if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// 16 bytes at a 16-byte aligned address.
IFR_DEV uint4 ld16(const uint8_t *p) {
    u32x4_a16 v = *(const u32x4_a16 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes at a 2-byte aligned address, read with naturally aligned loads
// that never leave [p, p+16): one dword-aligned 16-byte load from p & ~3 and
// one 2-byte load for the tail when p is not dword aligned, then a funnel
// shift.  (Q6_K blocks are 210 bytes and Q8_0 blocks 34, so their fields sit
// at 2-byte alignment.)
IFR_DEV uint4 ld16_a2(const uint8_t *p) {
    uintptr_t a = (uintptr_t)p;
    uint32_t sb = (uint32_t)(a & 3u); // 0 or 2
    const uint8_t *a0 = (const uint8_t *)(a & ~(uintptr_t)3);
    u32x4_a4 w = *(const u32x4_a4 *)a0;
    uint32_t tail = *(const uint16_t *)(a0 + (sb ? 16 : 12));
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(w.y, w.x, sb);
    r.y = __builtin_amdgcn_alignbyte(w.z, w.y, sb);
    r.z = __builtin_amdgcn_alignbyte(w.w, w.z, sb);
    r.w = __builtin_amdgcn_alignbyte(tail, w.w, sb);
    return r;
}

// 16 bytes at a 4-byte aligned address.
IFR_DEV uint4 ld16_a4(const uint8_t *p) {
    u32x4_a4 v = *(const u32x4_a4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

IFR_DEV uint32_t ld_u16(const uint8_t *p) { return *(const uint16_t *)p; }

// Bit 4 of byte k set to bit k of b (k = 0..3): the fifth bits of four
// 5-bit codes moved next to their low nibbles.
IFR_DEV uint32_t spread4_b4(uint32_t b) { return ((b * 0x00204081u) & 0x01010101u) << 4; }

// Byte k (0..11) of the 12-byte K-quant scale field held in three words.
IFR_DEV uint32_t sbyte(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t k) {
    uint32_t w = k < 4 ? w0 : (k < 8 ? w1 : w2);
    return (w >> ((k & 3u) * 8u)) & 0xFFu;
}

// get_scale_min_k4 (crates/inferi/src/quantization.rs:394-402) on the
// 12-byte field held in three words.
IFR_DEV void scale_min_k4(uint32_t j, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = sbyte(w0, w1, w2, j) & 63u;
        m = sbyte(w0, w1, w2, j + 4) & 63u;
    } else {
        sc = (sbyte(w0, w1, w2, j + 4) & 15u) | ((sbyte(w0, w1, w2, j - 4) >> 6) << 4);
        m = (sbyte(w0, w1, w2, j + 4) >> 4) | ((sbyte(w0, w1, w2, j) >> 6) << 4);
    }
}

// Byte B (0..3) of a word as a float: one v_cvt_f32_ubyteB.  Written as
// inline assembly because after a nibble mask the compiler otherwise splits
// it into a bit-field extract plus a conversion.
template <int B>
IFR_DEV float ub(uint32_t w) {
    float r;
    if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
    return r;
}

// Dot of the four bytes of w (as unsigned integers) with x[0..3].
IFR_DEV float dot4u(uint32_t w, const float *x, float acc) {
    acc = fmaf(ub<0>(w), x[0], acc);
    acc = fmaf(ub<1>(w), x[1], acc);
    acc = fmaf(ub<2>(w), x[2], acc);
    acc = fmaf(ub<3>(w), x[3], acc);
    return acc;
}

// RoPE frequency base^(-head_dim/hs): the exponent is an f32 division as in
// inferi-shaders/src/rope.rs:76-77, the power is evaluated in f64 and rounded
// once, i.e. the correctly rounded f32 value (an f32 powf may be an ulp off,
// which the angle pos*theta amplifies at long positions).
IFR_DEV float rope_theta_f32(float base, float head_dim, float hs) {
    return (float)pow((double)base, (double)(-head_dim / hs));
}

// splitmix64 finaliser: a bijective 64-bit mix.
IFR_DEV uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Orderable key of a float (larger float -> larger key).
IFR_DEV uint32_t f32_order_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Argmax key: larger value wins, lower index wins among equal values.
IFR_DEV uint64_t argmax_key(float v, uint32_t idx) {
    return ((uint64_t)f32_order_key(v) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

} // namespace ifr

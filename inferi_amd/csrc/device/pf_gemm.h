// Prefill GEMM on the matrix cores with the weights dequantized in the tile
// staging: Y[m][n] = sum_k X[m][k] * deq(W)[n][k] for a pass of M prompt
// tokens (X f16 [M][ldx], W rows of GGUF blocks, Y f32 [M][ldy]).
//
// The reference has no batched prompt path: it feeds the prompt through its
// decode step one token at a time (crates/inferi-chat/src/chat_llama2.rs:
// 137-160), i.e. every product is a GEMV over the same GGUF rows
// (crates/inferi-shaders/src/gemv_quant_q4_k.rs:97-182).  Here a pass's
// products are GEMMs: each 256 (n) x 64 (k) weight tile is read as GGUF
// blocks, dequantized with the reference's f32 arithmetic
// (crates/inferi/src/quantization.rs:47-392), rounded to f16 and staged in
// LDS, where the 256 token rows of the workgroup's X tile share it.
//
// Workgroup: 8 waves (two per SIMD, so one wave's stalls are the other's
// issue slots), a 256 (m) x 256 (n) tile of Y.  Wave w owns the 128 x 64
// sub-tile m in [128 (w & 1), +128), n in [64 (w >> 1), +64): 4 x 2 blocks
// of v_mfma_f32_32x32x16_f16 (128 f32 accumulators per lane).  K runs in
// steps of 64 through two LDS buffers: X arrives by direct global-to-LDS
// loads, issued a step ahead; W's GGUF bytes arrive in registers two steps
// ahead and are dequantized into the other buffer while the matrix cores
// work on the current one, so one barrier per step suffices.  (Four waves
// of 128 x 128, one per SIMD, measured 10-20% slower.)  Q4_K products take
// a warp-specialized form of the same tile (pf_gemm_ws_body, below), where
// four more waves do all the loading and dequantizing.
//
// Rows of the virtual n range come from up to three matrices of one GGUF
// type stacked one after another (n < n1: w0, n < n2: w1, else w2), so Q, K
// and V run as one product writing adjacent columns.  In the SwiGLU form
// (EPI 2) the tile's n rows alternate in runs of 32 between the gate (w0)
// and up (w1) rows of the same 32 FFN indices, so each lane holds gate and up
// of the same (m, j) and the epilogue writes h[m][j] = f16(u * silu(g))
// straight into the down product's input (the reference's silu, silu.rs:
// 24-53, on the two products, with the hardware exp2 and reciprocal of the
// decode step's epilogue, silu_fast: the library's expf and correctly
// rounded division took about 25 VALU instructions per value, 64 values per
// lane at the end of every tile while the matrix cores idle).
#pragma once
#include "pf_tiles.h"

namespace ifr {

constexpr int PG_BM = 256, PG_BN = 256, PG_BK = 64;
constexpr int PG_THREADS = 512;

// epilogues
constexpr int PG_STORE = 0;  // Y = X W^T
constexpr int PG_ADD = 1;    // Y += X W^T (the residual stream)
constexpr int PG_SWIGLU = 2; // h = f16(up * silu(gate)), gate/up interleaved by 32 rows

// LDS tiles: 256 rows of 64 halves (128 B) without padding; the 16-byte
// chunk c of row r sits at chunk c ^ s(r), s(r) = ((r / 2) ^ 4 (r % 2)) % 8.
// The sixteen consecutive rows whose 16-byte chunks one read pass serves (64
// banks of 4 bytes, two rows per bank line) fall on distinct banks; the
// dequantized row stores, two threads per row, meet fewer conflicts than
// with s(r) = (r / 2) % 8 (a microbenchmark of the two access patterns:
// reads 5.1 -> 4.7, stores 16.0 -> 14.1 cycles per wave instruction and CU;
// the 4095-token 8B prefill 69.4 -> 69.1 ms, alternated three times).
IFR_DEV uint32_t pg_swz_of(uint32_t r) { return ((r >> 1) ^ ((r & 1u) << 2)) & 7u; }
IFR_DEV uint32_t pg_swz(uint32_t r, uint32_t c) { return r * PG_BK + 8 * (c ^ pg_swz_of(r)); }

typedef __attribute__((address_space(3))) char lds_char_t;

// LDS byte address of a pointer into a __shared__ array.
IFR_DEV uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(const lds_char_t *)p; }

// 16 bytes per lane from global memory straight into LDS: lane i writes
// LDS bytes [lds + 16 i, +16) (global_load_lds_dwordx4, LDS base in M0).
// Issued as assembly so the compiler's wait-count tracking leaves these
// loads to the kernel's own waits; the caller waits with vmcnt before the
// LDS is read.
// The address is a wave-uniform base plus this lane's 32-bit byte offset.
// M0 is reserved by the compiler (it sets M0 itself before each of its own
// uses and ignores a clobber entry for it); the compiler-generated code of
// these kernels does not read M0.
IFR_DEV void lds_dma16(const void *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds));
}

// 16-byte global load issued as assembly (not counted by the compiler's
// wait tracking): the caller waits with s_waitcnt before reading r.
IFR_DEV void ld16_asm(u32x4_a16 &r, const uint8_t *p) { asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p)); }

// Weight staging of one thread: half (part p) of one tile row's 64 elements
// in a K step, stored as four swizzled 16-byte chunks.  Generic: the PfTile
// loader's elements [32 p, +32) (chunks 4p .. 4p + 3), with compiler-tracked
// loads.
template <int FMT>
struct PgHalf {
    static constexpr bool MANUAL = false;
    PfTile<FMT> t;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t p) { t.load(wrow, k0, p); }
    template <int N>
    IFR_DEV void wait() {}
    IFR_DEV void store(uint32_t k0, uint32_t p, _Float16 *tile, uint32_t r) const {
        _Float16 h[32];
        t.deq(k0, p, h);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint4 u;
            __builtin_memcpy(&u, &h[8 * c], 16);
            *(uint4 *)(tile + pg_swz(r, 4 * p + (uint32_t)c)) = u;
        }
    }
};
// The block affine map of the step's two sub-blocks 2g, 2g + 1 (g = (k0 %
// 256) / 64): y = d1 q + n1 (low nibbles), d2 q + n2 (high nibbles).
struct Q4kAffine {
    float d1, n1, d2, n2;
};
IFR_DEV Q4kAffine q4k_affine(const u32x4_a16 &hv, uint32_t k0) {
#pragma clang fp contract(off)
    uint32_t sc0, m0s, sc1, m1s;
    scale_min_pair((k0 % 256) / 64, hv.y, hv.z, hv.w, sc0, m0s, sc1, m1s);
    const float d = f16_to_f32(hv.x & 0xFFFFu), dm = f16_to_f32(hv.x >> 16);
    return Q4kAffine{d * (float)sc0, -(dm * (float)m0s), d * (float)sc1, -(dm * (float)m1s)};
}
// The 16 qs bytes of part p (bytes [32 g + 16 p, +16) of the block's qs):
// low nibbles -> chunks 2p, 2p + 1, high nibbles -> chunks 4 + 2p, 5 + 2p of
// tile row r.
IFR_DEV void q4k_store_part(const u32x4_a16 &qv, const Q4kAffine &f, uint32_t p, _Float16 *tile, uint32_t r) {
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t l = q[i] & 0x0F0F0F0Fu, h = (q[i] >> 4) & 0x0F0F0F0Fu;
        lo[2 * i] = pack_f16x2(fmaf(f.d1, ub<0>(l), f.n1), fmaf(f.d1, ub<1>(l), f.n1));
        lo[2 * i + 1] = pack_f16x2(fmaf(f.d1, ub<2>(l), f.n1), fmaf(f.d1, ub<3>(l), f.n1));
        hi[2 * i] = pack_f16x2(fmaf(f.d2, ub<0>(h), f.n2), fmaf(f.d2, ub<1>(h), f.n2));
        hi[2 * i + 1] = pack_f16x2(fmaf(f.d2, ub<2>(h), f.n2), fmaf(f.d2, ub<3>(h), f.n2));
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
        *(uint4 *)(tile + pg_swz(r, 2 * p + (uint32_t)c)) = make_uint4(lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]);
        *(uint4 *)(tile + pg_swz(r, 4 + 2 * p + (uint32_t)c)) = make_uint4(hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]);
    }
}
// Q4_K (quantization.rs:358-392): part p takes qs bytes [32 g + 16 p, +16)
// of the step's group g = (k0 % 256) / 64: their low nibbles are elements
// 16 p .. 16 p + 15 (sub-block 2g; chunks 2p, 2p + 1), their high nibbles
// 32 + 16 p .. (sub-block 2g + 1; chunks 4 + 2p, 5 + 2p).  y = d1 * q - m1
// with d1 = d * sc and m1 = dmin * m: d1 * q is exact in f32 (at most 11 +
// 6 + 4 significant bits), so the fused multiply-add rounds once, exactly as
// the reference's multiply then subtract does.  The loads are issued as
// assembly and waited for with wait<N> (N = loads issued after them that may
// stay in flight).
// The same values with one instruction less per weight: a 4-bit code q in
// bits 0-3 (4-7) of a 16-bit half is the f16 subnormal q 2^-24 (q 2^-20),
// exactly, so fma(d1 2^24, that, n1) is fma(d1, q, n1), the same single f32
// rounding, with the code's conversion folded into the mixed-precision FMA
// (v_fma_mix_f32 reads the half in place).  Masks take two codes per
// instruction, one in each half; f16 subnormal inputs are kept (the default
// f16 denormal mode).
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
IFR_DEV void q4k_store_part_mix(const u32x4_a16 &qv, const Q4kAffine &f, uint32_t p, _Float16 *tile, uint32_t r) {
    const float dl = f.d1 * 0x1p24f, dh = f.d2 * 0x1p20f; // exact: powers of two
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t u = q[i], v = q[i] >> 8;
        // bytes 0, 2 (u) and 1, 3 (v): low nibbles at bits 0-3, high at 4-7
        const f16x2v l02 = __builtin_bit_cast(f16x2v, u & 0x000F000Fu), l13 = __builtin_bit_cast(f16x2v, v & 0x000F000Fu);
        const f16x2v h02 = __builtin_bit_cast(f16x2v, u & 0x00F000F0u), h13 = __builtin_bit_cast(f16x2v, v & 0x00F000F0u);
        lo[2 * i] = pack_f16x2(fmaf(dl, (float)l02.x, f.n1), fmaf(dl, (float)l13.x, f.n1));
        lo[2 * i + 1] = pack_f16x2(fmaf(dl, (float)l02.y, f.n1), fmaf(dl, (float)l13.y, f.n1));
        hi[2 * i] = pack_f16x2(fmaf(dh, (float)h02.x, f.n2), fmaf(dh, (float)h13.x, f.n2));
        hi[2 * i + 1] = pack_f16x2(fmaf(dh, (float)h02.y, f.n2), fmaf(dh, (float)h13.y, f.n2));
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
        *(uint4 *)(tile + pg_swz(r, 2 * p + (uint32_t)c)) = make_uint4(lo[4 * c], lo[4 * c + 1], lo[4 * c + 2], lo[4 * c + 3]);
        *(uint4 *)(tile + pg_swz(r, 4 + 2 * p + (uint32_t)c)) = make_uint4(hi[4 * c], hi[4 * c + 1], hi[4 * c + 2], hi[4 * c + 3]);
    }
}
template <>
struct PgHalf<Q4_K> {
    static constexpr bool MANUAL = true;
    u32x4_a16 hv, qv;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0, uint32_t p) {
        const uint8_t *b = wrow + (size_t)(k0 / 256) * 144;
        ld16_asm(hv, b);
        ld16_asm(qv, b + 16 + 32 * ((k0 % 256) / 64) + 16 * p);
    }
    template <int N>
    IFR_DEV void wait() {
        asm volatile("s_waitcnt vmcnt(%2)" : "+v"(hv), "+v"(qv) : "n"(N));
    }
    IFR_DEV void store(uint32_t k0, uint32_t p, _Float16 *tile, uint32_t r) const {
        q4k_store_part(qv, q4k_affine(hv, k0), p, tile, r);
    }
};
// Q4_K staging of one whole tile row (both parts) per thread, for the
// warp-specialized form: the block header once, then the 32 qs bytes.
struct PgRowQ4K {
    u32x4_a16 hv, q0, q1;
    IFR_DEV void load(const uint8_t *wrow, uint32_t k0) {
        const uint8_t *b = wrow + (size_t)(k0 / 256) * 144;
        const uint8_t *q = b + 16 + 32 * ((k0 % 256) / 64);
        ld16_asm(hv, b);
        ld16_asm(q0, q);
        ld16_asm(q1, q + 16);
    }
    template <int N>
    IFR_DEV void wait() {
        asm volatile("s_waitcnt vmcnt(%3)" : "+v"(hv), "+v"(q0), "+v"(q1) : "n"(N));
    }
    IFR_DEV void store(uint32_t k0, _Float16 *tile, uint32_t r) const {
        const Q4kAffine f = q4k_affine(hv, k0);
        q4k_store_part_mix(q0, f, 0, tile, r);
        q4k_store_part_mix(q1, f, 1, tile, r);
    }
};

// One workgroup's state over the K loop.
template <int FMT>
struct PgCtx {
    _Float16 *xs[2], *ws[2];
    const _Float16 *x;
    uint32_t xoff[4];            // this lane's X rows of its four direct loads
    const uint8_t *wrow;
    uint32_t r, p, nk, lane, wave, wm, wn;
    PgHalf<FMT> st0, st1;
    float16v acc[4][2];

    // X of step k into buffer B: four 1 KB direct loads per wave (lane l of
    // load j fills row 32 w + 8 j + l / 8 at physical chunk l % 8)
    template <int B>
    IFR_DEV void load_x(uint32_t k) {
        const uint32_t dst = lds_addr(xs[B] + (32 * wave) * PG_BK);
#pragma unroll
        for (int j = 0; j < 4; j++) lds_dma16(x + k * PG_BK, xoff[j], __builtin_amdgcn_readfirstlane(dst + 1024 * j));
    }
    template <int B>
    IFR_DEV void mfma_step() {
        const _Float16 *xb = xs[B], *wb = ws[B];
        const uint32_t li = lane & 31u, hi = lane >> 5;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            half8v av[4], bv[2];
            const uint32_t c = 2 * (uint32_t)kk + hi;
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = *(const half8v *)(xb + pg_swz(wm + 32 * i + li, c));
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = *(const half8v *)(wb + pg_swz(wn + 32 * j + li, c));
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    }
    // step s on buffer B: X of step s + 1 and the weights of step s + 2 are
    // requested, the products of step s run while the weights of step s + 1
    // (register set B ^ 1) are dequantized into the other buffer; at the end
    // this wave's LDS stores are done and its X loads have landed (the weight
    // loads issued after them may stay in flight), then the barrier.  Steps
    // past the end load step nk - 1 again into buffers nobody reads.  Loads in
    // flight at the wait: the 2 weight loads of step s + 1, then 4 X loads and
    // 2 weight loads of this step.
    template <int B>
    IFR_DEV void step(uint32_t s) {
        PgHalf<FMT> &ld = B ? st1 : st0, &dq = B ? st0 : st1;
        load_x<B ^ 1>(min(s + 1, nk - 1));
        ld.load(wrow, min(s + 2, nk - 1) * PG_BK, p);
        dq.template wait<6>();
        dq.store(min(s + 1, nk - 1) * PG_BK, p, ws[B ^ 1], r);
        mfma_step<B>();
        if constexpr (PgHalf<FMT>::MANUAL)
            asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
};

// The workgroup's output tile.  Tiles run in n-fastest order: consecutive
// workgroups share an X tile.  Workgroup b runs on XCD b % 8; tile t = (b %
// 8) * per + b / 8 gives each XCD a contiguous run of tiles (per = tiles / 8
// when it divides).
IFR_DEV void pg_tile(const PfGemmArgs &a, uint32_t &m0, uint32_t &n0) {
    const uint32_t tn = a.tiles_n, tiles = tn * a.tiles_m;
    const uint32_t b = blockIdx.x;
    const uint32_t t = (tiles & 7u) == 0 ? (b & 7u) * (tiles >> 3) + (b >> 3) : b;
    m0 = (t / tn) * PG_BM;
    n0 = (t % tn) * PG_BN;
}

// GGUF row of tile row r (rows past N repeat the last row).
template <int EPI>
IFR_DEV const uint8_t *pg_wrow(const PfGemmArgs &a, uint32_t n0, uint32_t r) {
    if constexpr (EPI == PG_SWIGLU) {
        // wave column c = r / 64 holds FFN rows j in [n0 / 2 + 32 c, +32):
        // tile rows 64 c + i are gate row j, 64 c + 32 + i up row j
        const uint32_t j = min(n0 / 2 + 32 * (r >> 6) + (r & 31u), a.n1 - 1);
        return ((r >> 5) & 1u ? a.w1 : a.w0) + (size_t)j * a.row_bytes;
    } else {
        const uint32_t n = min(n0 + r, a.N - 1);
        const uint8_t *base = n < a.n1 ? a.w0 : n < a.n2 ? a.w1 : a.w2;
        const uint32_t nr = n < a.n1 ? n : n < a.n2 ? n - a.n1 : n - a.n2;
        return base + (size_t)nr * a.row_bytes;
    }
}

// One wave's (32 MI) x 64 share of the tile out of its accumulators.
// D[row][col] of block (i, j): col = lane % 32 (n), row = 8 (e / 4) + 4 (lane
// / 32) + e % 4 (m).
template <int EPI, int MI = 4>
IFR_DEV void pg_epilogue(const PfGemmArgs &a, const float16v (&acc)[MI][2], uint32_t lane, uint32_t wm, uint32_t wn,
                         uint32_t m0, uint32_t n0) {
    const uint32_t li = lane & 31u;
    if constexpr (EPI == PG_SWIGLU) {
        const uint32_t jn = n0 / 2 + wn / 2 + li;
        if (jn >= a.n1) return;
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                if (m < a.M) {
                    const float gg = acc[i][0][e], u = acc[i][1][e];
                    ((_Float16 *)a.y)[(size_t)m * a.ldy + jn] = f16_of(u * silu_fast(gg));
                }
            }
    } else {
        // Y (ADD: Y + acc) block by block.  A block's 16 residual loads go
        // out together, from rows clamped below M (a clamped row is read, not
        // written), so a lane waits once per block instead of once per
        // element behind each element's bounds branch (the O and down
        // products' epilogue, 67 MB read and written at the 8B shape).
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t n = n0 + wn + 32 * j + li;
            if (n >= a.N) continue;
#pragma unroll
            for (int i = 0; i < MI; i++) {
                float old[16];
                if constexpr (EPI == PG_ADD) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                        old[e] = ((const float *)a.y)[(size_t)min(m, a.M - 1) * a.ldy + n];
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                    if (m < a.M) {
                        float *yp = (float *)a.y + (size_t)m * a.ldy + n;
                        if constexpr (EPI == PG_ADD)
                            *yp = old[e] + acc[i][j][e];
                        else
                            *yp = acc[i][j][e];
                    }
                }
            }
        }
    }
}

template <int FMT, int EPI>
__device__ __attribute__((always_inline)) void pf_gemm_body(const PfGemmArgs &a) {
    // four LDS objects, so the compiler sees that the direct loads into one
    // buffer do not alias the operand reads of the other
    __shared__ __attribute__((aligned(1024))) _Float16 xs0[PG_BM * PG_BK], xs1[PG_BM * PG_BK];
    __shared__ __attribute__((aligned(1024))) _Float16 ws0[PG_BN * PG_BK], ws1[PG_BN * PG_BK];
    PgCtx<FMT> g;
    const uint32_t tid = threadIdx.x;
    g.xs[0] = xs0;
    g.xs[1] = xs1;
    g.ws[0] = ws0;
    g.ws[1] = ws1;
    g.lane = tid & 63u;
    g.wave = tid >> 6;
    // weight staging: thread t takes part t % 2 of tile row t / 2 (mapping
    // the 16 lanes of an LDS pass to 16 consecutive rows of one chunk, which
    // removes the store bank conflicts, measured 0.4 ms slower per 8B
    // prefill: the conflicts are not on the critical path)
    g.r = tid >> 1;
    g.p = tid & 1u;
    g.wm = 128 * (g.wave & 1u);
    g.wn = 64 * (g.wave >> 1);
    g.nk = a.K / PG_BK;
    g.x = (const _Float16 *)a.x;
    uint32_t m0, n0;
    pg_tile(a, m0, n0);

#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t row = 32 * g.wave + 8 * (uint32_t)j + (g.lane >> 3);
        const uint32_t c = (g.lane & 7u) ^ pg_swz_of(row);
        g.xoff[j] = 2 * (min(m0 + row, a.M - 1) * a.ldx + 8 * c);
    }
    const uint32_t r = g.r;
    g.wrow = pg_wrow<EPI>(a, n0, r);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) g.acc[i][j][e] = 0.0f;

    // prologue: X and weights of step 0 into buffer 0, weights of step 1 in
    // flight
    g.template load_x<0>(0);
    g.st0.load(g.wrow, 0, g.p);
    g.st1.load(g.wrow, min(1u, g.nk - 1) * PG_BK, g.p);
    g.st0.template wait<2>();
    g.st0.store(0, g.p, ws0, r);
    if constexpr (PgHalf<FMT>::MANUAL)
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (uint32_t s = 0; s < g.nk; s += 2) {
        g.template step<0>(s);
        if (s + 1 < g.nk) g.template step<1>(s + 1);
    }
    // the clamped loads past the end: their destination registers stay
    // allocated until they have landed
    if constexpr (PgHalf<FMT>::MANUAL)
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(g.st0.hv), "+v"(g.st0.qv), "+v"(g.st1.hv), "+v"(g.st1.qv)::"memory");
    else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    pg_epilogue<EPI>(a, g.acc, g.lane, g.wm, g.wn, m0, n0);
}

// The store epilogue of the stacked Q | K | V product with the RoPE and
// KV-cache store fused (a.rope, warp-specialized form, pairs (2i, 2i + 1)):
// what the store epilogue and pf_rope_kv_k together do, bit for bit.  Column
// n is element e of q (n < n1), k (n < n2) or v; its bias is added, then q
// and k rotate with the pair partner, column n ^ 1, held by lane ^ 1 (the
// accumulator's columns are the lanes, and q, k and v start at even
// columns), with the (cos, sin) of the row's position and theta_(e mod hs)/2
// from the pass's table; q goes to Y, k and v to the cache rows of positions
// p0 + m.  Eight rows at a time: their table loads go out together from
// rows clamped below M.
template <int MI>
IFR_DEV void pg_epilogue_rope(const PfGemmArgs &a, const float16v (&acc)[MI][2], uint32_t lane, uint32_t wm,
                              uint32_t wn, uint32_t m0, uint32_t n0) {
    constexpr int RB = 4; // rows per batch
    const uint32_t li = lane & 31u, odd = lane & 1u, hh = a.head_size / 2, kd = a.n2 - a.n1;
    // per column block j: the column, its vector (0 q, 1 k, 2 v), element,
    // bias and table column
    bool nok[2];
    uint32_t n[2], seg[2], e[2], tj[2];
    float bv[2];
    bool hb[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        n[j] = n0 + wn + 32 * j + li;
        nok[j] = n[j] < a.N; // the same for both lanes of a pair
        const uint32_t nc = nok[j] ? n[j] : a.N - 1;
        seg[j] = nc < a.n1 ? 0u : nc < a.n2 ? 1u : 2u;
        e[j] = nc - (seg[j] == 0 ? 0u : seg[j] == 1 ? a.n1 : a.n2);
        // the three bias (and, below, cache) pointers are taken in branches
        // of their own: a select among them becomes a load from an indexed
        // copy of the argument block in scratch memory
        hb[j] = false;
        bv[j] = 0.0f;
        if (seg[j] == 0) {
            if (a.q_bias) {
                hb[j] = true;
                bv[j] = a.q_bias[e[j]];
            }
        } else if (seg[j] == 1) {
            if (a.k_bias) {
                hb[j] = true;
                bv[j] = a.k_bias[e[j]];
            }
        } else if (a.v_bias) {
            hb[j] = true;
            bv[j] = a.v_bias[e[j]];
        }
        tj[j] = ((e[j] & ~1u) % a.head_size) >> 1;
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int h = 0; h < 16; h += RB) {
            uint32_t m[RB];
            float cs[2][RB], sn[2][RB];
#pragma unroll
            for (int q = 0; q < RB; q++) {
                const int ee = h + q;
                m[q] = m0 + wm + 32 * i + 8 * (ee / 4) + 4 * (lane >> 5) + (ee % 4);
                const uint32_t rowt = min(m[q], a.M - 1) * hh;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float2 t = *(const float2 *)((const char *)a.rope_cs + 8u * (rowt + tj[j]));
                    cs[j][q] = t.x;
                    sn[j][q] = t.y;
                }
            }
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < RB; q++) {
                    float v = acc[i][j][h + q];
                    if (hb[j]) v = v + bv[j];
                    // lane ^ 1's value: a DPP quad permutation [1, 0, 3, 2]
                    // (every lane, before any branch)
                    const float pv = __builtin_bit_cast(
                        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
                    if (seg[j] < 2) {
                        float x = odd ? pv : v, y = odd ? v : pv;
                        rope_rotate(x, y, cs[j][q], sn[j][q]);
                        v = odd ? y : x;
                    }
                    if (nok[j] && m[q] < a.M) {
                        // 32-bit byte offsets from the uniform bases (the
                        // host fuses only caches under 4 GB per layer)
                        const uint32_t off = (a.p0 + m[q]) * kd + e[j];
                        if (seg[j] == 0)
                            *(float *)((char *)a.y + 4u * (m[q] * a.ldy + n[j])) = v;
                        else if (seg[j] == 1 && a.kv_f16)
                            *(uint16_t *)((char *)a.k_cache + 2u * off) = f32_to_f16(v);
                        else if (seg[j] == 1)
                            *(float *)((char *)a.k_cache + 4u * off) = v;
                        else if (a.kv_f16)
                            *(uint16_t *)((char *)a.v_cache + 2u * off) = f32_to_f16(v);
                        else
                            *(float *)((char *)a.v_cache + 4u * off) = v;
                    }
                }
            // one batch's loads and addresses at a time (hoisted across
            // batches they spill beside the accumulators)
            __builtin_amdgcn_sched_barrier(0);
        }
}

// The warp-specialized form's tile: workgroups below tiles_full take whole
// tiles as pg_tile maps them; the rest take the last tiles_n * tiles_m -
// tiles_full tiles as 256 x 128 halves, two workgroups per tile, so that a
// launch whose tiles leave its last round part-empty (the Q/K/V product at
// the 8B shape: 384 tiles for 256 CUs) ends in a round of halves over every
// CU.  Returns whether this workgroup takes a half.
IFR_DEV bool pg_tile_ws(const PfGemmArgs &a, uint32_t &m0, uint32_t &n0) {
    const uint32_t tn = a.tiles_n, tiles = tn * a.tiles_m, tf = a.tiles_full;
    const uint32_t b = blockIdx.x;
    if (b < tf) {
        const uint32_t t = (tf & 7u) == 0 ? (b & 7u) * (tf >> 3) + (b >> 3) : b;
        m0 = (t / tn) * PG_BM;
        n0 = (t % tn) * PG_BN;
        return false;
    }
    // halves: each XCD (b % 8 with tf a multiple of 8) a contiguous run
    const uint32_t h = b - tf, H = 2 * (tiles - tf);
    const uint32_t u = (H & 7u) == 0 && (tf & 7u) == 0 ? (h & 7u) * (H >> 3) + (h >> 3) : h;
    const uint32_t t = tf + u / 2;
    m0 = (t / tn) * PG_BM;
    n0 = (t % tn) * PG_BN + (PG_BN / 2) * (u & 1u);
    return true;
}

// A 256 x 128 half tile (pg_tile_ws): the MFMA waves own 64 x 64 shares (2 x
// 2 blocks), wave w at m 64 (w % 4), n 64 (w / 4); the staging waves load the
// same 256 X rows and dequantize the half's 128 weight rows, two threads per
// row (PgHalf's split: part t % 2 of row t / 2).  Each output is the same
// MFMA chain over K as in a whole tile, so the results are the same bit for
// bit.
template <int EPI>
__device__ __attribute__((always_inline)) void pf_gemm_ws_half(const PfGemmArgs &a, _Float16 *xs0, _Float16 *xs1, _Float16 *ws0, _Float16 *ws1,
                                uint32_t m0, uint32_t n0) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nk = a.K / PG_BK;
    if (wave < 8) {
        const uint32_t wm = 64 * (wave & 3u), wn = 64 * (wave >> 2);
        const uint32_t li = lane & 31u, hi = lane >> 5;
        float16v acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
        auto step = [&](const _Float16 *xb, const _Float16 *wb) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                half8v av[2], bv[2];
                const uint32_t c = 2 * (uint32_t)kk + hi;
#pragma unroll
                for (int i = 0; i < 2; i++) av[i] = *(const half8v *)(xb + pg_swz(wm + 32 * i + li, c));
#pragma unroll
                for (int j = 0; j < 2; j++) bv[j] = *(const half8v *)(wb + pg_swz(wn + 32 * j + li, c));
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
            }
        };
        asm volatile("s_barrier" ::: "memory");
        for (uint32_t s = 0; s < nk; s += 2) {
            step(xs0, ws0);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (s + 1 < nk) {
                step(xs1, ws1);
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
        }
        if (EPI == PG_STORE && a.rope)
            pg_epilogue_rope<2>(a, acc, lane, wm, wn, m0, n0);
        else
            pg_epilogue<EPI, 2>(a, acc, lane, wm, wn, m0, n0);
        return;
    }
    const uint32_t t = tid - 512u, v = wave - 8u, r = t >> 1, p = t & 1u;
    const _Float16 *x = (const _Float16 *)a.x;
    uint32_t xoff[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t row = 64 * v + 8 * (uint32_t)j + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ pg_swz_of(row);
        xoff[j] = 2 * (min(m0 + row, a.M - 1) * a.ldx + 8 * c);
    }
    const uint32_t xdst0 = lds_addr(xs0 + (64 * v) * PG_BK), xdst1 = lds_addr(xs1 + (64 * v) * PG_BK);
    auto load_x = [&](uint32_t dst, uint32_t k) {
#pragma unroll
        for (int j = 0; j < 8; j++) lds_dma16(x + k * PG_BK, xoff[j], __builtin_amdgcn_readfirstlane(dst + 1024 * j));
    };
    const uint8_t *wrow = pg_wrow<EPI>(a, n0, r);
    PgHalf<Q4_K> st0, st1;
    auto store = [&](const PgHalf<Q4_K> &st, uint32_t k0, _Float16 *tile) {
        q4k_store_part_mix(st.qv, q4k_affine(st.hv, k0), p, tile, r);
    };
    // as the whole tile's staging with two weight loads per step: in
    // flight at the weight waits the 10 loads issued after them, at the
    // step's end the 2 weight loads of the step after next
    load_x(xdst0, 0);
    st0.load(wrow, 0, p);
    st1.load(wrow, min(1u, nk - 1) * PG_BK, p);
    st0.template wait<2>();
    store(st0, 0, ws0);
    asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (uint32_t s = 0; s < nk; s += 2) {
        load_x(xdst1, min(s + 1, nk - 1));
        st0.load(wrow, min(s + 2, nk - 1) * PG_BK, p);
        st1.template wait<10>();
        store(st1, min(s + 1, nk - 1) * PG_BK, ws1);
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (s + 1 < nk) {
            load_x(xdst0, min(s + 2, nk - 1));
            st1.load(wrow, min(s + 3, nk - 1) * PG_BK, p);
            st0.template wait<10>();
            store(st0, min(s + 2, nk - 1) * PG_BK, ws0);
            asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(st0.hv), "+v"(st0.qv), "+v"(st1.hv), "+v"(st1.qv)::"memory");
}

// Warp-specialized form of the Q4_K product (option pf_ws): the same tile,
// LDS layout, products and epilogue, with the work split by role over 12
// waves, three per SIMD.  Waves 0-7 only read operands from LDS and run the
// MFMAs (each its 128 x 64 share, as above); waves 8-11 only stage: thread t
// of them requests the X rows (direct loads, a step ahead) and tile row t's
// GGUF bytes (header and 32 qs bytes, two steps ahead) and dequantizes the
// whole row's 64 weights of the next step into the other buffer (one
// thread per row: conflict-free row stores).  The dequantization runs in
// waves of its own beside the MFMA waves' products instead of in their
// instruction stream (4095-token 8B prefill 65.9 -> 62.1 ms).  One barrier
// per step for all 12 waves, as in the eight-wave form; the results are the
// same bit for bit (the same f16 operands, the same MFMA chains).
constexpr int PGW_THREADS = 768;
template <int EPI>
__device__ __attribute__((always_inline)) void pf_gemm_ws_body(const PfGemmArgs &a) {
    __shared__ __attribute__((aligned(1024))) _Float16 xs0[PG_BM * PG_BK], xs1[PG_BM * PG_BK];
    __shared__ __attribute__((aligned(1024))) _Float16 ws0[PG_BN * PG_BK], ws1[PG_BN * PG_BK];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nk = a.K / PG_BK;
    uint32_t m0, n0;
    if (pg_tile_ws(a, m0, n0)) { // (uniform)
        pf_gemm_ws_half<EPI>(a, xs0, xs1, ws0, ws1, m0, n0);
        return;
    }

    if (wave < 8) {
        // MFMA waves
        const uint32_t wm = 128 * (wave & 1u), wn = 64 * (wave >> 1);
        PgCtx<Q4_K> g;
        g.lane = lane;
        g.wm = wm;
        g.wn = wn;
        g.xs[0] = xs0;
        g.xs[1] = xs1;
        g.ws[0] = ws0;
        g.ws[1] = ws1;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) g.acc[i][j][e] = 0.0f;
        asm volatile("s_barrier" ::: "memory");
        for (uint32_t s = 0; s < nk; s += 2) {
            g.template mfma_step<0>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (s + 1 < nk) {
                g.template mfma_step<1>();
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
        }
        if (EPI == PG_STORE && a.rope)
            pg_epilogue_rope<4>(a, g.acc, lane, wm, wn, m0, n0);
        else
            pg_epilogue<EPI>(a, g.acc, lane, wm, wn, m0, n0);
        return;
    }

    // staging waves: thread t owns tile row t and, for the X tile, rows
    // 64 v + 8 j + lane / 8 of its wave v's eight direct loads j
    const uint32_t t = tid - 512u, v = wave - 8u;
    const _Float16 *x = (const _Float16 *)a.x;
    uint32_t xoff[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t row = 64 * v + 8 * (uint32_t)j + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ pg_swz_of(row);
        xoff[j] = 2 * (min(m0 + row, a.M - 1) * a.ldx + 8 * c);
    }
    const uint32_t xdst0 = lds_addr(xs0 + (64 * v) * PG_BK), xdst1 = lds_addr(xs1 + (64 * v) * PG_BK);
    auto load_x = [&](uint32_t dst, uint32_t k) {
#pragma unroll
        for (int j = 0; j < 8; j++) lds_dma16(x + k * PG_BK, xoff[j], __builtin_amdgcn_readfirstlane(dst + 1024 * j));
    };
    const uint8_t *wrow = pg_wrow<EPI>(a, n0, t);
    PgRowQ4K st0, st1;
    // prologue: X and weights of step 0 into buffer 0, weights of step 1 in
    // flight (loads in flight at the first wait: the 3 of step 1)
    load_x(xdst0, 0);
    st0.load(wrow, 0);
    st1.load(wrow, min(1u, nk - 1) * PG_BK);
    st0.template wait<3>();
    st0.store(0, ws0, t);
    asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // step s: X of step s + 1 (8 loads) and the weights of step s + 2 (3)
    // are requested, then the weights of step s + 1 are waited for (the 11
    // just issued may stay in flight) and dequantized into the other buffer;
    // at the end the X loads have landed (the 3 weight loads may stay in
    // flight), then the barrier.  Steps past the end load step nk - 1 again
    // into buffers nobody reads.
    for (uint32_t s = 0; s < nk; s += 2) {
        load_x(xdst1, min(s + 1, nk - 1));
        st0.load(wrow, min(s + 2, nk - 1) * PG_BK);
        st1.template wait<11>();
        st1.store(min(s + 1, nk - 1) * PG_BK, ws1, t);
        asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (s + 1 < nk) {
            load_x(xdst0, min(s + 2, nk - 1));
            st1.load(wrow, min(s + 3, nk - 1) * PG_BK);
            st0.template wait<11>();
            st0.store(min(s + 2, nk - 1) * PG_BK, ws0, t);
            asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
    }
    // the clamped loads past the end: their destination registers stay
    // allocated until they have landed
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(st0.hv), "+v"(st0.q0), "+v"(st0.q1), "+v"(st1.hv), "+v"(st1.q0),
                 "+v"(st1.q1)::"memory");
}

} // namespace ifr

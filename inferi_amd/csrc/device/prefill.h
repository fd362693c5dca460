// Prompt (prefill) kernels: a chunk of M tokens through one decoder layer.
//
// The reference feeds a prompt through its decode step one token at a time
// (crates/inferi-chat/src/chat_llama2.rs:137-160).  Here the prompt's
// matrix products are GEMMs on the matrix cores: weight tiles of any GGUF
// quantized format are dequantized (the reference's arithmetic,
// quantization.rs:47-392) into LDS as f16, the activations arrive as f16, and v_mfma_f32_32x32x16_f16
// accumulates in f32.  Around them: embedding, RMSNorm to f16, RoPE plus
// the KV-cache store, causal attention over the cache, and silu(g) * u.
// The prompt's last token then goes through the ordinary decode step,
// which produces the logits and the next token.
#pragma once
#include "attention.h"

namespace ifr {


// ------------------------------------------------------------------ GEMM --
// Y[m][n] = sum_k X[m][k] * deq(W)[n][k]   (EPI 0: Y =, EPI 1: Y +=)
// X: f16, row m at x + m * ldx; W: rows of K/QK GGUF blocks; Y: f32, row m
// at y + m * ldy.  Tile 128 (m) x 128 (n), K steps of 64; four waves, each a
// 64 x 64 quadrant as 2 x 2 MFMA 32x32x16 tiles.  The next K step's global
// loads are issued before the current step's MFMAs.
constexpr int PF_BM = 128, PF_BN = 128, PF_BK = 64;
constexpr int PF_LDS = PF_BK + 8; // halves per LDS row: 144 B, so the 32 rows an MFMA operand read touches spread over the banks

// Weight tiles by format: row r's elements [k0 + 32*hs, +32) (k0 a multiple
// of 64, hs 0 or 1), loaded as raw bytes (load) and dequantized with the
// reference's f32 arithmetic, contraction off, then rounded to f16 (deq).
// Runtime offsets select among loaded registers; nothing is indexed by a
// runtime value, so the staging stays in registers.
IFR_DEV uint32_t pick4(const uint4 &v, uint32_t i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
// byte l (0..31) of two 16-byte registers, l known at compile time after unrolling
IFR_DEV uint32_t byte32(const uint4 &a, const uint4 &b, int l) {
    const uint32_t w = l < 16 ? pick4(a, (uint32_t)(l >> 2)) : pick4(b, (uint32_t)((l - 16) >> 2));
    return (w >> (8 * (l & 3))) & 0xFFu;
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
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(q0, q1, l);
            const float q = (float)(hs ? (b >> 4) : (b & 15u));
            h[l] = (_Float16)(d1 * q - mm);
        }
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
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(q0, q1, l);
            const uint32_t q = (hs ? (b >> 4) : (b & 15u)) + (((byte32(e0, e1, l) >> sh) & 1u) ? 16u : 0u);
            h[l] = (_Float16)(d1 * (float)q - mm);
        }
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
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t qlb = byte32(l0, l1, l);
            const uint32_t nib = k < 2 ? (qlb & 15u) : (qlb >> 4);
            const uint32_t hb = (byte32(h0, h1, l) >> (2 * k)) & 3u;
            const int q = (int)(nib | (hb << 4)) - 32;
            h[l] = (_Float16)(d * (l < 16 ? s_lo : s_hi) * (float)q);
        }
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
#pragma unroll
        for (int l = 0; l < 32; l++) h[l] = (_Float16)(d * (float)(int)(int8_t)byte32(q0, q1, l));
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
#pragma unroll
        for (int l = 0; l < 32; l++) h[l] = (_Float16)__uint_as_float(pick4(v[l >> 2], (uint32_t)(l & 3)));
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
#pragma unroll
        for (int l = 0; l < 32; l++) h[l] = (_Float16)((float)(int)(int8_t)byte32(q0, q1, l) * d);
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
#pragma unroll
        for (int l = 0; l < 32; l++) {
            const uint32_t b = byte32(blk.qs, blk.qs, l & 15);
            uint32_t q = l < 16 ? (b & 15u) : (b >> 4);
            if constexpr (Blk32<FMT>::FIVE) q |= ((blk.qh >> l) & 1u) << 4;
            float y;
            if constexpr (Blk32<FMT>::AFF) y = (float)q * d + m;
            else y = (float)((int)q - (int)Blk32<FMT>::H) * d;
            h[l] = (_Float16)y;
        }
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

template <int FMT, int EPI>
__device__ void gemm_f16_body(const PfGemmArgs &a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[PF_BM][PF_LDS];
    __shared__ __attribute__((aligned(16))) _Float16 ws[PF_BN][PF_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * PF_BM, n0 = blockIdx.x * PF_BN;

    // global -> register staging: thread t owns tile row t/2, halves [32*(t%2), +32)
    const uint32_t r = (uint32_t)tid >> 1, hseg = (uint32_t)tid & 1u;
    const bool xrow_ok = m0 + r < a.M, wrow_ok = n0 + r < a.N;
    const _Float16 *xrow = (const _Float16 *)a.x + (size_t)min(m0 + r, a.M - 1) * a.ldx;
    const uint8_t *wrow = a.w + (size_t)min(n0 + r, a.N - 1) * a.row_bytes;
    uint4 xv[4];
    PfTile<FMT> wt;
    auto gload = [&](uint32_t k0) {
        const uint4 *xp = (const uint4 *)(xrow + k0 + 32 * hseg);
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = xrow_ok ? xp[i] : make_uint4(0, 0, 0, 0);
        wt.load(wrow, k0, hseg);
    };
    // this thread's 32 weights into LDS as f16 (a row past N as zeros)
    auto lstore = [&](uint32_t k0) {
        _Float16 h[32];
        wt.deq(k0, hseg, h);
#pragma unroll
        for (int i = 0; i < 32; i++) h[i] = wrow_ok ? h[i] : (_Float16)0.0f;
        uint4 *wd = (uint4 *)&ws[r][32 * hseg];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint4 u;
            __builtin_memcpy(&u, &h[8 * i], 16);
            wd[i] = u;
        }
        uint4 *xd = (uint4 *)&xs[r][32 * hseg];
#pragma unroll
        for (int i = 0; i < 4; i++) xd[i] = xv[i];
    };

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const uint32_t wm = 64 * (uint32_t)(wave >> 1), wn = 64 * (uint32_t)(wave & 1);
    const uint32_t li = (uint32_t)lane & 31u, lk = 8 * ((uint32_t)lane >> 5);
    gload(0);
    for (uint32_t k0 = 0; k0 < a.K; k0 += PF_BK) {
        __syncthreads(); // the previous step's operand reads are done
        lstore(k0);
        if (k0 + PF_BK < a.K) gload(k0 + PF_BK);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < PF_BK; kk += 16) {
            half8v av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; i++) av[i] = *(const half8v *)&xs[wm + 32 * i + li][kk + lk];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = *(const half8v *)&ws[wn + 32 * j + li][kk + lk];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    }
    // D[row][col]: col = lane % 32, row = 8*(e/4) + 4*(lane/32) + e%4
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t n = n0 + wn + 32 * j + li;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                if (m < a.M && n < a.N) {
                    float *yp = a.y + (size_t)m * a.ldy + n;
                    if constexpr (EPI == 1)
                        *yp += acc[i][j][e];
                    else
                        *yp = acc[i][j][e];
                }
            }
        }
}

// W -> f16 [N][K] with the GEMM tiles' dequant arithmetic (so the f16
// weights are the ones the fused GEMM multiplies): thread t takes row
// t / (K/32), elements [k0 + 32 hs, +32) of it (k0 a multiple of 64).
template <int FMT>
__device__ void pf_deq_f16_body(const PfDeqArgs &a) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t segs = a.K / 32;
    const uint32_t r = t / segs, sg = t % segs;
    if (r >= a.N) return;
    const uint32_t k0 = (sg >> 1) * 64, hs = sg & 1u;
    PfTile<FMT> wt;
    wt.load(a.w + (size_t)r * a.row_bytes, k0, hs);
    _Float16 h[32];
    wt.deq(k0, hs, h);
    uint4 *dst = (uint4 *)(a.out + (size_t)r * a.K + k0 + 32 * hs);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint4 u;
        __builtin_memcpy(&u, &h[8 * i], 16);
        dst[i] = u;
    }
}

// ------------------------------------------------------------ pointwise --

// X[m] = dequant(table)[tok[p0 + m]]
IFR_DEV void pf_embed_body(const PfArgs &a) {
    float *xo = (float *)a.x;
    const uint32_t m = blockIdx.x;
    const uint32_t tok = a.tokens[a.p0 + m];
    const uint8_t *row = a.table + (size_t)tok * a.row_bytes;
    for (uint32_t i = threadIdx.x; i < a.hidden; i += blockDim.x)
        xo[(size_t)m * a.hidden + i] = deq_elem(a.fmt, row, i);
}

// xh[m] = f16((x[m] * (1/sqrt(mean(x[m]^2) + eps))) * gamma), rms_norm.rs:81-121
IFR_DEV void pf_rmsnorm_f16_body(const PfArgs &a) {
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, n = a.hidden;
    const float *x = (const float *)a.x + (size_t)m * n;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) t += red[w];
    const float rs = 1.0f / sqrtf(t / (float)n + a.eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
        ((_Float16 *)a.xh)[(size_t)m * a.ldh + i] = (_Float16)((x[i] * rs) * a.gamma[i]);
}

// Token m (position p0 + m) of qkv [M][q_dim + 2 kv_dim]: RoPE on q (in
// place) and k, then k and v to the cache rows (rope.rs:51-92 with the
// state's theta table).
IFR_DEV void pf_rope_kv_body(const PfArgs &a) {
    const uint32_t m = blockIdx.x, pos = a.p0 + m, hs = a.head_size;
    float *row = (float *)a.qkv + (size_t)m * a.ld_qkv;
    const uint32_t qd = a.q_dim, kd = a.kv_dim;
    // each thread owns whole rotation pairs of q | k: pair i of a vector
    // rotates (e0, e1) = (2i, 2i+1), or NeoX (rope.rs:97-141): within head
    // h = 2i / hs, (h hs + j, h hs + j + hs/2) with j = i mod hs/2; the
    // biases (Qwen2) are added first, as transformer.rs:434-445 orders it
    for (uint32_t i = threadIdx.x; i < (qd + kd) / 2; i += blockDim.x) {
        const bool is_q = 2 * i < qd;
        const uint32_t pi = is_q ? i : i - qd / 2; // pair index within its vector
        uint32_t e0, e1;
        if (a.neox) {
            const uint32_t h = (2 * pi) / hs, j = pi % (hs / 2);
            e0 = h * hs + j;
            e1 = e0 + hs / 2;
        } else {
            e0 = 2 * pi;
            e1 = e0 + 1;
        }
        const uint32_t base = is_q ? 0 : qd;
        float x0 = row[base + e0], x1 = row[base + e1];
        const float *bias = is_q ? a.q_bias : a.k_bias;
        if (bias) {
            x0 = x0 + bias[e0];
            x1 = x1 + bias[e1];
        }
        // theta index j (the table holds base^(-2j/hs)); rope_pair takes 2j
        const uint32_t tj = a.neox ? 2 * (pi % (hs / 2)) : e0;
        rope_pair(x0, x1, tj, hs, pos, a.rope_tab);
        if (is_q) {
            row[e0] = x0;
            row[e1] = x1;
        } else {
            const size_t off = (size_t)pos * kd;
            if (a.kv_f16) {
                ((uint16_t *)a.k_cache)[off + e0] = f32_to_f16(x0);
                ((uint16_t *)a.k_cache)[off + e1] = f32_to_f16(x1);
            } else {
                ((float *)a.k_cache)[off + e0] = x0;
                ((float *)a.k_cache)[off + e1] = x1;
            }
        }
    }
    for (uint32_t i = threadIdx.x; i < kd; i += blockDim.x) {
        float v = row[qd + kd + i];
        if (a.v_bias) v = v + a.v_bias[i];
        const size_t off = (size_t)pos * kd + i;
        if (a.kv_f16)
            ((uint16_t *)a.v_cache)[off] = f32_to_f16(v);
        else
            ((float *)a.v_cache)[off] = v;
    }
}

// h[m][j] = f16(u * (g / (1 + exp(-g)))), g = gu[m][j], u = gu[m][F + j] (silu.rs:24-53)
IFR_DEV void pf_silu_body(const PfArgs &a) {
    const uint32_t m = blockIdx.y, F = a.ffn;
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= F) return;
    const float *gu = (const float *)a.gu;
    const float g = gu[(size_t)m * 2 * F + j], u = gu[(size_t)m * 2 * F + F + j];
    ((_Float16 *)a.xh)[(size_t)m * a.ldh + j] = (_Float16)(u * (g / (1.0f + expf(-g))));
}

// ------------------------------------------------------------ attention --
// Causal attention of the chunk's queries (positions p0 .. p0+M-1) over the
// cache rows [0, position], on the matrix cores (flash attention).
// Workgroup (h, qt): KV head h, its G = kv_mul query heads and QT = 64 / G
// queries, i.e. QT * G <= 64 rows r = qi * G + j (rows past QT * G hold
// nothing).  Head dims run to HSP (the head size rounded up to 64 or 128;
// dims past the head size are zeros).  Per key tile of 64 cache rows:
//   S = Q K^T     (f16 operands from LDS, 4 waves x one 32x32 MFMA tile)
//   running softmax per row in base-2 units (q pre-scaled by
//   log2(e)/sqrt(hs)); P = 2^(S - m) as f16
//   O = alpha O + P V   (4 waves x 32 rows x HSP/2 dims)
// and out = O / l is written as f16 for the O GEMM.
constexpr int PF_ROWS = 64, PF_KT = 64;

template <int HSP, bool F16>
__device__ void pf_attn_body(const PfArgs &a) {
    constexpr int R = PF_ROWS, NT = 256;
    constexpr int HSL = HSP + 8, KTP = PF_KT + 8; // padded LDS rows (halves)
    constexpr int DT = HSP / 64;                  // 32x32 O tiles per wave along the dims
    __shared__ __attribute__((aligned(16))) _Float16 qh[R][HSL];
    __shared__ __attribute__((aligned(16))) _Float16 kh[PF_KT][HSL];
    __shared__ __attribute__((aligned(16))) _Float16 vt[HSP][KTP];
    __shared__ __attribute__((aligned(16))) _Float16 ph[R][KTP];
    __shared__ float sf[R][PF_KT + 1];
    __shared__ float alpha_s[R], l_s[R];
    __shared__ int32_t qpos_s[R]; // position of row r's query, -1 for an unused row
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t G = a.kv_mul, hs = a.head_size, QT = (uint32_t)PF_ROWS / G;
    const uint32_t kvh = blockIdx.x, qt0 = blockIdx.y * QT;
    const uint32_t nq = min(QT, a.M - qt0);
    const float qscale = 1.44269504088896341f / sqrtf((float)hs);
    const float *qbase = (const float *)a.qkv;
    for (uint32_t i = tid; i < (uint32_t)R * HSP; i += NT) {
        const uint32_t rr = i / HSP, d = i % HSP, qi = rr / G, j = rr % G;
        const float v = (qi < nq && d < hs) ? qbase[(size_t)(qt0 + qi) * a.ld_qkv + (kvh * G + j) * hs + d] : 0.0f;
        qh[rr][d] = (_Float16)(v * qscale);
    }
    if (tid < R) {
        const uint32_t qi = (uint32_t)tid / G;
        qpos_s[tid] = qi < nq ? (int32_t)(a.p0 + qt0 + qi) : -1;
    }
    // softmax ownership: row sr, keys [16 * sq, 16 * sq + 16)
    const uint32_t sr = (uint32_t)tid >> 2, sq = (uint32_t)tid & 3u;
    float m_run = -INFINITY, l_run = 0.0f;
    // MFMA roles
    const uint32_t li = (uint32_t)lane & 31u, lk = 8 * ((uint32_t)lane >> 5);
    const uint32_t srow = 32 * (uint32_t)(wave >> 1), skey = 32 * (uint32_t)(wave & 1); // S tile of this wave
    const uint32_t orow = 32 * (uint32_t)(wave >> 1), odim = (HSP / 2) * (uint32_t)(wave & 1); // O block
    float16v oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[t][e] = 0.0f;

    const uint32_t last = a.p0 + qt0 + nq - 1; // largest query position of the tile
    for (uint32_t k0 = 0; k0 <= last; k0 += PF_KT) {
        __syncthreads(); // previous tile's operands are consumed
        for (uint32_t i = tid; i < (uint32_t)PF_KT * HSP; i += NT) {
            const uint32_t kr = i / HSP, d = i % HSP, kp = k0 + kr;
            _Float16 kk = (_Float16)0.0f, vv = (_Float16)0.0f;
            if (kp <= last && d < hs) {
                const size_t off = (size_t)kp * a.kv_dim + (size_t)kvh * hs + d;
                if constexpr (F16) {
                    const uint16_t kb = ((const uint16_t *)a.k_cache)[off], vb = ((const uint16_t *)a.v_cache)[off];
                    __builtin_memcpy(&kk, &kb, 2);
                    __builtin_memcpy(&vv, &vb, 2);
                } else {
                    kk = (_Float16)((const float *)a.k_cache)[off];
                    vv = (_Float16)((const float *)a.v_cache)[off];
                }
            }
            kh[kr][d] = kk;
            vt[d][kr] = vv;
        }
        __syncthreads();
        // S tile: rows srow.., keys skey..
        {
            float16v sacc;
#pragma unroll
            for (int e = 0; e < 16; e++) sacc[e] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < HSP; kk += 16) {
                const half8v av = *(const half8v *)&qh[srow + li][kk + lk];
                const half8v bv = *(const half8v *)&kh[skey + li][kk + lk];
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, sacc, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = srow + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                const uint32_t key = skey + li;
                sf[row][key] = ((int32_t)(k0 + key) <= qpos_s[row]) ? sacc[e] : -INFINITY;
            }
        }
        __syncthreads();
        // running softmax: 4 threads per row, 16 keys each
        {
            float mt = -INFINITY;
#pragma unroll
            for (int k = 0; k < 16; k++) mt = fmaxf(mt, sf[sr][16 * sq + k]);
            mt = fmaxf(mt, __shfl_xor(mt, 1, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 2, 64));
            const float mn = fmaxf(m_run, mt);
            // a row with no key yet (mn = -inf) keeps alpha 1 and p 0
            const float al = (mn == -INFINITY) ? 1.0f : exp2f(m_run - mn);
            float ls = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float p = (mn == -INFINITY) ? 0.0f : exp2f(sf[sr][16 * sq + k] - mn);
                ls += p;
                ph[sr][16 * sq + k] = (_Float16)p;
            }
            ls += __shfl_xor(ls, 1, 64);
            ls += __shfl_xor(ls, 2, 64);
            l_run = l_run * al + ls;
            m_run = mn;
            if (sq == 0) alpha_s[sr] = al;
        }
        __syncthreads();
        // O = alpha O + P V
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = orow + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                oacc[t][e] *= alpha_s[row];
            }
#pragma unroll
        for (int kk = 0; kk < PF_KT; kk += 16) {
            const half8v av = *(const half8v *)&ph[orow + li][kk + lk];
#pragma unroll
            for (int t = 0; t < DT; t++) {
                const half8v bv = *(const half8v *)&vt[odim + 32 * t + li][kk + lk];
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, oacc[t], 0, 0, 0);
            }
        }
    }
    if (sq == 0) l_s[sr] = l_run;
    __syncthreads();
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t row = orow + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
            const uint32_t qi = row / G, dim = odim + 32 * t + li;
            if (qpos_s[row] >= 0 && dim < hs)
                ((_Float16 *)a.xh)[(size_t)(qt0 + qi) * a.ldh + (kvh * G + row % G) * hs + dim] =
                    (_Float16)(oacc[t][e] / l_s[row]);
        }
}

} // namespace ifr

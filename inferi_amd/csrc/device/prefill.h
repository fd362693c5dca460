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
#include "pf_gemm.h"
#include "pf_tiles.h"

namespace ifr {


// ------------------------------------------------------------------ GEMM --
// The small-tile form of the prefill GEMM (device/pf_gemm.h has the
// 256 x 256 form and the argument conventions): Y[m][n] = sum_k X[m][k] *
// deq(W)[n][k] with the same epilogues (EPI: PG_STORE, PG_ADD, PG_SWIGLU)
// and stacked matrices, for products with too few 256 x 256 tiles to fill
// the chip.  Tile 128 (m) x 128 (n), K steps of 64; four waves, each a
// 64 x 64 quadrant as 2 x 2 MFMA 32x32x16 tiles.  The next K step's global
// loads are issued before the current step's MFMAs.  Each output element
// sums its k in the same order as the large form (steps of 64, products of
// 16), so both forms give the same results bit for bit.
constexpr int PF_BM = 128, PF_BN = 128, PF_BK = 64;
constexpr int PF_LDS = PF_BK + 8; // halves per LDS row: 144 B, so the 32 rows an MFMA operand read touches spread over the banks

template <int FMT, int EPI>
__device__ void gemm_f16_body(const PfGemmArgs &a) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[PF_BM][PF_LDS];
    __shared__ __attribute__((aligned(16))) _Float16 ws[PF_BN][PF_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t m0 = blockIdx.y * PF_BM, n0 = blockIdx.x * PF_BN;

    // global -> register staging: thread t owns tile row t/2, halves
    // [32*(t%2), +32); rows past M or N repeat the last row (their outputs
    // are not stored)
    const uint32_t r = (uint32_t)tid >> 1, hseg = (uint32_t)tid & 1u;
    const _Float16 *xrow = (const _Float16 *)a.x + (size_t)min(m0 + r, a.M - 1) * a.ldx;
    const uint8_t *wrow;
    if constexpr (EPI == PG_SWIGLU) {
        // wave column c = r / 64 holds FFN rows j in [n0 / 2 + 32 c, +32):
        // tile rows 64 c + i are gate row j, 64 c + 32 + i up row j
        const uint32_t j = min(n0 / 2 + 32 * (r >> 6) + (r & 31u), a.n1 - 1);
        wrow = ((r >> 5) & 1u ? a.w1 : a.w0) + (size_t)j * a.row_bytes;
    } else {
        const uint32_t n = min(n0 + r, a.N - 1);
        const uint8_t *base = n < a.n1 ? a.w0 : n < a.n2 ? a.w1 : a.w2;
        const uint32_t nr = n < a.n1 ? n : n < a.n2 ? n - a.n1 : n - a.n2;
        wrow = base + (size_t)nr * a.row_bytes;
    }
    u32x4_a16 x0, x1, x2, x3; // the next K step's X segment
    PfTile<FMT> wt;
    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    const uint32_t wm = 64 * (uint32_t)(wave >> 1), wn = 64 * (uint32_t)(wave & 1);
    const uint32_t li = (uint32_t)lane & 31u, lk = 8 * ((uint32_t)lane >> 5);
    const u32x4_a16 *xp = (const u32x4_a16 *)(xrow + 32 * hseg);
    x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
    wt.load(wrow, 0, hseg);
    for (uint32_t k0 = 0; k0 < a.K; k0 += PF_BK) {
        __syncthreads(); // the previous step's operand reads are done
        {
            // this thread's 32 weights into LDS as f16, then its X segment
            _Float16 h[32];
            wt.deq(k0, hseg, h);
            uint4 *wd = (uint4 *)&ws[r][32 * hseg];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint4 u;
                __builtin_memcpy(&u, &h[8 * i], 16);
                wd[i] = u;
            }
            u32x4_a16 *xd = (u32x4_a16 *)&xs[r][32 * hseg];
            xd[0] = x0, xd[1] = x1, xd[2] = x2, xd[3] = x3;
        }
        if (k0 + PF_BK < a.K) {
            const u32x4_a16 *xn = xp + (k0 + PF_BK) / 8;
            x0 = xn[0], x1 = xn[1], x2 = xn[2], x3 = xn[3];
            wt.load(wrow, k0 + PF_BK, hseg);
        }
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
    if constexpr (EPI == PG_SWIGLU) {
        const uint32_t jn = n0 / 2 + wn / 2 + li;
        if (jn >= a.n1) return;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                if (m < a.M) {
                    const float g = acc[i][0][e], u = acc[i][1][e];
                    ((_Float16 *)a.y)[(size_t)m * a.ldy + jn] = f16_of(u * silu_fast(g));
                }
            }
    } else {
        // eight values at a time; their residual loads (ADD) go out together
        // from rows clamped below M, so a lane waits once per eight values,
        // not once per value behind its bounds branch (eight, not sixteen:
        // the form keeps its three waves per SIMD)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t n = n0 + wn + 32 * j + li;
                if (n >= a.N) continue;
#pragma unroll
                for (int h = 0; h < 16; h += 8) {
                    float old[8];
                    if constexpr (EPI == PG_ADD) {
#pragma unroll
                        for (int e = h; e < h + 8; e++) {
                            const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                            old[e - h] = ((const float *)a.y)[(size_t)min(m, a.M - 1) * a.ldy + n];
                        }
                    }
#pragma unroll
                    for (int e = h; e < h + 8; e++) {
                        const uint32_t m = m0 + wm + 32 * i + 8 * (e / 4) + 4 * ((uint32_t)lane >> 5) + (e % 4);
                        if (m < a.M) {
                            float *yp = (float *)a.y + (size_t)m * a.ldy + n;
                            if constexpr (EPI == PG_ADD)
                                *yp = old[e - h] + acc[i][j][e];
                            else
                                *yp = acc[i][j][e];
                        }
                    }
                }
            }
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
// Rows of a multiple of 4 elements (every model here) go 16 bytes per lane;
// other widths element by element.
IFR_DEV void pf_rmsnorm_f16_body(const PfArgs &a) {
    __shared__ float red[16];
    const uint32_t m = blockIdx.x, n = a.hidden;
    const float *x = (const float *)a.x + (size_t)m * n;
    _Float16 *xh = (_Float16 *)a.xh + (size_t)m * a.ldh;
    const bool vec = (n & 3u) == 0 && (a.ldh & 3u) == 0 && ((uintptr_t)a.gamma & 15u) == 0;
    float ss = 0.0f;
    // vector path: the thread's first RC float4 of x and of gamma are loaded
    // together up front (indices clamped into the row; a clamped one adds
    // nothing and is not stored) and kept for the second pass, so the row
    // costs one memory round trip, not one per float4 and pass
    constexpr uint32_t RC = 4;
    float4 xv[RC], gv[RC];
    const uint32_t step = 4 * blockDim.x;
    if (vec) {
#pragma unroll
        for (uint32_t c = 0; c < RC; c++) {
            const uint32_t i = min(4 * threadIdx.x + step * c, n - 4);
            xv[c] = *(const float4 *)(x + i);
            gv[c] = *(const float4 *)(a.gamma + i);
        }
#pragma unroll
        for (uint32_t c = 0; c < RC; c++) {
            const float4 v = xv[c];
            if (4 * threadIdx.x + step * c < n) {
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
        }
        for (uint32_t i = 4 * threadIdx.x + step * RC; i < n; i += step) {
            const float4 v = *(const float4 *)(x + i);
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
    } else {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) t += red[w];
    const float rs = 1.0f / sqrtf(t / (float)n + a.eps);
    if (vec) {
#pragma unroll
        for (uint32_t c = 0; c < RC; c++) {
            const uint32_t i = 4 * threadIdx.x + step * c;
            if (i < n) {
                const float4 v = xv[c], g = gv[c];
                uint2 u;
                u.x = pack_f16x2((v.x * rs) * g.x, (v.y * rs) * g.y);
                u.y = pack_f16x2((v.z * rs) * g.z, (v.w * rs) * g.w);
                *(uint2 *)(xh + i) = u;
            }
        }
        for (uint32_t i = 4 * threadIdx.x + step * RC; i < n; i += step) {
            const float4 v = *(const float4 *)(x + i), g = *(const float4 *)(a.gamma + i);
            uint2 u;
            u.x = pack_f16x2((v.x * rs) * g.x, (v.y * rs) * g.y);
            u.y = pack_f16x2((v.z * rs) * g.z, (v.w * rs) * g.w);
            *(uint2 *)(xh + i) = u;
        }
    } else {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) xh[i] = f16_of((x[i] * rs) * a.gamma[i]);
    }
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
        // theta index j (the table holds base^(-2j/hs)): the pass's (cos,
        // sin) of pos * theta_j
        const uint32_t tj = a.neox ? pi % (hs / 2) : (e0 % hs) >> 1;
        const float *cs = a.rope_cs + ((size_t)m * (hs / 2) + tj) * 2;
        rope_rotate(x0, x1, cs[0], cs[1]);
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

// The pass's RoPE angles: rope_cs[m][j] = (cos, sin) of (p0 + m) * theta_j
// for j < head_size / 2 (sincosf, as the decode step's rope_pair), shared by
// every head and layer of the pass (pf_rope_kv_k and the Q/K/V product's
// fused epilogue read it).
IFR_DEV void pf_rope_tab_body(const PfArgs &a) {
    const uint32_t m = blockIdx.x, j = threadIdx.x, hh = a.head_size / 2;
    if (j >= hh) return;
    const float ang = (float)(a.p0 + m) * a.rope_tab[j];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    a.rope_cs[((size_t)m * hh + j) * 2] = cs;
    a.rope_cs[((size_t)m * hh + j) * 2 + 1] = sn;
}

// h[m][j] = f16(u * silu(g)), g = gu[m][j], u = gu[m][F + j] (silu.rs:
// 24-53), for layers whose gate and up matrices differ in type (the others
// take the GEMM's SwiGLU epilogue, the same arithmetic: silu_fast, the
// hardware exp2 and reciprocal, as the decode step's gate/up epilogue)
IFR_DEV void pf_silu_body(const PfArgs &a) {
    const uint32_t m = blockIdx.y, F = a.ffn;
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= F) return;
    const float *gu = (const float *)a.gu;
    const float g = gu[(size_t)m * 2 * F + j], u = gu[(size_t)m * 2 * F + F + j];
    ((_Float16 *)a.h)[(size_t)m * F + j] = f16_of(u * silu_fast(g));
}

// ------------------------------------------------------------ attention --
// Causal attention of the chunk's queries (positions p0 .. p0+M-1) over the
// cache rows [0, position], on the matrix cores (flash attention).
// Workgroup (h, t): KV head h and a tile of QT = 128 / G queries, i.e. the
// 128 rows r = qi * G + j (query qi, query head j of the G = kv_mul heads of
// KV head h; rows past QT * G hold nothing).  Wave w owns rows 32w .. 32w+31,
// one per lane pair (lanes l and l + 32 share row l % 32).  Head dims run to
// HSP (the head size rounded up to 64 or 128; the padding is zeros).  Per
// tile of 64 cache rows (K and V^T staged in LDS, double-buffered, loaded
// from memory one tile ahead):
//   S^T = K Q^T      (Q^T, scaled by log2(e)/sqrt(hs), stays in registers as
//                     the B operand; 2 x HSP/16 v_mfma_f32_32x32x16_f16)
//   running softmax per row in base-2 units, in registers: each lane holds
//   16 of its row's 32 scores per 32-key block (its half of the keys);
//   P^T (f16) is then the B operand of
//   O^T = V^T P^T    (HSP/32 x 4 MFMAs), the k index of both operands
//                     running over the keys in the order the score
//                     accumulator holds them (4 keys of this lane half, 4 of
//                     the other, ...), so P^T needs no shuffle;
// and out = O / l is written as f16 for the O GEMM.  The last query tiles,
// which see the most keys, are dispatched first.
constexpr int PFA_WAVES = 4, PFA_ROWS = 32 * PFA_WAVES, PFA_KT = 64; // keys per tile
constexpr int PFA_KB = PFA_KT / 32;                                      // 32-key blocks per tile
// A row's softmax reference maximum moves only when a tile's maximum passes
// it by more than this (base-2 units): the weights 2^(s - m) then stay below
// 2^PFA_LAZY (f16 holds them at the same relative precision as weights
// below 1), and O and l, both taken against the same reference, keep their
// ratio.  The rescale of O (its accumulators live in AGPRs: a read, a
// multiply and a write per value) is skipped for a wave none of whose rows
// moved.
constexpr float PFA_LAZY = 8.0f;

// x with its bits 2 and 3 exchanged
IFR_DEV uint32_t swap23(uint32_t x) {
    const uint32_t t = ((x >> 2) ^ (x >> 3)) & 1u;
    return x ^ (t << 2) ^ (t << 3);
}

template <int HSP, bool F16>
__device__ void pf_attn_body(const PfArgs &a) {
    constexpr int KC = HSP / 16;          // k-chunks of the scores (head dims)
    constexpr int DT = HSP / 32;          // O^T tiles along the head dims
    constexpr int KP = HSP + 8;           // K tile row pitch (halves)
    // V^T row pitch (halves): 16-byte rows for the one-read operands, and 36
    // dwords, so the 16 rows li of a 16-byte read pass start on 16 distinct
    // 4-bank groups
    constexpr int VP = PFA_KT + 8;
    constexpr int CPK = HSP / 8;          // 8-dim chunks per key row
    constexpr int R = PFA_KT * CPK / 256; // keys each thread stages per tile (chunk dc of each)
    static_assert(R == 2 || R == 4, "head sizes padded to 64 or 128");
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][PFA_KT][KP];
    __shared__ __attribute__((aligned(16))) _Float16 vts[2][HSP][VP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t G = a.kv_mul, hs = a.head_size, QT = (uint32_t)PFA_ROWS / G;
    const uint32_t ntiles = (a.M + QT - 1) / QT;
    const uint32_t kvh = blockIdx.x, q0 = (ntiles - 1 - blockIdx.y) * QT;
    const uint32_t nq = min(QT, a.M - q0);
    const uint32_t li = (uint32_t)lane & 31u, hl = (uint32_t)lane >> 5;
    const uint32_t r = (uint32_t)wave * 32 + li, qi = r / G, j = r % G;
    const bool row_ok = qi < nq;
    const int32_t qpos = row_ok ? (int32_t)(a.p0 + q0 + qi) : -1;
    const uint32_t qlast = a.p0 + q0 + nq - 1;  // largest query position of the tile
    const uint32_t ntk = qlast / PFA_KT + 1;    // key tiles

    // This thread stages keys R gk .. R gk + R - 1 of the tile, dims
    // 8 dc .. +8 of each: dc = lane % 4 + 4 x (wave % (CPK / 4)), gk = lane / 4
    // + 16 x (wave / (CPK / 4)); one load instruction reads 64 contiguous bytes
    // (four chunks) of 16 key rows.  K goes to LDS as it is (ks[key][dim]);
    // V transposed (vts[dim][key']) with key' = key with its bits 2 and 3
    // swapped: the 8 keys that lane half hl of an O^T operand needs (4 hl ..
    // 4 hl + 3 and 8 + 4 hl .. of a 16-key chunk, the score accumulator's
    // order) then sit in one 16-byte run at 8 hl, and this thread's R keys
    // stay adjacent, one 4- or 8-byte store per dim.  The loads are
    // unconditional (a load behind a branch is drained at the branch's join,
    // which would make the next tile's loads wait before this tile's
    // products): a key past the tile's last query reads that query's row
    // instead, a finite cache row whose weight the causal mask makes exactly
    // 0, and a chunk past the head size reads the last chunk, which meets Q's
    // zero padding in the scores and feeds only output dims that are never
    // written.
    const uint32_t dc = ((uint32_t)lane & 3u) + 4u * ((uint32_t)wave % (CPK / 4));
    const uint32_t gk = ((uint32_t)lane >> 2) + 16u * ((uint32_t)wave / (CPK / 4));
    // V^T column of this thread's first key; rows with bit 4 set (dims
    // 16-31 of each 32) hold their 32-key blocks' two 16-key halves
    // exchanged, which puts the four rows 8 apart that one 16-lane pass of
    // the stores writes on distinct banks (the reads apply the same exchange)
    const uint32_t vcol = swap23(R * gk) ^ (16u * ((dc >> 1) & 1u));
    uint4 kraw[R][F16 ? 1 : 2], vraw[R][F16 ? 1 : 2];
    auto gload = [&](uint32_t t) {
        const size_t col = (size_t)kvh * hs + min(dc, hs / 8 - 1) * 8;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint32_t kp = t * PFA_KT + R * gk + (uint32_t)i;
            const size_t off = (size_t)min(kp, qlast) * a.kv_dim + col;
#pragma unroll
            for (int h = 0; h < (F16 ? 1 : 2); h++) {
                if (F16) {
                    kraw[i][h] = *(const uint4 *)((const uint16_t *)a.k_cache + off);
                    vraw[i][h] = *(const uint4 *)((const uint16_t *)a.v_cache + off);
                } else {
                    kraw[i][h] = *(const uint4 *)((const float *)a.k_cache + off + 4 * h);
                    vraw[i][h] = *(const uint4 *)((const float *)a.v_cache + off + 4 * h);
                }
            }
        }
    };
    // 16-bit element e of a staged 8-element chunk, as f16 bits
    auto half_of = [&](const uint4 (&raw)[F16 ? 1 : 2], int e) -> uint32_t {
        if constexpr (F16) {
            const uint32_t w = e < 2 ? raw[0].x : e < 4 ? raw[0].y : e < 6 ? raw[0].z : raw[0].w;
            return (e & 1) ? (w >> 16) : (w & 0xFFFFu);
        } else {
            const uint4 &q = raw[e >> 2];
            const uint32_t w = (e & 3) == 0 ? q.x : (e & 3) == 1 ? q.y : (e & 3) == 2 ? q.z : q.w;
            return (uint32_t)__builtin_bit_cast(uint16_t, f16_of(__uint_as_float(w)));
        }
    };
    auto lstore = [&](uint32_t b) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            uint4 u;
            if constexpr (F16) {
                u = kraw[i][0];
            } else {
                u.x = half_of(kraw[i], 0) | half_of(kraw[i], 1) << 16;
                u.y = half_of(kraw[i], 2) | half_of(kraw[i], 3) << 16;
                u.z = half_of(kraw[i], 4) | half_of(kraw[i], 5) << 16;
                u.w = half_of(kraw[i], 6) | half_of(kraw[i], 7) << 16;
            }
            *(uint4 *)&ks[b][R * gk + (uint32_t)i][8 * dc] = u;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if constexpr (R == 4) {
                uint2 v;
                v.x = half_of(vraw[0], e) | half_of(vraw[1], e) << 16;
                v.y = half_of(vraw[2], e) | half_of(vraw[3], e) << 16;
                *(uint2 *)&vts[b][8 * dc + (uint32_t)e][vcol] = v;
            } else {
                *(uint32_t *)&vts[b][8 * dc + (uint32_t)e][vcol] = half_of(vraw[0], e) | half_of(vraw[1], e) << 16;
            }
        }
    };

    // Q^T operand: dims 16c + 8 hl .. +8 of this lane's row
    const float qscale = 1.44269504088896341f / sqrtf((float)hs);
    half8v qb[KC];
    {
        const float *qrow = (const float *)a.qkv + (size_t)(q0 + (row_ok ? qi : 0)) * a.ld_qkv + (size_t)(kvh * G + j) * hs;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const uint32_t d = 16 * (uint32_t)c + 8 * hl;
            float4 x0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), x1 = x0;
            if (row_ok && d < hs) {
                x0 = *(const float4 *)(qrow + d);
                x1 = *(const float4 *)(qrow + d + 4);
            }
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) qb[c][e] = (_Float16)(xv[e] * qscale);
        }
    }

    float16v o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[t][e] = 0.0f;
    float m_run = ATTN_M0, l_run = 0.0f;
    // (uniform) every row of the wave holds a query of the chunk, and the
    // wave's smallest query position: a key tile at or below it needs no
    // causal mask
    const bool wave_rows_ok = ((uint32_t)wave * 32 + 31) / G < nq;
    const int32_t wave_qmin = (int32_t)(a.p0 + q0 + ((uint32_t)wave * 32) / G);

    gload(0);
    lstore(0);
    __syncthreads();
    for (uint32_t t = 0; t < ntk; t++) {
        const uint32_t b = t & 1u, k0 = t * PFA_KT;
        // the next tile's loads (the last tile reloads itself, unused), not
        // behind a branch
        gload(min(t + 1, ntk - 1));
        // S^T for keys k0 + 32 u + (8 (e / 4) + 4 hl + e % 4), this lane's row
        float16v sacc[PFA_KB];
#pragma unroll
        for (int u = 0; u < PFA_KB; u++) {
#pragma unroll
            for (int e = 0; e < 16; e++) sacc[u][e] = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; c++) {
                const half8v av = *(const half8v *)&ks[b][32 * u + li][16 * c + 8 * hl];
                sacc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qb[c], sacc[u], 0, 0, 0);
            }
        }
        // causal mask (a tile reaching past the wave's first query, or a
        // wave with rows past the chunk) and the running softmax of this
        // lane's row
        if (!wave_rows_ok || (int32_t)(k0 + PFA_KT - 1) > wave_qmin) {
#pragma unroll
            for (int u = 0; u < PFA_KB; u++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int32_t kp = (int32_t)(k0 + 32 * u + 8 * (e / 4) + 4 * hl + (e % 4));
                    sacc[u][e] = kp <= qpos ? sacc[u][e] : -INFINITY;
                }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int u = 0; u < PFA_KB; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) mt = fmaxf(mt, sacc[u][e]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        // the reference maximum moves (and O, l are rescaled) only where a
        // row's tile maximum passes it by more than PFA_LAZY; a row with no
        // valid key yet keeps m_run = ATTN_M0 and every p = 0
        if (__ballot(mt > m_run + PFA_LAZY)) {
            const float mn = fmaxf(m_run, mt);
            const float al = softmax_exp2(m_run - mn);
            l_run *= al;
            m_run = mn;
#pragma unroll
            for (int d = 0; d < DT; d++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[d][e] *= al;
        }
        float ls = 0.0f;
        half8v pb[PFA_KB][2];
#pragma unroll
        for (int u = 0; u < PFA_KB; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float pv = softmax_exp2(sacc[u][e] - m_run);
                ls += pv;
                pb[u][e / 8][e % 8] = (_Float16)pv;
            }
        l_run += ls;
        // O^T += V^T P^T over the tile's 4 chunks of 16 keys
#pragma unroll
        for (int u = 0; u < PFA_KB; u++)
#pragma unroll
            for (int cc = 0; cc < 2; cc++) {
                // V^T columns: key bits 2 and 3 swapped, halves exchanged on rows with bit 4 set
                const uint32_t kb = (32 * u + 16 * cc + 8 * hl) ^ (16u * ((li >> 4) & 1u));
#pragma unroll
                for (int d = 0; d < DT; d++) {
                    const half8v av = *(const half8v *)&vts[b][32 * d + li][kb];
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb[u][cc], o[d], 0, 0, 0);
                }
            }
        if (t + 1 < ntk) lstore(b ^ 1u);
        __syncthreads();
    }
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if (row_ok) {
        _Float16 *orow = (_Float16 *)a.xh + (size_t)(q0 + qi) * a.ldh + (size_t)(kvh * G + j) * hs;
        const float inv = 1.0f / l_tot;
#pragma unroll
        for (int d = 0; d < DT; d++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t dim = 32 * d + 8 * (e / 4) + 4 * hl + (e % 4);
                if (dim < hs) orow[dim] = (_Float16)(o[d][e] * inv);
            }
    }
}

} // namespace ifr

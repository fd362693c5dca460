// Flash-decoding attention for one token over a [seq][kv_dim] KV cache.
//
// Grid (n_kv_heads, n_splits).  Workgroup (h, s) serves the G = kv_mul query
// heads that share KV head h (grouped-query attention reads each K/V row once
// for all of them, where the reference's fused_attention reads it once per
// query head: fused_attention.rs:66-241) over the s-th chunk of the positions
// [0, pos].  The chunk length is ceil((pos+1)/n_splits), computed on the
// device from the device-resident position, so one launch shape serves every
// position (and a captured graph can be replayed).
//
// Per workgroup: scores q.k_t / sqrt(hs) for the chunk into LDS, chunk max m
// and l = sum exp(s - m), o = sum exp(s - m) v_t; the partial (m, l, o) goes
// to global memory.  A second, small kernel (attn_merge_body) combines the
// partials of each query head: out = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.
// The kernel boundary orders the two: merging inside the first kernel would
// need device-scope fences, which on this chip write back and invalidate the
// whole L2 of the XCD for every workgroup.
#pragma once
#include "gemv.h"

namespace ifr {

constexpr int ATTN_THREADS = 256;
constexpr int ATTN_CMAX = 256; // longest chunk a workgroup accepts
constexpr int ATTN_CMIN = 64;  // shortest chunk a split is given (unless T is shorter)
constexpr int ATTN_MERGE_MAX = 256;  // most splits one KV head may have
constexpr int ATTN_UNROLL = 8; // rows per thread loaded before use

template <bool F16>
IFR_DEV void load_kv8(const void *cache, size_t off, float *v) {
    if constexpr (F16) {
        const uint4 u = *(const uint4 *)((const uint16_t *)cache + off);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = f16_to_f32(w[i] & 0xFFFFu);
            v[2 * i + 1] = f16_to_f32(w[i] >> 16);
        }
    } else {
        const float4 a = *(const float4 *)((const float *)cache + off);
        const float4 b = *(const float4 *)((const float *)cache + off + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

template <int TPP>
IFR_DEV float group_sum(float v) {
    if constexpr (TPP == 16) return sum16(v);
    else return sum8(v);
}

template <int HS, int G, bool F16>
__device__ void attn_body(const AttnArgs &a) {
    constexpr int TPP = HS / 8;                 // lanes per position (8 dims each)
    constexpr int PPP = ATTN_THREADS / TPP;     // positions per pass
    constexpr int LPW = 64 / TPP;               // positions per wave
    __shared__ float sc[G][ATTN_CMAX];
    __shared__ float ml[G][2];
    __shared__ float red[4][TPP][8 * G];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kvh = blockIdx.x, s = blockIdx.y, S = a.n_splits;
    const uint32_t T = min(*a.pos + 1, a.seq_cap);
    // chunk: at least ATTN_CMIN positions (short contexts use few splits, so
    // the merge reads few partials); the host sizes n_splits so that the
    // chunk never exceeds ATTN_CMAX, the min keeps LDS in bounds regardless
    const uint32_t C = min(max((T + S - 1) / S, (uint32_t)ATTN_CMIN), (uint32_t)ATTN_CMAX);
    const uint32_t n_act = (T + C - 1) / C;
    const uint32_t t0 = s * C;
    if (t0 >= T) return;
    const uint32_t n = min(C, T - t0);

    const int dc = tid % TPP, pg = tid / TPP;
    const size_t head_off = (size_t)kvh * HS + (size_t)dc * 8;

    // this thread's 8 query dims of every head of the group
    float q[G][8];
#pragma unroll
    for (int j = 0; j < G; j++) {
        const float4 u = *(const float4 *)(a.q + (size_t)(kvh * G + j) * HS + dc * 8);
        const float4 w = *(const float4 *)(a.q + (size_t)(kvh * G + j) * HS + dc * 8 + 4);
        q[j][0] = u.x; q[j][1] = u.y; q[j][2] = u.z; q[j][3] = u.w;
        q[j][4] = w.x; q[j][5] = w.y; q[j][6] = w.z; q[j][7] = w.w;
    }
    const float inv_div = sqrtf((float)HS);

    // ---- scores
    for (uint32_t base = 0; base < n; base += PPP * ATTN_UNROLL) {
        float kv[ATTN_UNROLL][8];
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; u++) {
            const uint32_t tt = base + (uint32_t)(pg + PPP * u);
            if (tt < n) load_kv8<F16>(a.k_cache, (size_t)(t0 + tt) * a.kv_dim + head_off, kv[u]);
        }
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; u++) {
            const uint32_t tt = base + (uint32_t)(pg + PPP * u);
            if (base + PPP * u >= n) break; // uniform across the workgroup
#pragma unroll
            for (int j = 0; j < G; j++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(q[j][e], kv[u][e], d);
                d = group_sum<TPP>(d);
                if (dc == 0 && tt < n) sc[j][tt] = d / inv_div;
            }
        }
    }
    __syncthreads();

    // ---- softmax statistics: head j handled by 256/G consecutive threads
    {
        constexpr int TPH = ATTN_THREADS / G;
        const int j = tid / TPH, r = tid % TPH;
        float m = -INFINITY;
        for (uint32_t t = r; t < n; t += TPH) m = fmaxf(m, sc[j][t]);
        // reduce over TPH threads: within a wave, then across waves via LDS
        if constexpr (TPH >= 64) {
            m = wave_max(m);
        } else {
            m = max16(m);
            if constexpr (TPH == 32) m = fmaxf(m, __shfl_xor(m, 16, 64));
        }
        __shared__ float tmp[4];
        if constexpr (TPH > 64) {
            if (lane == 0) tmp[wave] = m;
            __syncthreads();
            const int w0 = (j * TPH) / 64;
            m = tmp[w0];
            for (int w = 1; w < TPH / 64; w++) m = fmaxf(m, tmp[w0 + w]);
            __syncthreads();
        }
        float l = 0.0f;
        for (uint32_t t = r; t < n; t += TPH) {
            const float p = expf(sc[j][t] - m);
            sc[j][t] = p;
            l += p;
        }
        if constexpr (TPH >= 64) {
            l = wave_sum(l);
        } else {
            l = sum16(l);
            if constexpr (TPH == 32) l += __shfl_xor(l, 16, 64);
        }
        if constexpr (TPH > 64) {
            if (lane == 0) tmp[wave] = l;
            __syncthreads();
            const int w0 = (j * TPH) / 64;
            l = tmp[w0];
            for (int w = 1; w < TPH / 64; w++) l += tmp[w0 + w];
        }
        if (r == 0) {
            ml[j][0] = m;
            ml[j][1] = l;
        }
    }
    __syncthreads();

    // ---- o = sum_t p_t v_t
    float o[G][8];
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[j][e] = 0.0f;
    for (uint32_t base = 0; base < n; base += PPP * ATTN_UNROLL) {
        float kv[ATTN_UNROLL][8];
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; u++) {
            const uint32_t tt = base + (uint32_t)(pg + PPP * u);
            if (tt < n) load_kv8<F16>(a.v_cache, (size_t)(t0 + tt) * a.kv_dim + head_off, kv[u]);
        }
#pragma unroll
        for (int u = 0; u < ATTN_UNROLL; u++) {
            const uint32_t tt = base + (uint32_t)(pg + PPP * u);
            if (tt < n) {
#pragma unroll
                for (int j = 0; j < G; j++) {
                    const float p = sc[j][tt];
#pragma unroll
                    for (int e = 0; e < 8; e++) o[j][e] = fmaf(p, kv[u][e], o[j][e]);
                }
            }
        }
    }
    // reduce over the LPW position groups of the wave (lanes dc + TPP*k) ...
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[j][e];
#pragma unroll
            for (int sh = TPP; sh < 64; sh <<= 1) v += __shfl_xor(v, sh, 64);
            o[j][e] = v;
        }
    // ... then over the 4 waves
    if (lane < TPP) {
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) red[wave][lane][8 * j + e] = o[j][e];
    }
    __syncthreads();

    // ---- write this split's partial
    const size_t pidx = ((size_t)kvh * S + s) * G;
    for (int i = tid; i < G * HS; i += ATTN_THREADS) {
        const int j = i / HS, d = i % HS, c2 = d / 8, e = d % 8;
        const float v = (red[0][c2][8 * j + e] + red[1][c2][8 * j + e]) + (red[2][c2][8 * j + e] + red[3][c2][8 * j + e]);
        a.part_o[(pidx + j) * HS + d] = v;
    }
    if (tid < G) {
        a.part_ml[(pidx + tid) * 2] = ml[tid][0];
        a.part_ml[(pidx + tid) * 2 + 1] = ml[tid][1];
    }
}

// Merge of the split partials: one workgroup of ATTN_MERGE_THREADS per query
// head; thread (q, d) sums splits q, q + Q, ... for head dim d, all of its
// loads issued before use, then the Q groups are combined in LDS.
constexpr int ATTN_MERGE_THREADS = 512;

template <int HS, int G>
__device__ void attn_merge_body(const AttnArgs &a) {
    constexpr int Q = ATTN_MERGE_THREADS / HS;             // split groups
    constexpr int PER = (ATTN_MERGE_MAX + Q - 1) / Q;      // splits per thread at most
    __shared__ float wgt[ATTN_MERGE_MAX];
    __shared__ float part[Q][HS];
    __shared__ float Lsum;
    const int tid = threadIdx.x;
    const uint32_t h = blockIdx.x, kvh = h / G, j = h % G, S = a.n_splits;
    const uint32_t T = min(*a.pos + 1, a.seq_cap);
    const uint32_t C = min(max((T + S - 1) / S, (uint32_t)ATTN_CMIN), (uint32_t)ATTN_CMAX);
    const uint32_t n_act = (T + C - 1) / C;
    for (uint32_t t = tid; t < n_act; t += ATTN_MERGE_THREADS)
        wgt[t] = a.part_ml[(((size_t)kvh * S + t) * G + j) * 2];
    __syncthreads();
    if (tid < 64) {
        float M = -INFINITY;
        for (uint32_t t = tid; t < n_act; t += 64) M = fmaxf(M, wgt[t]);
        M = wave_max(M);
        float L = 0.0f;
        for (uint32_t t = tid; t < n_act; t += 64) {
            const float w = expf(wgt[t] - M);
            wgt[t] = w;
            L = fmaf(a.part_ml[(((size_t)kvh * S + t) * G + j) * 2 + 1], w, L);
        }
        L = wave_sum(L);
        if (tid == 0) Lsum = L;
    }
    __syncthreads();
    const int d = tid % HS, q = tid / HS;
    const float *po = a.part_o + ((size_t)kvh * S * G + j) * HS + d; // split t at po[t * G * HS]
    float v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const uint32_t t = (uint32_t)(q + Q * u);
        v[u] = t < n_act ? po[(size_t)t * G * HS] : 0.0f;
    }
    float O = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const uint32_t t = (uint32_t)(q + Q * u);
        if (t < n_act) O = fmaf(v[u], wgt[t], O);
    }
    part[q][d] = O;
    __syncthreads();
    // head dims are written (and quantized for the next GEMV: a head is
    // HS/16 whole activation groups) by the first HS threads
    if (tid < ((HS + 63) / 64) * 64) {
        const bool ok = tid < HS;
        float r = 0.0f;
        if (ok) {
#pragma unroll
            for (int k = 0; k < Q; k++) r += part[k][tid];
            r /= Lsum;
            a.out[(size_t)h * HS + tid] = r;
        }
        if (a.xq_out) quant16(r, ok, a.xq_out, a.n_out, (uint32_t)(h * HS + tid), tid & 63);
    }
}

} // namespace ifr

// Flash-decoding attention for one token over a [seq][kv_dim] KV cache.
//
// Grid (n_kv_heads, n_splits).  Workgroup (h, s) serves the G = kv_mul query
// heads that share KV head h (grouped-query attention reads each K/V row once
// for all of them, where the reference's fused_attention reads it once per
// query head: fused_attention.rs:66-241) over the s-th chunk of the positions
// [0, pos].  The chunk length is ceil((pos+1)/n_splits), at least ATTN_CMIN,
// computed on the device from the device-resident position, so one launch
// shape serves every position (and a captured graph can be replayed).
//
// A position's K (and V) row of one head is read by TPP = HS/8 lanes, 8 dims
// each.  Per batch a thread issues the K and the V rows of its ATTN_BATCH
// positions together, then forms the scores q.k / sqrt(hs) (a DPP sum over
// the TPP lanes) and folds them into a running softmax (m, l, o) per query
// head.  The per-thread states are combined over the wave with shuffles and
// over the workgroup through LDS; the chunk's partial (m, l, o) goes to
// global memory.  A second, small kernel (attn_merge_body) combines the
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
constexpr int ATTN_BATCH = 4;  // positions per thread whose K and V are loaded together

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

// Running-softmax update: fold a state (m2, l2, o2) into (m, l, o).  An
// empty state has m = -inf, l = 0, o = 0.
template <int N>
IFR_DEV void softmax_fold(float &m, float &l, float *o, float m2, float l2, const float *o2) {
    const float mn = fmaxf(m, m2);
    const float a1 = m == -INFINITY ? 0.0f : expf(m - mn);
    const float a2 = m2 == -INFINITY ? 0.0f : expf(m2 - mn);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < N; e++) o[e] = o[e] * a1 + o2[e] * a2;
    m = mn;
}

template <int HS, int G, bool F16>
__device__ void attn_body(const AttnArgs &a) {
    constexpr int TPP = HS / 8;             // lanes per position (8 dims each)
    constexpr int PPW = 64 / TPP;           // positions per wave and pass
    constexpr int NW = ATTN_THREADS / 64;   // waves
    constexpr int PPP = NW * PPW;           // positions per workgroup and pass
    constexpr int U = ATTN_BATCH;
    __shared__ float wo[NW][G][HS];
    __shared__ float wml[NW][G][2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kvh = blockIdx.x, s = blockIdx.y, S = a.n_splits;
    const uint32_t T = min(*a.pos + 1, a.seq_cap);
    // chunk: at least ATTN_CMIN positions (short contexts use few splits, so
    // the merge reads few partials); the host sizes n_splits so that the
    // chunk never exceeds ATTN_CMAX
    const uint32_t C = min(max((T + S - 1) / S, (uint32_t)ATTN_CMIN), (uint32_t)ATTN_CMAX);
    const uint32_t t0 = s * C;
    if (t0 >= T) return;
    const uint32_t n = min(C, T - t0);

    const int dc = lane % TPP;
    const uint32_t pg = (uint32_t)(wave * PPW + lane / TPP);
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

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int j = 0; j < G; j++) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[j][e] = 0.0f;
    }

    for (uint32_t base = 0; base < n; base += PPP * U) {
        float kr[U][8], vr[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t tt = base + pg + PPP * u;
            // a position past the chunk reads the chunk's first row (in bounds) and is masked below
            const size_t off = (size_t)(t0 + (tt < n ? tt : 0)) * a.kv_dim + head_off;
            load_kv8<F16>(a.k_cache, off, kr[u]);
            load_kv8<F16>(a.v_cache, off, vr[u]);
        }
#pragma unroll
        for (int j = 0; j < G; j++) {
            float sc[U];
            float mb = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; u++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(q[j][e], kr[u][e], d);
                d = group_sum<TPP>(d) / inv_div;
                sc[u] = (base + pg + PPP * u < n) ? d : -INFINITY;
                mb = fmaxf(mb, sc[u]);
            }
            if (mb == -INFINITY) continue; // no position of this batch for this thread
            const float mn = fmaxf(m[j], mb);
            const float al = m[j] == -INFINITY ? 0.0f : expf(m[j] - mn);
            float lsum = l[j] * al, ov[8];
#pragma unroll
            for (int e = 0; e < 8; e++) ov[e] = o[j][e] * al;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = expf(sc[u] - mn); // 0 for a masked position
                lsum += p;
#pragma unroll
                for (int e = 0; e < 8; e++) ov[e] = fmaf(p, vr[u][e], ov[e]);
            }
            m[j] = mn;
            l[j] = lsum;
#pragma unroll
            for (int e = 0; e < 8; e++) o[j][e] = ov[e];
        }
    }

    // combine the PPW position groups of the wave (lanes dc + TPP*k)
#pragma unroll
    for (int sh = TPP; sh < 64; sh <<= 1) {
#pragma unroll
        for (int j = 0; j < G; j++) {
            const float m2 = __shfl_xor(m[j], sh, 64), l2 = __shfl_xor(l[j], sh, 64);
            float o2[8];
#pragma unroll
            for (int e = 0; e < 8; e++) o2[e] = __shfl_xor(o[j][e], sh, 64);
            softmax_fold<8>(m[j], l[j], o[j], m2, l2, o2);
        }
    }
    if (lane < TPP) {
#pragma unroll
        for (int j = 0; j < G; j++) {
#pragma unroll
            for (int e = 0; e < 8; e++) wo[wave][j][dc * 8 + e] = o[j][e];
            if (dc == 0) {
                wml[wave][j][0] = m[j];
                wml[wave][j][1] = l[j];
            }
        }
    }
    __syncthreads();

    // ... then over the waves, and write this split's partial
    const size_t pidx = ((size_t)kvh * S + s) * G;
    for (int i = tid; i < G * HS; i += ATTN_THREADS) {
        const int j = i / HS, d = i % HS;
        float M = wml[0][j][0];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wml[w][j][0]);
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++)
            if (wml[w][j][0] != -INFINITY) v = fmaf(expf(wml[w][j][0] - M), wo[w][j][d], v);
        a.part_o[(pidx + j) * HS + d] = v;
        if (d == 0) {
            float L = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++)
                if (wml[w][j][0] != -INFINITY) L = fmaf(expf(wml[w][j][0] - M), wml[w][j][1], L);
            a.part_ml[(pidx + j) * 2] = M;
            a.part_ml[(pidx + j) * 2 + 1] = L;
        }
    }
}

// Merge of the split partials: one workgroup of ATTN_MERGE_THREADS per query
// head; thread (q, d) sums splits q, q + Q, ... for head dim d.  Every
// partial load is issued at the start, then the split weights e^(m_s - M)
// are formed in LDS and the Q groups combined there.
constexpr int ATTN_MERGE_THREADS = 512;

template <int HS, int G>
__device__ void attn_merge_body(const AttnArgs &a) {
    constexpr int Q = ATTN_MERGE_THREADS / HS;             // split groups
    constexpr int PER = (ATTN_MERGE_MAX + Q - 1) / Q;      // splits per thread at most
    __shared__ float wm[ATTN_MERGE_MAX], wl[ATTN_MERGE_MAX];
    __shared__ float part[Q][HS];
    __shared__ float Lsum;
    const int tid = threadIdx.x;
    const uint32_t h = blockIdx.x, kvh = h / G, j = h % G, S = a.n_splits;
    const uint32_t T = min(*a.pos + 1, a.seq_cap);
    const uint32_t C = min(max((T + S - 1) / S, (uint32_t)ATTN_CMIN), (uint32_t)ATTN_CMAX);
    const uint32_t n_act = (T + C - 1) / C;
    const int d = tid % HS, qg = tid / HS;
    const float *po = a.part_o + ((size_t)kvh * S * G + j) * HS + d; // split t at po[t * G * HS]
    float v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const uint32_t t = (uint32_t)(qg + Q * u);
        v[u] = t < n_act ? po[(size_t)t * G * HS] : 0.0f;
    }
    for (uint32_t t = tid; t < n_act; t += ATTN_MERGE_THREADS) {
        const float *ml = a.part_ml + (((size_t)kvh * S + t) * G + j) * 2;
        wm[t] = ml[0];
        wl[t] = ml[1];
    }
    __syncthreads();
    if (tid < 64) {
        float M = -INFINITY;
        for (uint32_t t = tid; t < n_act; t += 64) M = fmaxf(M, wm[t]);
        M = wave_max(M);
        float L = 0.0f;
        for (uint32_t t = tid; t < n_act; t += 64) {
            const float w = expf(wm[t] - M);
            wm[t] = w;
            L = fmaf(wl[t], w, L);
        }
        L = wave_sum(L);
        if (tid == 0) Lsum = L;
    }
    __syncthreads();
    float O = 0.0f;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const uint32_t t = (uint32_t)(qg + Q * u);
        if (t < n_act) O = fmaf(v[u], wm[t], O);
    }
    part[qg][d] = O;
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

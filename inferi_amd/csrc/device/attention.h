// Flash-decoding attention for one token over a [seq][kv_dim] KV cache.
//
// Grid (n_kv_heads, n_splits).  Workgroup (h, s) serves the G = kv_mul query
// heads that share KV head h (grouped-query attention reads each K/V row once
// for all of them, where the reference's fused_attention reads it once per
// query head: fused_attention.rs:66-241) over the s-th chunk of the positions
// [0, pos].  The chunk length is ceil((pos+1)/n_splits) rounded up to whole
// batches, computed on the device from the device-resident position, so one
// launch shape serves every position (and a captured graph can be replayed).
//
// A position's K (and V) row of one head is read by TPP = HS/8 lanes, 8 dims
// each.  Per batch a thread issues the K and the V rows of its ATTN_BATCH
// positions together, then forms the scores q.k / sqrt(hs) (a DPP sum over
// the TPP lanes) and folds them into a running softmax (m, l, o) per query
// head.  The per-thread states are combined through LDS; the chunk's partial
// (m, l, o) goes to global memory.  A second, small kernel (attn_merge_body) combines the
// partials of each query head: out = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.
// The kernel boundary orders the two.  (Merging in the last split workgroup
// of each KV head instead, with an arrival counter, measured slower: with
// device-scope release fences every workgroup writes back its XCD's L2, and
// even with write-through partial stores one workgroup per KV head reading
// all splits' partials takes longer than the second launch.)
#pragma once
#include "gemv.h"

namespace ifr {

constexpr int ATTN_THREADS = 256;
constexpr int ATTN_CMAX = 256; // longest chunk a workgroup accepts
constexpr int ATTN_MERGE_MAX = 256;  // most splits one KV head may have
constexpr int ATTN_BATCH = 4;  // positions per thread whose K and V are loaded together

// Eight consecutive cache elements of one row, kept raw until used (f16:
// u; f32: u and w), so a batch's loads are issued back to back and the
// conversions wait for the data only where the scores need it.
template <bool F16>
struct KV8 {
    uint4 u, w;
};
template <bool F16>
IFR_DEV void kv8_load(const void *cache, size_t off, KV8<F16> &r) {
    if constexpr (F16) {
        r.u = *(const uint4 *)((const uint16_t *)cache + off);
    } else {
        r.u = *(const uint4 *)((const float *)cache + off);
        r.w = *(const uint4 *)((const float *)cache + off + 4);
    }
}
template <bool F16>
IFR_DEV void kv8_zero(KV8<F16> &r) {
    r.u = make_uint4(0u, 0u, 0u, 0u);
    r.w = r.u;
}
// element e (0..7) as f32, read where it is multiplied (an f16 element
// widened inside the FMA, which the compiler folds into a mixed-precision
// FMA, so no converted copy of the batch is kept)
template <bool F16>
IFR_DEV float kv8_at(const KV8<F16> &r, int e) {
    const uint32_t w = e < 2 ? r.u.x : e < 4 ? r.u.y : e < 6 ? r.u.z : r.u.w;
    if constexpr (F16) {
        return f16_to_f32((e & 1) ? (w >> 16) : (w & 0xFFFFu));
    } else {
        const uint32_t w2 = e == 0 ? r.u.x : e == 1 ? r.u.y : e == 2 ? r.u.z : e == 3 ? r.u.w
                          : e == 4 ? r.w.x : e == 5 ? r.w.y : e == 6 ? r.w.z : r.w.w;
        return __uint_as_float(w2);
    }
}

template <int TPP>
IFR_DEV float group_sum(float v) {
    if constexpr (TPP == 16) return sum16(v);
    else return sum8(v);
}

// Positions per batch of one workgroup (every thread loads ATTN_BATCH
// positions): the chunk of a split is a multiple of it.
template <int HS>
constexpr uint32_t attn_quantum() { return (uint32_t)(ATTN_THREADS / (HS / 8)) * ATTN_BATCH; }

// Chunk length of every split for T positions over S splits: at least one
// batch, a whole number of batches, at most ATTN_CMAX (the host sizes S so
// that T <= S * ATTN_CMAX).
template <int HS>
IFR_DEV uint32_t attn_chunk(uint32_t T, uint32_t S) {
    constexpr uint32_t Q = attn_quantum<HS>();
    const uint32_t c = max((T + S - 1) / S, Q);
    return min((c + Q - 1) / Q * Q, (uint32_t)ATTN_CMAX);
}

// Scores are kept in base-2 units: q is pre-scaled by log2(e)/sqrt(hs), so
// e^(s - m) of the reference's softmax is 2^(s2 - m2) here, and the partial
// maxima handed to the merge are in the same units.
// LDS of one attention item (one split of one KV head).
template <int HS, int G>
struct AttnLds {
    static constexpr int NPG = ATTN_THREADS / 64 * (64 / (HS / 8)); // position groups
    float og[NPG][G][HS]; // per position group: unnormalised o
    float mg[NPG][G], lg[NPG][G];
    float wg[NPG][G], Mh[G];
};

// Positions of the split [t0, t0 + C) below T.  Written without a select
// on t0 < T: hipcc (ROCm 7.2) folds `t0 < T ? min(C, T - t0) : 0`, when the
// result is only compared with other values, into min(C, T - t0) and the
// subtraction then wraps for an empty split.
IFR_DEV uint32_t split_len(uint32_t t0, uint32_t C, uint32_t T) {
    const uint32_t end = min(T, t0 + C);
    return end - min(end, t0);
}

// One split s of KV head kvh, computed by the ATTN_THREADS threads tid of a
// workgroup that call it together.  Every thread of the workgroup passes the
// same barriers: threads of an inactive item (active false) take part in
// them and do nothing else, so several items can share one workgroup.  COH:
// partials written with coherent stores (read in the same launch).
template <int HS, int G, bool F16, bool COH>
__device__ void attn_item(const AttnArgs &a, uint32_t kvh, uint32_t s, int tid, bool active, AttnLds<HS, G> &L) {
    constexpr int TPP = HS / 8;             // lanes per position (8 dims each)
    constexpr int PPW = 64 / TPP;           // positions per wave and pass
    constexpr int NW = ATTN_THREADS / 64;   // waves
    constexpr int PPP = NW * PPW;           // positions per workgroup and pass
    constexpr int NPG = PPP;                // position groups (threads sharing a dim slice)
    constexpr int U = ATTN_BATCH;
    auto &og = L.og;
    auto &mg = L.mg;
    auto &lg = L.lg;
    auto &wg = L.wg;
    auto &Mh = L.Mh;

    // arguments in one batch of scalar loads (the compiler would otherwise
    // fetch them in dependent round trips next to their first uses); an
    // empty asm that emits nothing
    asm volatile("" ::"s"(a.q), "s"(a.k_cache), "s"(a.v_cache), "s"(a.part_o), "s"(a.part_ml), "s"(a.pos),
                 "s"(a.kv_dim), "s"(a.n_splits), "s"(a.seq_cap));
    // the device position, as a vector load issued before every other load:
    // loads complete in issue order, so waiting for it waits for nothing else
    const uint32_t pos_dev = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t S = a.n_splits;
    constexpr uint32_t Qb = attn_quantum<HS>();
    const int dc = lane % TPP;
    const uint32_t pg = (uint32_t)(wave * PPW + lane / TPP);
    const size_t head_off = (size_t)kvh * HS + (size_t)dc * 8;
    const size_t pidx = ((size_t)kvh * S + s) * G;

    // this thread's 8 query dims of every head of the group, pre-scaled
    const float qs = 1.44269504088896341f / sqrtf((float)HS);
    float q[G][8];
#pragma unroll
    for (int j = 0; j < G; j++) {
        const float4 u = *(const float4 *)(a.q + (size_t)(kvh * G + j) * HS + dc * 8);
        const float4 w = *(const float4 *)(a.q + (size_t)(kvh * G + j) * HS + dc * 8 + 4);
        q[j][0] = u.x * qs; q[j][1] = u.y * qs; q[j][2] = u.z * qs; q[j][3] = u.w * qs;
        q[j][4] = w.x * qs; q[j][5] = w.y * qs; q[j][6] = w.z * qs; q[j][7] = w.w * qs;
    }

    // When S batches cover the whole cache (S * Qb >= seq_cap) every chunk is
    // one batch of Qb positions at s * Qb, known before the device position
    // arrives: the first batch's K and V loads go out together with the
    // position load (rows clamped into the cache, masked below).
    const bool fixed = S * Qb >= a.seq_cap;
    KV8<F16> kr[ATTN_BATCH], vr[ATTN_BATCH];
    auto load_batch = [&](uint32_t t0, uint32_t base, uint32_t n) {
#pragma unroll
        for (int u = 0; u < ATTN_BATCH; u++) {
            const uint32_t tt = base + pg + PPP * u;
            const uint32_t row = n ? t0 + (tt < n ? tt : 0) : min(t0 + tt, a.seq_cap - 1);
            const size_t off = (size_t)row * a.kv_dim + head_off;
            kv8_load<F16>(a.k_cache, off, kr[u]);
            kv8_load<F16>(a.v_cache, off, vr[u]);
        }
    };
    if (fixed && active) load_batch(s * Qb, 0, 0);
    __builtin_amdgcn_sched_barrier(0); // the batch's loads stay together
    const uint32_t T = min((uint32_t)__builtin_amdgcn_readfirstlane(pos_dev) + 1u, a.seq_cap);
    const uint32_t C = fixed ? Qb : attn_chunk<HS>(T, S);
    const uint32_t t0 = s * C;
    if (active && t0 >= T && tid < G) {
        // an empty split: a partial the merge gives weight 0
        st_out<COH>(a.part_ml + (pidx + tid) * 2, -INFINITY);
        st_out<COH>(a.part_ml + (pidx + tid) * 2 + 1, 0.0f);
    }
    const bool live = active && t0 < T;
    const uint32_t n = active ? split_len(t0, C, T) : 0u;

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int j = 0; j < G; j++) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[j][e] = 0.0f;
    }

    for (uint32_t base = 0; base < n; base += PPP * U) {
        if (!fixed || base) load_batch(t0, base, n);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; u++)
            if (base + pg + PPP * u >= n) {
                // a masked row (possibly never written): its values must not reach the sums
                kv8_zero<F16>(vr[u]);
            }
#pragma unroll
        for (int j = 0; j < G; j++) {
            float sc[U];
            float mb = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; u++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) d = fmaf(q[j][e], kv8_at<F16>(kr[u], e), d);
                d = group_sum<TPP>(d);
                sc[u] = (base + pg + PPP * u < n) ? d : -INFINITY;
                mb = fmaxf(mb, sc[u]);
            }
            if (mb == -INFINITY) continue; // no position of this batch for this thread
            const float mn = fmaxf(m[j], mb);
            const float al = exp2f(m[j] - mn); // 0 while m[j] is still -inf
            float lsum = l[j] * al, ov[8];
#pragma unroll
            for (int e = 0; e < 8; e++) ov[e] = o[j][e] * al;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = exp2f(sc[u] - mn); // 0 for a masked position
                lsum += p;
#pragma unroll
                for (int e = 0; e < 8; e++) ov[e] = fmaf(p, kv8_at<F16>(vr[u], e), ov[e]);
            }
            m[j] = mn;
            l[j] = lsum;
#pragma unroll
            for (int e = 0; e < 8; e++) o[j][e] = ov[e];
        }
    }

    // combine the NPG position groups through LDS: states, then per-head
    // maxima and weights 2^(m_g - M), then the weighted sums of o
    if (live) {
#pragma unroll
        for (int j = 0; j < G; j++) {
#pragma unroll
            for (int e = 0; e < 8; e++) og[pg][j][dc * 8 + e] = o[j][e];
            if (dc == 0) {
                mg[pg][j] = m[j];
                lg[pg][j] = l[j];
            }
        }
    }
    __syncthreads();
    if (live && tid < G) {
        float M = -INFINITY;
        for (int g = 0; g < NPG; g++) M = fmaxf(M, mg[g][tid]);
        Mh[tid] = M;
    }
    __syncthreads();
    if (live)
        for (int i = tid; i < NPG * G; i += ATTN_THREADS) {
            const int g = i / G, j = i % G;
            wg[g][j] = exp2f(mg[g][j] - Mh[j]); // 0 for a group that saw no position
        }
    __syncthreads();

    if (live)
        for (int i = tid; i < G * HS; i += ATTN_THREADS) {
            const int j = i / HS, d = i % HS;
            float v = 0.0f;
#pragma unroll
            for (int g = 0; g < NPG; g++) v = fmaf(wg[g][j], og[g][j][d], v);
            st_out<COH>(a.part_o + (pidx + j) * HS + d, v);
            if (d == 0) {
                float Ls = 0.0f;
#pragma unroll
                for (int g = 0; g < NPG; g++) Ls = fmaf(wg[g][j], lg[g][j], Ls);
                st_out<COH>(a.part_ml + (pidx + j) * 2, Mh[j]);
                st_out<COH>(a.part_ml + (pidx + j) * 2 + 1, Ls);
            }
        }
}

template <int HS, int G, bool F16>
__device__ void attn_body(const AttnArgs &a) {
    __shared__ AttnLds<HS, G> L;
    attn_item<HS, G, F16, false>(a, blockIdx.x, blockIdx.y, (int)threadIdx.x, true, L);
}

// The split kernel with q.k on the matrix cores (head size 128, f16 cache,
// G <= 4 query heads per KV head).  Workgroup (h, s): 4 waves of 32
// positions, chunk C (a multiple of 128) from s*C.  Per block of 32
// positions a wave forms the scores with v_mfma_f32_32x32x16_f16, A = the
// query as 2G rows (the f16 high part of 256*q of every head, then the f16
// low part, so hi + lo carries ~22 bits), B = the 32 K rows straight from
// the cache (lane l: row l % 32, dims 16k + 8(l / 32)..+8): lane l then holds
// the high-part sums of position l % 32 (l < 32) or the low-part sums
// (l >= 32), added across the two halves.  The wave's running softmax and
// P.V stay in fp32 on the vector ALUs: 16 lanes span a row's 128 dims, the
// four lane groups take 8 positions each and are summed by lane shuffles.
// The four waves' states combine through LDS into the split's partial.
// Scores are in base-2 units as in attn_body.
constexpr int ATTN2_WAVES = 4, ATTN2_PW = 32;
constexpr uint32_t ATTN2_QB = ATTN2_WAVES * ATTN2_PW; // positions per block of a workgroup

template <int G>
__device__ void attn2_body(const AttnArgs &a) {
    constexpr int HS = 128;
    static_assert(G <= 4, "2G query rows in the first 8 rows of the 32-row operand");
    __shared__ float pl[ATTN2_WAVES][G][ATTN2_PW];
    __shared__ float ow[ATTN2_WAVES][G][HS];
    __shared__ float mw[ATTN2_WAVES][G], lw[ATTN2_WAVES][G], wt[ATTN2_WAVES][G], Mh[G];
    asm volatile("" ::"s"(a.q), "s"(a.k_cache), "s"(a.v_cache), "s"(a.part_o), "s"(a.part_ml), "s"(a.pos),
                 "s"(a.kv_dim), "s"(a.n_splits), "s"(a.seq_cap));
    const uint32_t pos_dev = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t kvh = blockIdx.x, s = blockIdx.y, S = a.n_splits;
    const uint32_t li = (uint32_t)lane & 31u, lk = 8u * ((uint32_t)lane >> 5);
    const uint32_t vg = (uint32_t)lane >> 4, vd = 8u * ((uint32_t)lane & 15u); // P.V: positions 8vg.., dims vd..
    const size_t pidx = ((size_t)kvh * S + s) * G;
    const uint16_t *kc = (const uint16_t *)a.k_cache, *vc = (const uint16_t *)a.v_cache;
    const uint32_t C = a.chunk, t0 = s * C;
    const uint32_t nblk = C / ATTN2_QB;

    // this block's K (MFMA layout) and V (P.V layout) rows, clamped into the cache
    uint4 kb[8], vb[8];
    auto load_block = [&](uint32_t blk) {
        const uint32_t p0 = t0 + blk * ATTN2_QB + (uint32_t)wave * ATTN2_PW;
        const uint32_t kr = min(p0 + li, a.seq_cap - 1);
        const uint16_t *krow = kc + (size_t)kr * a.kv_dim + (size_t)kvh * HS + lk;
#pragma unroll
        for (int k = 0; k < 8; k++) kb[k] = *(const uint4 *)(krow + 16 * k);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t vr = min(p0 + 8 * vg + (uint32_t)u, a.seq_cap - 1);
            vb[u] = *(const uint4 *)(vc + (size_t)vr * a.kv_dim + (size_t)kvh * HS + vd);
        }
    };
    load_block(0);
    __builtin_amdgcn_sched_barrier(0);

    // the query operand: row li < G: hi(256 q_li), G <= li < 2G: lo, else 0
    // (scaled by log2(e)/sqrt(hs) and by 2^8, undone on the scores exactly)
    half8v aq[8];
    {
        const float qs = 1.44269504088896341f / sqrtf((float)HS) * 256.0f;
        const uint32_t h = li < (uint32_t)G ? li : li - G;
        const bool used = li < 2u * G;
        const float *qrow = a.q + (size_t)(kvh * G + (used ? h : 0u)) * HS + lk;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 x0 = *(const float4 *)(qrow + 16 * k), x1 = *(const float4 *)(qrow + 16 * k + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = xv[e] * qs;
                const _Float16 hi = (_Float16)v;
                const _Float16 lo = (_Float16)(v - (float)hi);
                aq[k][e] = !used ? (_Float16)0.0f : li < (uint32_t)G ? hi : lo;
            }
        }
    }

    const uint32_t T = min((uint32_t)__builtin_amdgcn_readfirstlane(pos_dev) + 1u, a.seq_cap);
    const uint32_t n = split_len(t0, C, T);

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int j = 0; j < G; j++) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[j][e] = 0.0f;
    }
    for (uint32_t blk = 0; blk * ATTN2_QB < n; blk++) {
        const uint32_t b0 = blk * ATTN2_QB + (uint32_t)wave * ATTN2_PW; // this wave's first position in the chunk
        float16v acc;
#pragma unroll
        for (int e = 0; e < 16; e++) acc[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            half8v bv;
            __builtin_memcpy(&bv, &kb[k], 16);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq[k], bv, acc, 0, 0, 0);
        }
        // rows 0..3 of lanes < 32 and 4..7 of lanes >= 32 (registers 0..3):
        // G = 4: hi of head e in lanes < 32, lo of head e in lanes >= 32
        const bool pos_ok = b0 + li < n;
        float sc[G];
#pragma unroll
        for (int j = 0; j < G; j++) {
            // row j (hi) sits in register j of lanes < 32 when j < 4; row G + j
            // (lo) in register (G + j) - 4 of lanes >= 32 when G + j >= 4,
            // else in register G + j of lanes < 32
            const float mine = acc[j];
            const float hi = __shfl(mine, (int)li, 64);
            float lo;
            if constexpr (G == 4) {
                lo = __shfl(acc[j], (int)li + 32, 64);
            } else {
                const int r = G + j;
                const float cand = r < 4 ? acc[r < 4 ? r : 0] : acc[r >= 4 ? r - 4 : 0];
                lo = __shfl(cand, r < 4 ? (int)li : (int)li + 32, 64);
            }
            sc[j] = pos_ok ? (hi + lo) * (1.0f / 256.0f) : -INFINITY;
        }
        // the wave's new maxima, probabilities and their sums (positions in lanes 0..31)
        float p[G];
#pragma unroll
        for (int j = 0; j < G; j++) {
            const float bm = wave_max(lane < 32 ? sc[j] : -INFINITY);
            const float mn = fmaxf(m[j], bm);
            const float al = mn == -INFINITY ? 1.0f : exp2f(m[j] - mn);
            p[j] = (lane < 32 && sc[j] != -INFINITY) ? exp2f(sc[j] - mn) : 0.0f;
            l[j] = l[j] * al + wave_sum(p[j]);
            m[j] = mn;
#pragma unroll
            for (int e = 0; e < 8; e++) o[j][e] *= al;
        }
        if (lane < 32) {
#pragma unroll
            for (int j = 0; j < G; j++) pl[wave][j][li] = p[j];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): this wave's LDS writes are visible to it
        // P.V: lane group vg takes positions 8vg..8vg+7 of the wave's 32, 8 dims
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const bool vok = b0 + 8 * vg + (uint32_t)u < n;
            const uint4 w = vok ? vb[u] : make_uint4(0u, 0u, 0u, 0u); // masked rows never reach the sums
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < G; j++) {
                const float pj = pl[wave][j][8 * vg + u];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t hb = (e & 1) ? (ww[e >> 1] >> 16) : (ww[e >> 1] & 0xFFFFu);
                    o[j][e] = fmaf(pj, f16_to_f32(hb), o[j][e]);
                }
            }
        }
        // next block's rows (none past the chunk's positions)
        if ((blk + 1) * ATTN2_QB < n) load_block(blk + 1);
    }
    // the four lane groups of the wave hold disjoint positions of the same dims
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            o[j][e] += __shfl_xor(o[j][e], 16, 64);
            o[j][e] += __shfl_xor(o[j][e], 32, 64);
        }
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) ow[wave][j][vd + e] = o[j][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < G; j++) {
            mw[wave][j] = m[j];
            lw[wave][j] = l[j];
        }
    }
    __syncthreads();
    if (tid < G) {
        float M = -INFINITY;
        for (int w = 0; w < ATTN2_WAVES; w++) M = fmaxf(M, mw[w][tid]);
        Mh[tid] = M;
        for (int w = 0; w < ATTN2_WAVES; w++) wt[w][tid] = mw[w][tid] == -INFINITY ? 0.0f : exp2f(mw[w][tid] - M);
    }
    __syncthreads();
    if (n == 0) {
        // an empty split: a partial the merge gives weight 0
        if (tid < G) {
            a.part_ml[(pidx + tid) * 2] = -INFINITY;
            a.part_ml[(pidx + tid) * 2 + 1] = 0.0f;
        }
        return;
    }
    for (int i = tid; i < G * HS; i += ATTN2_WAVES * 64) {
        const int j = i / HS, d = i % HS;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < ATTN2_WAVES; w++) v = fmaf(wt[w][j], ow[w][j][d], v);
        a.part_o[(pidx + j) * HS + d] = v;
        if (d == 0) {
            float L = 0.0f;
#pragma unroll
            for (int w = 0; w < ATTN2_WAVES; w++) L = fmaf(wt[w][j], lw[w][j], L);
            a.part_ml[(pidx + j) * 2] = Mh[j];
            a.part_ml[(pidx + j) * 2 + 1] = L;
        }
    }
}

// Merge of the split partials, one wave per 16 output values (dims
// 16c..16c+15 of one query head): lane = (subset r = lane / 16, dim
// 16c + lane % 16); subset r folds splits r, r + 4, ... into a running
// (M, L, O) with base-2 weights, then the four subsets combine through lane
// shuffles: out = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s.  No LDS and no
// barrier.  Every split of the launch is read (an empty one carries m = -inf
// and is skipped), so no load waits for the position.
constexpr uint32_t ATTN_MERGE_SUBSETS = 4;
constexpr uint32_t ATTN_MERGE_CHUNK = 24; // splits of a subset whose loads are in flight together

IFR_DEV void merge_fold(float &M, float &L, float &O, float m, float l, float o) {
    if (m == -INFINITY) return; // an empty split (its o was never written)
    const float Mn = fmaxf(M, m);
    const float a = exp2f(M - Mn), b = exp2f(m - Mn); // a = 0 while M is -inf
    L = fmaf(l, b, L * a);
    O = fmaf(o, b, O * a);
    M = Mn;
}

template <int HS, int G>
__device__ void attn_merge_body(const AttnArgs &a) {
    constexpr uint32_t NR = ATTN_MERGE_SUBSETS, CH = ATTN_MERGE_CHUNK;
    const int lane = (int)threadIdx.x;
    const uint32_t grp = blockIdx.x, h = grp / (HS / 16), c = grp % (HS / 16);
    const uint32_t kvh = h / G, j = h % G, S = a.n_splits;
    const uint32_t r = (uint32_t)lane / 16, d = c * 16 + (uint32_t)lane % 16;
    const float *po = a.part_o + ((size_t)kvh * S * G + j) * HS + d; // split t at po[t * G * HS]
    const float *pml = a.part_ml + ((size_t)kvh * S * G + j) * 2;    // split t at pml[t * G * 2]
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (uint32_t t0 = r; t0 < S; t0 += NR * CH) {
        float mv[CH], lv[CH], ov[CH];
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) {
            const uint32_t t = t0 + NR * u;
            const bool ok = t < S;
            mv[u] = ok ? pml[(size_t)t * G * 2] : -INFINITY;
            lv[u] = ok ? pml[(size_t)t * G * 2 + 1] : 0.0f;
            ov[u] = ok ? po[(size_t)t * G * HS] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) merge_fold(M, L, O, mv[u], lv[u], ov[u]);
    }
    // the four subsets of each dim: lanes d, d + 16, d + 32, d + 48
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        const float Mo = __shfl_xor(M, off, 64), Lo = __shfl_xor(L, off, 64), Oo = __shfl_xor(O, off, 64);
        const float Mn = fmaxf(M, Mo);
        const float wa = M == -INFINITY ? 0.0f : exp2f(M - Mn), wb = Mo == -INFINITY ? 0.0f : exp2f(Mo - Mn);
        L = fmaf(Lo, wb, L * wa);
        O = fmaf(Oo, wb, O * wa);
        M = Mn;
    }
    const float res = O / L;
    const uint32_t oi = h * HS + d;
    const bool ok = lane < 16;
    if (ok && a.out) a.out[oi] = res;
    if (a.xq_out) quant16(ok ? res : 0.0f, ok, a.xq_out, a.n_out, oi, lane);
}

} // namespace ifr

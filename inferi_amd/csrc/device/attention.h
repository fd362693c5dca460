// Flash-decoding attention for one token over a [seq][kv_dim] KV cache.
//
// Grid (n_kv_heads * n_sub, n_splits).  Workgroup (x, s) serves up to GT of
// the G = kv_mul query heads that share KV head h = x / n_sub: heads
// (x % n_sub) * GT .. +GT of the group, those below G (grouped-query
// attention reads each K/V row once for all of them, where the reference's
// fused_attention reads it once per query head: fused_attention.rs:66-241,
// which takes any kv_mul and head size).  A group of more than 8 heads is
// split into n_sub sub-groups of GT.  Workgroup (x, s) covers the s-th chunk
// of the positions [0, pos].  The chunk length is ceil((pos+1)/n_splits)
// rounded up to whole batches, computed on the device from the
// device-resident position, so one launch shape serves every position (and a
// captured graph can be replayed).
//
// A position's K (and V) row of one head is read by TPP = HSP/8 lanes, 8 dims
// each, HSP being the head size rounded up to 64 or 128 (lanes past the head
// size load nothing and hold zeros).  Per batch a thread issues the K and the
// V rows of its ATTN_BATCH positions together, then forms the scores
// q.k / sqrt(hs) (a DPP sum over the TPP lanes) and folds them into a running
// softmax (m, l, o) per query head.  The per-thread states are combined
// through LDS; the chunk's partial (m, l, o) goes to global memory.  A second,
// small kernel (attn_merge_body) combines the partials of each query head:
// out = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.  The kernel boundary
// orders the two.  (Merging in the last split workgroup of each KV head
// instead, with an arrival counter, measured slower: with device-scope
// release fences every workgroup writes back its XCD's L2, and even with
// write-through partial stores one workgroup per KV head reading all splits'
// partials takes longer than the second launch.)
#pragma once
#include "gemv.h"

namespace ifr {

constexpr int ATTN_THREADS = 256;
constexpr int ATTN_BATCH = 4;  // positions per thread whose K and V are loaded together
constexpr int ATTN_GT_MAX = 8; // query heads one workgroup serves
// Start of a running maximum: finite, so that no max minus max is inf - inf
// (NaN) before the first valid score and no branch has to guard it; any real
// score is far above it, and 2^(it - score) is 0.
constexpr float ATTN_M0 = -1.0e30f;

// 2^x for softmax weights and rescales: the hardware v_exp_f32 (results
// below 2^-126 flush to 0, weights too small to change any sum; 2^-inf = 0).
IFR_DEV float softmax_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Eight consecutive cache elements of one row, kept raw until used (f16:
// u; f32: u and w), so a batch's loads are issued back to back and the
// conversions wait for the data only where the scores need it.
template <bool F16>
struct KV8 {
    uint4 u, w;
};
// The loads are non-temporal: a step reads each cache row once, and the
// streaming hint keeps them from displacing lines the step reuses (8B
// shape at 4.1 K positions: attention 11.81 -> 11.36 us per layer, -5
// us/token, alternated on one box).  The same hint on the GEMVs' weight
// loads measured far slower (gate/up 15.0 -> 18.8 us per layer), and on
// the partials' stores slower (+5 us/token).
IFR_DEV uint4 ld16_stream(const void *p) {
    const u32x4_a16 v = __builtin_nontemporal_load((const u32x4_a16 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <bool F16>
IFR_DEV void kv8_load(const void *cache, size_t off, KV8<F16> &r) {
    if constexpr (F16) {
        r.u = ld16_stream((const uint16_t *)cache + off);
    } else {
        r.u = ld16_stream((const float *)cache + off);
        r.w = ld16_stream((const float *)cache + off + 4);
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
template <int HSP>
constexpr uint32_t attn_quantum() { return (uint32_t)(ATTN_THREADS / (HSP / 8)) * ATTN_BATCH; }

// Chunk length of every split for T positions over S splits: at least one
// batch and a whole number of batches, so S chunks cover T.
template <int HSP>
IFR_DEV uint32_t attn_chunk(uint32_t T, uint32_t S) {
    constexpr uint32_t Q = attn_quantum<HSP>();
    const uint32_t c = max((T + S - 1) / S, Q);
    return (c + Q - 1) / Q * Q;
}

// Scores are kept in base-2 units: q is pre-scaled by log2(e)/sqrt(hs), so
// e^(s - m) of the reference's softmax is 2^(s2 - m2) here, and the partial
// maxima handed to the merge are in the same units.
template <int HSP, int GT>
struct AttnLds {
    static constexpr int NPG = ATTN_THREADS / 64 * (64 / (HSP / 8)); // position groups
    // per position group: unnormalised o, in a lane-half order: the thread
    // with dims 8c .. 8c+7 writes 8c..8c+3 at word 4c and 8c+4..8c+7 at
    // word HSP/2 + 4c, so the TPP threads of a group fill one contiguous row
    // per store (no bank conflicts); attn_og_dim maps a word back to its dim
    float og[NPG][GT][HSP];
    float mg[NPG][GT], lg[NPG][GT];
    float wg[NPG][GT], Mh[GT];
};

// Dim of word w of an og row (its lane-half order, see AttnLds).
template <int HSP>
IFR_DEV uint32_t attn_og_dim(uint32_t w) {
    constexpr uint32_t HH = HSP / 2;
    return (w % HH) / 4 * 8 + (w / HH) * 4 + w % 4;
}

// Positions of the split [t0, t0 + C) below T.  Written without a select
// on t0 < T: hipcc (ROCm 7.2) folds `t0 < T ? min(C, T - t0) : 0`, when the
// result is only compared with other values, into min(C, T - t0) and the
// subtraction then wraps for an empty split.
IFR_DEV uint32_t split_len(uint32_t t0, uint32_t C, uint32_t T) {
    const uint32_t end = min(T, t0 + C);
    return end - min(end, t0);
}

// Partials are laid out per query head h = kvh * G + j:
// part_o[(h * S + s) * hs + d], part_ml[(h * S + s) * 2 + {0: m, 1: l}].
template <int HSP, int GT, bool F16>
__device__ void attn_split_body(const AttnArgs &a) {
    constexpr int TPP = HSP / 8;            // lanes per position (8 dims each)
    constexpr int PPW = 64 / TPP;           // positions per wave and pass
    constexpr int NW = ATTN_THREADS / 64;   // waves
    constexpr int PPP = NW * PPW;           // positions per workgroup and pass
    constexpr int NPG = PPP;                // position groups (threads sharing a dim slice)
    constexpr int U = ATTN_BATCH;
    __shared__ AttnLds<HSP, GT> L;
    auto &og = L.og;
    auto &mg = L.mg;
    auto &lg = L.lg;
    auto &wg = L.wg;
    auto &Mh = L.Mh;

    // arguments in one batch of scalar loads (the compiler would otherwise
    // fetch them in dependent round trips next to their first uses); an
    // empty asm that emits nothing
    asm volatile("" ::"s"(a.q), "s"(a.k_cache), "s"(a.v_cache), "s"(a.part_o), "s"(a.part_ml), "s"(a.pos),
                 "s"(a.kv_dim), "s"(a.n_splits), "s"(a.seq_cap), "s"(a.head_size), "s"(a.kv_mul), "s"(a.n_sub));
    // the device position, as a vector load issued before every other load:
    // loads complete in issue order, so waiting for it waits for nothing else
    const uint32_t pos_dev = __hip_atomic_load(a.pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t S = a.n_splits, hs = a.head_size, G = a.kv_mul;
    const uint32_t kvh = blockIdx.x / a.n_sub, j0 = (blockIdx.x % a.n_sub) * GT, s = blockIdx.y;
    const uint32_t nj = j0 < G ? min((uint32_t)GT, G - j0) : 0u; // heads of this workgroup
    constexpr uint32_t Qb = attn_quantum<HSP>();
    const int dc = lane % TPP;
    const bool dim_ok = (uint32_t)dc * 8 < hs;
    const uint32_t pg = (uint32_t)(wave * PPW + lane / TPP);
    const uint32_t h0 = kvh * G + j0; // first query head of the workgroup

    // this thread's 8 query dims of every head, loaded here without a
    // branch (a head past the workgroup's and a lane past the head size read
    // a valid head's last dims) and scaled, or zeroed, once the K and V loads
    // are out
    const uint32_t nq_heads = gridDim.x / a.n_sub * G;
    const uint32_t dq = min((uint32_t)dc, hs / 8 - 1) * 8;
    float4 qu[GT], qw[GT];
#pragma unroll
    for (int j = 0; j < GT; j++) {
        const float *qp = a.q + (size_t)min(h0 + (uint32_t)j, nq_heads - 1) * hs + dq;
        qu[j] = *(const float4 *)qp;
        qw[j] = *(const float4 *)(qp + 4);
    }

    // When S batches cover the host's bound on the positions (S * Qb >=
    // spec_rows), every chunk is one batch of Qb positions at s * Qb as long
    // as pos + 1 <= spec_rows: the first batch's K and V loads go out together
    // with the position load (rows clamped below spec_rows, masked below).  A
    // position past the bound falls back to chunks computed from it (the
    // early loads are then discarded).  The loads sit behind no branch (the
    // early batch is requested whatever the bound, and a lane past the head
    // size reads the head's last 8 dims, which meet its zero q and feed only
    // dims that are never stored): the compiler drains loads behind a branch
    // where the branches join, and the position could then be read only
    // after every K and V row had arrived.
    const bool early = S * Qb >= a.spec_rows;
    const size_t head_ld = (size_t)kvh * hs + (size_t)min((uint32_t)dc, hs / 8 - 1) * 8;
    KV8<F16> kr[ATTN_BATCH], vr[ATTN_BATCH];
    auto load_batch = [&](uint32_t t0, uint32_t base, uint32_t n) {
#pragma unroll
        for (int u = 0; u < ATTN_BATCH; u++) {
            const uint32_t tt = base + pg + PPP * u;
            const uint32_t row = n ? t0 + (tt < n ? tt : 0) : min(t0 + tt, min(a.spec_rows, a.seq_cap) - 1);
            const size_t off = (size_t)row * a.kv_dim + head_ld;
            kv8_load<F16>(a.k_cache, off, kr[u]);
            kv8_load<F16>(a.v_cache, off, vr[u]);
        }
    };
    load_batch(s * Qb, 0, 0);
    __builtin_amdgcn_sched_barrier(0); // the batch's loads stay together
    const float qs = 1.44269504088896341f / sqrtf((float)hs);
    float q[GT][8];
#pragma unroll
    for (int j = 0; j < GT; j++) {
        const float sj = (uint32_t)j < nj && dim_ok ? qs : 0.0f; // q is finite: 0 * q = 0
        const float4 u = qu[j], w = qw[j];
        q[j][0] = u.x * sj; q[j][1] = u.y * sj; q[j][2] = u.z * sj; q[j][3] = u.w * sj;
        q[j][4] = w.x * sj; q[j][5] = w.y * sj; q[j][6] = w.z * sj; q[j][7] = w.w * sj;
    }
    const uint32_t T = min((uint32_t)__builtin_amdgcn_readfirstlane(pos_dev) + 1u, a.seq_cap);
    const bool fixed = early && T <= a.spec_rows;
    const uint32_t C = fixed ? Qb : attn_chunk<HSP>(T, S);
    const uint32_t t0 = s * C;
    if (t0 >= T && (uint32_t)tid < nj) {
        // an empty split: a partial the merge gives weight 0
        a.part_ml[((size_t)(h0 + tid) * S + s) * 2] = -INFINITY;
        a.part_ml[((size_t)(h0 + tid) * S + s) * 2 + 1] = 0.0f;
    }
    const bool live = t0 < T;
    const uint32_t n = split_len(t0, C, T);

    float m[GT], l[GT], o[GT][8];
#pragma unroll
    for (int j = 0; j < GT; j++) {
        m[j] = ATTN_M0;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) o[j][e] = 0.0f;
    }

    for (uint32_t base = 0; base < n; base += PPP * U) {
        if (!fixed || base) load_batch(t0, base, n);
        __builtin_amdgcn_sched_barrier(0);
        if (base + PPP * U > n) { // (uniform) the batch runs past the split's positions
#pragma unroll
            for (int u = 0; u < U; u++)
                if (base + pg + PPP * u >= n) {
                    // a masked row (possibly never written): its values must not reach the sums
                    kv8_zero<F16>(vr[u]);
                }
        }
#pragma unroll
        for (int j = 0; j < GT; j++) {
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
            // mb is -inf when none of this thread's positions is valid: then
            // mn = m[j], al = 1 and every p = 0
            const float mn = fmaxf(m[j], mb);
            const float al = softmax_exp2(m[j] - mn); // 0 on the first valid batch
            float lsum = l[j] * al, ov[8];
#pragma unroll
            for (int e = 0; e < 8; e++) ov[e] = o[j][e] * al;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float p = softmax_exp2(sc[u] - mn); // 0 for a masked position
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
        for (int j = 0; j < GT; j++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                og[pg][j][dc * 4 + e] = o[j][e];
                og[pg][j][HSP / 2 + dc * 4 + e] = o[j][4 + e];
            }
            if (dc == 0) {
                mg[pg][j] = m[j];
                lg[pg][j] = l[j];
            }
        }
    }
    __syncthreads();
    if (live && tid < GT) {
        float M = -INFINITY;
        for (int g = 0; g < NPG; g++) M = fmaxf(M, mg[g][tid]);
        Mh[tid] = M;
    }
    __syncthreads();
    if (live)
        for (int i = tid; i < NPG * GT; i += ATTN_THREADS) {
            const int g = i / GT, j = i % GT;
            wg[g][j] = softmax_exp2(mg[g][j] - Mh[j]); // 0 for a group that saw no position (m = ATTN_M0)
        }
    __syncthreads();

    if (live)
        for (int i = tid; i < GT * HSP; i += ATTN_THREADS) {
            // consecutive threads read consecutive og words (word w, dim d)
            const uint32_t j = (uint32_t)i / HSP, w = (uint32_t)i % HSP, d = attn_og_dim<HSP>(w);
            if (j >= nj || d >= hs) continue;
            float v = 0.0f;
#pragma unroll
            for (int g = 0; g < NPG; g++) v = fmaf(wg[g][j], og[g][j][w], v);
            const size_t ph = (size_t)(h0 + j) * S + s;
            a.part_o[ph * hs + d] = v;
            if (d == 0) {
                float Ls = 0.0f;
#pragma unroll
                for (int g = 0; g < NPG; g++) Ls = fmaf(wg[g][j], lg[g][j], Ls);
                a.part_ml[ph * 2] = Mh[j];
                a.part_ml[ph * 2 + 1] = Ls;
            }
        }
}

// Merge of the split partials, one wave per 16 consecutive output values
// (element i of the n_heads * hs output is dim i % hs of query head i / hs):
// lane = (subset r = lane / 16, output 16c + lane % 16); subset r takes
// splits r, r + 4, ... in chunks of ATTN_MERGE_CHUNK whose loads are in
// flight together: the chunk's maximum first, then its weighted sums in four
// independent accumulators, folded into a running (M, L, O) with base-2
// weights (no chain of rescales through the chunk); then the four subsets
// combine through lane shuffles:
// out = sum_s 2^(m_s-M) o_s / sum_s 2^(m_s-M) l_s.  No LDS and no barrier.
// Every split of the launch is read (an empty one carries m = -inf and is
// skipped), so no load waits for the position.
constexpr uint32_t ATTN_MERGE_SUBSETS = 4;
constexpr uint32_t ATTN_MERGE_CHUNK = 24; // splits of a subset whose loads are in flight together

__device__ inline void attn_merge_body(const AttnArgs &a) {
    constexpr uint32_t NR = ATTN_MERGE_SUBSETS, CH = ATTN_MERGE_CHUNK;
    // the arguments in one batch of scalar loads (left to itself the compiler
    // reads the sizes, divides, and only then fetches the partials' addresses
    // from the other half of the argument block: two round trips before the
    // first load); an empty asm that emits nothing
    asm volatile("" ::"s"(a.part_o), "s"(a.part_ml), "s"(a.out), "s"(a.xq_out), "s"(a.n_splits), "s"(a.head_size),
                 "s"(a.n_out));
    const int lane = (int)threadIdx.x;
    const uint32_t hs = a.head_size, S = a.n_splits;
    const uint32_t r = (uint32_t)lane / 16, oi = blockIdx.x * 16 + (uint32_t)lane % 16;
    const bool in = oi < a.n_out;
    const uint32_t h = in ? oi / hs : 0, d = in ? oi % hs : 0;
    const float *po = a.part_o + (size_t)h * S * hs + d; // split t at po[t * hs]
    const float *pml = a.part_ml + (size_t)h * S * 2;    // split t at pml[t * 2]
    float M = ATTN_M0, L = 0.0f, O = 0.0f;
    for (uint32_t t0 = r; t0 < S; t0 += NR * CH) {
        float mv[CH], lv[CH], ov[CH];
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) {
            // loads from a split in range (a past-the-end slot rereads the
            // last split, then counts as empty), so no load sits behind a branch
            const uint32_t t = t0 + NR * u, tc = min(t, S - 1);
            const bool ok = t < S;
            const float mm = pml[(size_t)tc * 2], ll = pml[(size_t)tc * 2 + 1], oo = po[(size_t)tc * hs];
            mv[u] = ok ? mm : -INFINITY;
            lv[u] = ok ? ll : 0.0f;
            ov[u] = oo;
        }
        // the chunk's maximum (a pairwise tree), then its sums at that base
        float mx[CH];
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) mx[u] = mv[u];
#pragma unroll
        for (uint32_t w = 1; w < CH; w <<= 1)
#pragma unroll
            for (uint32_t u = 0; u + w < CH; u += 2 * w) mx[u] = fmaxf(mx[u], mx[u + w]);
        const float Mn = fmaxf(M, mx[0]); // at least ATTN_M0: finite
        float Ls[4] = {0.0f, 0.0f, 0.0f, 0.0f}, Os[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t u = 0; u < CH; u++) {
            // an empty split (m = -inf) weighs 0 and its o, never written, is not read into the sum
            const float b = softmax_exp2(mv[u] - Mn);
            Ls[u % 4] = fmaf(lv[u], b, Ls[u % 4]);
            Os[u % 4] = fmaf(mv[u] == -INFINITY ? 0.0f : ov[u], b, Os[u % 4]);
        }
        const float sc = softmax_exp2(M - Mn);
        L = fmaf(L, sc, (Ls[0] + Ls[1]) + (Ls[2] + Ls[3]));
        O = fmaf(O, sc, (Os[0] + Os[1]) + (Os[2] + Os[3]));
        M = Mn;
    }
    // the four subsets of each output: lanes i, i + 16, i + 32, i + 48
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        const float Mo = __shfl_xor(M, off, 64), Lo = __shfl_xor(L, off, 64), Oo = __shfl_xor(O, off, 64);
        const float Mn = fmaxf(M, Mo); // both at least ATTN_M0
        const float wa = softmax_exp2(M - Mn), wb = softmax_exp2(Mo - Mn);
        L = fmaf(Lo, wb, L * wa);
        O = fmaf(Oo, wb, O * wa);
        M = Mn;
    }
    const float res = O / L;
    const bool ok = lane < 16 && in;
    if (ok && a.out) a.out[oi] = res;
    if (a.xq_out) quant16(ok ? res : 0.0f, ok, a.xq_out, a.n_out, oi, lane);
}

} // namespace ifr

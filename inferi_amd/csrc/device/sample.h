// Token sampling on the device: Sampler::sample
// (crates/inferi/src/models/sampler.rs:32-131), so the logits never leave
// the device.  Up to four kernels:
//   sample_exp     many workgroups: partial sums of exp(y - max), y = logits / T;
//   sample_prob    many workgroups: probabilities out, and per chunk of 256
//                  (multinomial) or per level-0 bucket of the top-p candidates
//                  (probability bits 30..20) their mass and count, summed
//                  exactly in 64-bit integers;
//   sample_group   many workgroups (top-p only): the candidates' sort keys
//                  grouped by level-0 bucket (a counting sort);
//   sample_select  one workgroup: the choice, and the end of a decode step.
//
// The probabilities follow the reference's arithmetic step for step: the
// logits divided by the temperature (:38), exp(y - max) and each divided by
// the sum (SoftMax::run_cpu, crates/inferi/src/ops/softmax.rs:130-143); only
// the order of that sum differs (a fixed tree instead of a left-to-right
// loop).  The running sums the sampler compares with a threshold (the CDF
// walk of sample_mult :60-76; the truncation and the walk of sample_topp
// :83-131) are computed exactly, on the probabilities truncated to multiples
// of 2^-40 held as 64-bit integers, so a choice is deterministic and is the
// one the reference's algorithm makes with exact sums.  The reference's f32
// running sums drift from the exact ones by their own rounding; only a coin
// within that drift of a boundary can be decided differently.
//
// Top-p never sorts.  Its sorted order (probability descending, index
// ascending: the reference's stable sort, :101) is walked by weighted radix
// selection: the level-0 histogram locates the bucket where the running mass
// crosses the threshold, and within that bucket's group of keys two finer
// levels (bits 19..9, then 8..0) locate the probability; among equal
// probabilities the crossing is the k-th in ascending index, found by radix
// over the index bits.
#pragma once
#include "common.h"
#include "elementwise.h"

namespace ifr {

constexpr uint32_t SMP_THREADS = 1024; // sample_select
constexpr uint32_t SMP_WAVES = SMP_THREADS / 64;
constexpr uint32_t SMP_CHUNK = 256;
constexpr uint32_t SMP_MAX_CHUNKS = SAMPLE_MAX_N / SMP_CHUNK; // one per thread of sample_select
constexpr uint32_t SMP_CAP = 8192;                            // group keys held in LDS
constexpr uint32_t SMPG_THREADS = 256;                        // sample_exp / sample_prob / sample_group

// floor(p * 2^40) for 0 <= p < 2^23, from the bits (p * 2^40 is exact, the
// truncation drops the fraction).  Sums of 2^22 probabilities fit 64 bits.
IFR_DEV uint64_t prob_fx(float p) {
    const uint32_t u = __float_as_uint(p);
    const int32_t e = (int32_t)(u >> 23);
    if (e == 0 || (u >> 31)) return 0; // zero, subnormal (< 2^-126) or negative
    const uint64_t m = (u & 0x7FFFFFu) | 0x800000u;
    const int32_t sh = e - 110; // p * 2^40 = m * 2^(e - 127 - 23 + 40)
    return sh >= 0 ? m << sh : (sh > -64 ? m >> -sh : 0);
}

// Coin in [0, 1) drawn from (seed, position): 24 bits of mix64, the
// resolution of an f32 uniform.
IFR_DEV float seeded_coin(uint64_t seed, uint32_t pos) {
    const uint64_t r = mix64(seed + (uint64_t)pos * 0x9E3779B97F4A7C15ull);
    return (float)(uint32_t)(r >> 40) * (1.0f / 16777216.0f);
}

// Sort key of top-p: larger probability first, lower index first among equal
// probabilities.
IFR_DEV uint64_t smp_key(uint32_t bits, uint32_t i) { return ((uint64_t)bits << 32) | (uint64_t)(0xFFFFFFFFu - i); }
IFR_DEV uint64_t key_fx(uint64_t key) { return prob_fx(__uint_as_float((uint32_t)(key >> 32))); }
IFR_DEV uint32_t key_index(uint64_t key) { return 0xFFFFFFFFu - (uint32_t)key; }

IFR_DEV uint64_t wave_sum_u64(uint64_t v) {
    for (int sh = 32; sh >= 1; sh >>= 1) v += __shfl_xor(v, sh, 64);
    return v;
}
IFR_DEV uint64_t wave_max_u64(uint64_t v) {
    for (int sh = 32; sh >= 1; sh >>= 1) {
        const uint64_t o = __shfl_xor(v, sh, 64);
        v = o > v ? o : v;
    }
    return v;
}
IFR_DEV uint64_t wave_min_u64(uint64_t v) {
    for (int sh = 32; sh >= 1; sh >>= 1) {
        const uint64_t o = __shfl_xor(v, sh, 64);
        v = o < v ? o : v;
    }
    return v;
}
IFR_DEV uint64_t wave_incl_scan_u64(uint64_t v, uint32_t lane) {
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint64_t o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

// Four consecutive values from i (zero past n); v is 16-byte aligned.
IFR_DEV void smp_ld4(const float *v, uint32_t i, uint32_t n, float (&x)[4]) {
    if (i + 4 <= n) {
        const float4 t = *(const float4 *)(v + i);
        x[0] = t.x;
        x[1] = t.y;
        x[2] = t.z;
        x[3] = t.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) x[k] = i + k < n ? v[i + k] : 0.0f;
    }
}

// Scratch views (offsets in kargs.h).
IFR_DEV float *smpw_part(uint8_t *w) { return (float *)(w + SMPW_PART); }
IFR_DEV uint64_t *smpw_mass(uint8_t *w) { return (uint64_t *)(w + SMPW_MASS); }
IFR_DEV uint32_t *smpw_cnt(uint8_t *w) { return (uint32_t *)(w + SMPW_CNT); }
IFR_DEV uint64_t *smpw_chunk(uint8_t *w) { return (uint64_t *)(w + SMPW_CHUNK); }
IFR_DEV uint32_t *smpw_n0(uint8_t *w) { return (uint32_t *)(w + SMPW_N0); }
IFR_DEV uint64_t *smpw_kmin(uint8_t *w) { return (uint64_t *)(w + SMPW_KMIN); }
IFR_DEV uint32_t *smpw_cur(uint8_t *w) { return (uint32_t *)(w + SMPW_CUR); }
IFR_DEV uint64_t *smpw_keys(uint8_t *w) { return (uint64_t *)(w + SMPW_KEYS); }

IFR_DEV bool smp_nucleus(float topp) { return !(topp <= 0.0f || topp >= 1.0f); }               // sampler.rs:44
IFR_DEV float smp_cutoff(float topp, uint32_t n) { return (1.0f - topp) / ((float)n - 1.0f); } // sampler.rs:91

// Whether this decode step samples: not when the next token is forced
// (sample_next_token, crates/inferi-chat/src/sampler.rs:100-103) or the
// position is saturated.  Without a step, always.
IFR_DEV bool smp_active(const SampleArgs &a, uint32_t pos) {
    return !a.ctl || (pos + 1 < a.ctl->max_pos && pos + 1 >= a.ctl->n_forced);
}

// Largest argmax key of the part keys, to every thread of the workgroup:
// smp_key_load reads this thread's share (issue it with the kernel's other
// independent loads), smp_key_max reduces (wk: one entry per wave).
IFR_DEV uint64_t smp_key_load(const SampleArgs &a) {
    uint64_t k = 0;
    for (uint32_t i = threadIdx.x; i < a.n_parts; i += blockDim.x) k = a.part_keys[i] > k ? a.part_keys[i] : k;
    return k;
}
IFR_DEV uint64_t smp_key_max(const SampleArgs &a, uint64_t *wk, uint64_t k) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    k = wave_max_u64(k);
    if (lane == 0) wk[wave] = k;
    __syncthreads();
    for (uint32_t w = 0; w < nw; w++) k = wk[w] > k ? wk[w] : k;
    return k;
}
// max of y = logits / T from the largest key.
IFR_DEV float smp_ymax(const SampleArgs &a, uint64_t key) {
    const uint32_t ok = (uint32_t)(key >> 32);
    const float v = __uint_as_float((ok & 0x80000000u) ? (ok & 0x7FFFFFFFu) : ~ok);
    return a.keys_of_y ? v : v / a.temperature;
}

// ------------------------------------------------------------ sample_exp
// Workgroup g: the sum of exp(y - max) over elements [2048 g, 2048 g + 2048)
// in a fixed order; also clears the histograms and cursors the next kernels
// accumulate into.
IFR_DEV void sample_exp_body(const SampleArgs &a) {
    __shared__ uint64_t wk[SMPG_THREADS / 64];
    __shared__ float ws[SMPG_THREADS / 64];
    const uint32_t pos = a.ctl ? a.ctl->pos : 0;
    if (!smp_active(a, pos)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (uint32_t i = blockIdx.x * SMPG_THREADS + tid; i < 2048; i += gridDim.x * SMPG_THREADS) {
        smpw_mass(a.work)[i] = 0;
        smpw_cnt(a.work)[i] = 0;
        smpw_cur(a.work)[i] = 0;
    }
    if (blockIdx.x == 0 && tid == 0) {
        *smpw_n0(a.work) = 0;
        *smpw_kmin(a.work) = ~0ull;
    }
    const uint32_t n = a.n;
    float x[2][4];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++)
        smp_ld4(a.logits, blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2) + 4 * tid, n, x[h]);
    const float m = smp_ymax(a, smp_key_max(a, wk, smp_key_load(a)));
    const float T = a.temperature;
    float s = 0.0f;
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t i0 = blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2) + 4 * tid;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (i0 + k < n) s += expf(x[h][k] / T - m);
    }
    s = wave_sum(s);
    if (lane == 0) ws[wave] = s;
    __syncthreads();
    if (tid == 0) smpw_part(a.work)[blockIdx.x] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// ----------------------------------------------------------- sample_prob
// p = exp(y - max) / s over the same elements, s the sum of every
// workgroup's part in a fixed order (the same in every workgroup).
// Multinomial: the mass of each chunk of 256.  Top-p: the candidates'
// (p >= cutoff) mass and count per level-0 bucket, their number and the
// smallest candidate key (the last element of the sorted list).
IFR_DEV void sample_prob_body(const SampleArgs &a) {
    __shared__ uint64_t hm[2048];
    __shared__ uint32_t hc[2048];
    __shared__ uint64_t wk[SMPG_THREADS / 64];
    __shared__ uint32_t wn[SMPG_THREADS / 64];
    __shared__ float s_sh;
    const uint32_t pos = a.ctl ? a.ctl->pos : 0;
    if (!smp_active(a, pos)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n = a.n, G = gridDim.x;
    const float T = a.temperature;
    // independent loads first: the logits, the exp parts, the argmax keys
    float xx[2][4];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++)
        smp_ld4(a.logits, blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2) + 4 * tid, n, xx[h]);
    float v = 0.0f;
    if (wave == 0) { // G <= 128 parts
        const float *part = smpw_part(a.work);
        v = (lane < G ? part[lane] : 0.0f) + (lane + 64 < G ? part[lane + 64] : 0.0f);
    }
    const uint64_t k0 = smp_key_load(a);
    if (wave == 0) {
        v = wave_sum(v);
        if (lane == 0) s_sh = v;
    }
    const float m = smp_ymax(a, smp_key_max(a, wk, k0));
    const bool nucleus = smp_nucleus(a.topp);
    const float cutoff = smp_cutoff(a.topp, n);
    if (nucleus)
        for (uint32_t b = tid; b < 2048; b += SMPG_THREADS) {
            hm[b] = 0;
            hc[b] = 0;
        }
    __syncthreads();
    const float s = s_sh;
    uint32_t ncand = 0;
    uint64_t kmin = ~0ull;
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t i0 = blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2) + 4 * tid;
        float pr[4];
#pragma unroll
        for (int k = 0; k < 4; k++) pr[k] = i0 + k < n ? expf(xx[h][k] / T - m) / s : 0.0f;
        if (i0 + 4 <= n) {
            *(float4 *)(a.probs + i0) = make_float4(pr[0], pr[1], pr[2], pr[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (i0 + k < n) a.probs[i0 + k] = pr[k];
        }
        if (!nucleus) {
            // wave w covers chunk 8 g + 4 h + w
            const uint64_t cm = wave_sum_u64(prob_fx(pr[0]) + prob_fx(pr[1]) + prob_fx(pr[2]) + prob_fx(pr[3]));
            const uint32_t c = (blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2)) / SMP_CHUNK + wave;
            if (lane == 0) smpw_chunk(a.work)[c] = cm;
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (i0 + k < n && pr[k] >= cutoff) {
                    const uint32_t u = __float_as_uint(pr[k]);
                    atomicAdd(&hm[u >> 20], (unsigned long long)prob_fx(pr[k]));
                    atomicAdd(&hc[u >> 20], 1u);
                    ncand++;
                    const uint64_t key = smp_key(u, i0 + k);
                    kmin = key < kmin ? key : kmin;
                }
            }
        }
    }
    if (!nucleus) return;
    ncand = (uint32_t)wave_sum_u64(ncand);
    kmin = wave_min_u64(kmin);
    if (lane == 0) {
        wn[wave] = ncand;
        wk[wave] = kmin;
    }
    __syncthreads();
    for (uint32_t b = tid; b < 2048; b += SMPG_THREADS)
        if (hc[b]) {
            atomicAdd((unsigned long long *)&smpw_mass(a.work)[b], (unsigned long long)hm[b]);
            atomicAdd(&smpw_cnt(a.work)[b], hc[b]);
        }
    if (tid == 0) {
        const uint32_t nc = wn[0] + wn[1] + wn[2] + wn[3];
        uint64_t km = wk[0];
        for (uint32_t w = 1; w < SMPG_THREADS / 64; w++) km = wk[w] < km ? wk[w] : km;
        if (nc) {
            atomicAdd(smpw_n0(a.work), nc);
            atomicMin((unsigned long long *)smpw_kmin(a.work), (unsigned long long)km);
        }
    }
}

// ---------------------------------------------------------- sample_group
// Counting sort of the top-p candidates' keys by level-0 bucket: bucket b's
// keys fill smpw_keys[off(b), off(b) + count(b)), off(b) the number of
// candidates in higher buckets.  Each workgroup reserves one range per
// bucket it holds (a global cursor) and fills it in any order.
IFR_DEV void sample_group_body(const SampleArgs &a) {
    __shared__ uint32_t off[2048];
    __shared__ uint32_t lc[2048];
    __shared__ uint32_t wt[SMPG_THREADS / 64];
    const uint32_t pos = a.ctl ? a.ctl->pos : 0;
    if (!smp_active(a, pos) || !smp_nucleus(a.topp)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n = a.n;
    const float cutoff = smp_cutoff(a.topp, n);
    // off(b) = sum of the counts of buckets above b: thread t holds buckets
    // 2047 - 8t .. 2040 - 8t (descending), scanned across the workgroup
    // independent loads first: this workgroup's probabilities, the counts
    float pr[8];
    uint32_t ii[8];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t i0 = blockIdx.x * SAMPLE_GROUP_ELEMS + h * (SAMPLE_GROUP_ELEMS / 2) + 4 * tid;
        float x[4];
        smp_ld4(a.probs, i0, n, x);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            pr[4 * h + k] = x[k];
            ii[4 * h + k] = i0 + k;
        }
    }
    const uint32_t *cnt = smpw_cnt(a.work);
    uint32_t c8[8], run = 0;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        c8[q] = cnt[2047 - 8 * tid - q];
        run += c8[q];
    }
    uint32_t incl = run;
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) wt[wave] = incl;
    for (uint32_t b = tid; b < 2048; b += SMPG_THREADS) lc[b] = 0;
    __syncthreads();
    uint32_t ex = incl - run;
    for (uint32_t w = 0; w < wave; w++) ex += wt[w];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        off[2047 - 8 * tid - q] = ex;
        ex += c8[q];
    }
    // this workgroup's candidates per bucket
#pragma unroll
    for (int q = 0; q < 8; q++)
        if (ii[q] < n && pr[q] >= cutoff) atomicAdd(&lc[__float_as_uint(pr[q]) >> 20], 1u);
    __syncthreads();
    // reserve a range per bucket; lc becomes the fill cursor
    for (uint32_t b = tid; b < 2048; b += SMPG_THREADS)
        if (lc[b]) {
            off[b] += atomicAdd(&smpw_cur(a.work)[b], lc[b]);
            lc[b] = 0;
        }
    __syncthreads();
    uint64_t *keys = smpw_keys(a.work);
#pragma unroll
    for (int q = 0; q < 8; q++)
        if (ii[q] < n && pr[q] >= cutoff) {
            const uint32_t u = __float_as_uint(pr[q]);
            const uint32_t r = atomicAdd(&lc[u >> 20], 1u);
            keys[off[u >> 20] + r] = smp_key(u, ii[q]);
        }
}

// --------------------------------------------------------- sample_select

struct SmpLds {
    uint64_t h0[2048];            // level-0 histogram of candidate mass (bits 30..20)
    uint32_t c0[2048];            // level-0 candidate counts
    uint64_t h[2048];             // finer levels: masses, then index counts
    uint32_t cnt[512], mini[512]; // level 2: keys and smallest index per bucket
    uint64_t keys[SMP_CAP];       // the group being searched, when it fits
    uint64_t wtot[SMP_WAVES];
    uint64_t wkey[SMP_WAVES];
    int32_t win;
    uint64_t win_excl;
    uint32_t found_idx;
    uint32_t ctl_pos;
};

// Thread order is sequence order and thread t holds v.  Returns, to every
// thread, the first thread whose inclusive prefix sum exceeds t (-1: none),
// the prefix before it in excl and the sum of all in total.
IFR_DEV int32_t block_first_exceeding(SmpLds &L, uint64_t v, uint64_t t, uint64_t &excl, uint64_t &total) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t incl = wave_incl_scan_u64(v, lane);
    if (lane == 63) L.wtot[wave] = incl;
    if (tid == 0) L.win = -1;
    __syncthreads();
    uint64_t base = 0, tot = 0;
    for (uint32_t w = 0; w < SMP_WAVES; w++) {
        const uint64_t s = L.wtot[w];
        base += w < wave ? s : 0;
        tot += s;
    }
    incl += base;
    const uint64_t ex = incl - v;
    if (ex <= t && t < incl) { // at most one thread: the intervals are disjoint
        L.win = (int32_t)tid;
        L.win_excl = ex;
    }
    __syncthreads();
    const int32_t w = L.win;
    excl = L.win_excl;
    total = tot;
    __syncthreads(); // L.win and L.wtot are rewritten by the next call
    return w;
}

// Buckets h[0..nb) visited from the highest (desc) or the lowest: the first
// whose running sum, starting at `above` (<= t), exceeds t.  Returns it (-1:
// none) and leaves in `above` the sum before it (all of it when there is
// none).  nb <= 2048.
IFR_DEV int32_t smp_find_bucket(SmpLds &L, const uint64_t *h, uint32_t nb, uint64_t &above, uint64_t t,
                                bool desc = true) {
    auto at = [&](uint32_t d) { return desc ? nb - 1 - d : d; };
    const uint32_t d0 = 2 * threadIdx.x, d1 = d0 + 1;
    const uint64_t a0 = d0 < nb ? h[at(d0)] : 0, a1 = d1 < nb ? h[at(d1)] : 0;
    uint64_t ex, total;
    const int32_t w = block_first_exceeding(L, a0 + a1, t - above, ex, total);
    if (w < 0) {
        above += total;
        return -1;
    }
    const uint32_t e0 = 2 * (uint32_t)w;
    const uint64_t m0 = h[at(e0)];
    if (ex + m0 > t - above) {
        above += ex;
        return (int32_t)at(e0);
    }
    above += ex + m0;
    return (int32_t)at(e0 + 1);
}

// Sum over the workgroup of one value per thread (every thread gets it).
IFR_DEV uint64_t smp_block_sum(SmpLds &L, uint64_t v) {
    uint64_t ex, total;
    block_first_exceeding(L, v, ~0ull, ex, total);
    return total;
}

// Wave 0 scans chunk c with weights wt(p, i) and finds the element at which
// the running weight first exceeds t; every thread gets its index (`fallback`
// if no element does).
template <class Wt>
IFR_DEV uint32_t smp_locate(SmpLds &L, const float *p, uint32_t n, uint32_t c, uint64_t t, uint32_t fallback, Wt wt) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x, i0 = c * SMP_CHUNK + 4 * lane;
        float x[4];
        smp_ld4(p, i0, n, x);
        uint64_t w[4];
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = i0 + k < n ? wt(x[k], i0 + k) : 0;
        const uint64_t s = w[0] + w[1] + w[2] + w[3];
        const uint64_t incl = wave_incl_scan_u64(s, lane);
        const uint64_t ex = incl - s;
        const bool hit = ex <= t && t < incl;
        if (__ballot(hit) == 0) {
            if (lane == 0) L.found_idx = fallback;
        } else if (hit) {
            uint64_t run = ex;
            uint32_t j = 3;
            bool got = false;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                run += w[k];
                if (!got && run > t) {
                    j = (uint32_t)k;
                    got = true;
                }
            }
            L.found_idx = i0 + j;
        }
    }
    __syncthreads();
    const uint32_t r = L.found_idx;
    __syncthreads();
    return r;
}

// Copies the group seg[0..C) into L.keys when it fits.
IFR_DEV void smp_seg_load(SmpLds &L, const uint64_t *seg, uint32_t C) {
    if (C > SMP_CAP) return;
    for (uint32_t e = threadIdx.x; e < C; e += 4 * SMP_THREADS) {
        uint64_t k[4];
#pragma unroll
        for (int j = 0; j < 4; j++) k[j] = seg[min(e + j * SMP_THREADS, C - 1)];
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (e + j * SMP_THREADS < C) L.keys[e + j * SMP_THREADS] = k[j];
    }
    __syncthreads();
}

// Calls f(key) for every key of the group seg[0..C): from L.keys when it was
// copied there, else from global memory with four loads in flight per thread.
template <class F>
IFR_DEV void smp_seg_for(const SmpLds &L, const uint64_t *seg, uint32_t C, F &&f) {
    if (C <= SMP_CAP) {
        for (uint32_t e = threadIdx.x; e < C; e += SMP_THREADS) f(L.keys[e]);
        return;
    }
    for (uint32_t e = threadIdx.x; e < C; e += 4 * SMP_THREADS) {
        uint64_t k[4];
#pragma unroll
        for (int j = 0; j < 4; j++) k[j] = seg[min(e + j * SMP_THREADS, C - 1)];
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (e + j * SMP_THREADS < C) f(k[j]);
    }
}

// Within the group seg[0..C) of level-0 bucket b0 (its candidates' keys, in
// any order): the element of the sorted list (probability desc, index asc)
// at which the running mass, starting at `above` (the mass of the higher
// buckets), first exceeds t, counting only keys >= bound (the list up to
// and including the key `bound`; 0: all).  Returns its key (0 if none; the
// callers pass a group that holds the crossing) and the running mass there.
IFR_DEV uint64_t smp_select_group(SmpLds &L, const uint64_t *seg, uint32_t C, uint32_t b0, uint64_t above, uint64_t t,
                                  uint64_t bound, uint64_t &cum) {
    const uint32_t tid = threadIdx.x;
    smp_seg_load(L, seg, C);
    // level 1: bits 19..9
    for (uint32_t b = tid; b < 2048; b += SMP_THREADS) L.h[b] = 0;
    __syncthreads();
    smp_seg_for(L, seg, C, [&](uint64_t key) {
        if (key >= bound) atomicAdd(&L.h[(uint32_t)(key >> 41) & 0x7FFu], (unsigned long long)key_fx(key));
    });
    __syncthreads();
    const int32_t b1 = smp_find_bucket(L, L.h, 2048, above, t);
    if (b1 < 0) return 0;
    // level 2: bits 8..0, with key counts and the smallest index
    for (uint32_t b = tid; b < 512; b += SMP_THREADS) {
        L.h[b] = 0;
        L.cnt[b] = 0;
        L.mini[b] = 0xFFFFFFFFu;
    }
    __syncthreads();
    smp_seg_for(L, seg, C, [&](uint64_t key) {
        const uint32_t u = (uint32_t)(key >> 32);
        if (key >= bound && ((u >> 9) & 0x7FFu) == (uint32_t)b1) {
            const uint32_t d = u & 0x1FFu;
            atomicAdd(&L.h[d], (unsigned long long)key_fx(key));
            atomicAdd(&L.cnt[d], 1u);
            atomicMin(&L.mini[d], key_index(key));
        }
    });
    __syncthreads();
    const int32_t b2 = smp_find_bucket(L, L.h, 512, above, t);
    if (b2 < 0) return 0;
    const uint32_t v = (b0 << 20) | ((uint32_t)b1 << 9) | (uint32_t)b2;
    const uint64_t w = prob_fx(__uint_as_float(v));
    if (w == 0) return 0;
    // the keys with probability bits v each add w: the running mass first
    // exceeds t at the k-th of them (from 0) in ascending index
    const uint64_t k = (t - above) / w;
    const uint32_t count = L.cnt[b2], first = L.mini[b2];
    uint32_t idx = first;
    if (count != 1) {
        // radix over the index: bits 17..9, then 8..0 (indices < 2^18)
        uint64_t below = 0;
        int32_t ia = -1, ib = -1;
        for (int lvl = 0; lvl < 2; lvl++) {
            for (uint32_t b = tid; b < 512; b += SMP_THREADS) L.h[b] = 0;
            __syncthreads();
            smp_seg_for(L, seg, C, [&](uint64_t key) {
                const uint32_t i = key_index(key);
                if (key >= bound && (uint32_t)(key >> 32) == v && (lvl == 0 || (i >> 9) == (uint32_t)ia))
                    atomicAdd(&L.h[lvl == 0 ? i >> 9 : i & 0x1FFu], 1ull);
            });
            __syncthreads();
            (lvl == 0 ? ia : ib) = smp_find_bucket(L, L.h, 512, below, k, false);
            if ((lvl == 0 ? ia : ib) < 0) return 0;
        }
        idx = ((uint32_t)ia << 9) | (uint32_t)ib;
    }
    cum = above + (k + 1) * w;
    return smp_key(v, idx);
}

IFR_DEV void sample_select_body(const SampleArgs &a) {
    __shared__ SmpLds L;
    const uint32_t tid = threadIdx.x;

    const uint32_t n = a.n, nch = (n + SMP_CHUNK - 1) / SMP_CHUNK;
    const bool nucleus = smp_nucleus(a.topp);
    // every independent load first: the position, the coin, the argmax keys,
    // the chunk masses or the level-0 histograms
    if (tid == 0 && a.ctl) L.ctl_pos = a.ctl->pos;
    const float dev_coin = a.coin ? *a.coin : 0.0f;
    const uint64_t k0 = smp_key_load(a);
    uint64_t cm = 0, n0 = 0, kmin = 0;
    if (!nucleus) {
        cm = tid < nch ? smpw_chunk(a.work)[tid] : 0;
    } else {
        for (uint32_t b = tid; b < 2048; b += SMP_THREADS) {
            L.h0[b] = smpw_mass(a.work)[b];
            L.c0[b] = smpw_cnt(a.work)[b];
        }
        n0 = *smpw_n0(a.work);
        kmin = *smpw_kmin(a.work);
    }
    __syncthreads();
    uint32_t pos = 0;
    if (a.ctl) {
        pos = L.ctl_pos;
        if (pos + 1 >= a.ctl->max_pos) return; // saturated: step_advance does nothing either
        if (pos + 1 < a.ctl->n_forced) {
            if (tid == 0) step_advance(a.ctl, a.tokens, a.rope_pos, a.attn_pos, pos, 0);
            return;
        }
    }
    float coin = a.coin ? dev_coin : seeded_coin(a.seed, pos + 1);
    coin = fminf(fmaxf(coin, 0.0f), 0x1.fffffep-1f); // [0, 1); NaN -> 0
    const uint32_t amax = key_index(smp_key_max(a, L.wkey, k0));
    __syncthreads();

    uint32_t idx;
    if (!nucleus) {
        // sample_mult (:60-76): the first index whose running mass exceeds
        // the coin, n - 1 if none does
        const uint64_t cfx = prob_fx(coin);
        uint64_t ex, total;
        const int32_t c = block_first_exceeding(L, cm, cfx, ex, total);
        idx = c < 0 ? n - 1
                    : smp_locate(L, a.probs, n, (uint32_t)c, cfx - ex, n - 1,
                                 [](float x, uint32_t) -> uint64_t { return prob_fx(x); });
    } else {
        const uint64_t *keys = smpw_keys(a.work);
        // the group of bucket b starts after the candidates of higher buckets
        auto group = [&](int32_t b) {
            uint64_t v = 0;
            for (uint32_t q = (uint32_t)b + 1 + 2 * tid; q < (uint32_t)b + 3 + 2 * tid; q++) v += q < 2048 ? L.c0[q] : 0;
            return keys + smp_block_sum(L, v);
        };
        if (n0 == 0) {
            // no probability reaches the cutoff: the reference's sample_topp
            // has nothing to sort and fails; take the most probable token
            idx = amax;
        } else {
            // sample_topp (:83-131): truncate where the running mass of the
            // sorted candidates exceeds topp (or keep them all: the last
            // candidate, kmin) ...
            const uint64_t tfx = prob_fx(a.topp);
            uint64_t above1 = 0;
            const int32_t b1 = smp_find_bucket(L, L.h0, 2048, above1, tfx);
            uint64_t lkey = kmin, cum = above1;
            if (b1 >= 0) {
                const uint64_t *g = group(b1);
                lkey = smp_select_group(L, g, L.c0[b1], (uint32_t)b1, above1, tfx, 0, cum);
                if (!lkey) { // cannot happen: the bucket holds the crossing
                    lkey = kmin;
                    cum = smp_block_sum(L, L.h0[2 * tid] + L.h0[2 * tid + 1]);
                }
            }
            // ... then the first element of the truncated list whose running
            // mass exceeds coin * cumulative mass (the last one if none does)
            const uint64_t rfx = (uint64_t)((double)coin * (double)cum);
            const int32_t bl = (int32_t)(lkey >> 52); // the truncation point's bucket
            for (uint32_t q = tid; q < 2048; q += SMP_THREADS) { // level-0 masses of the truncated list
                if ((int32_t)q < bl) L.h0[q] = 0;
                else if ((int32_t)q == bl && b1 >= 0) L.h0[q] = cum - above1;
            }
            __syncthreads();
            uint64_t above2 = 0;
            const int32_t b2 = smp_find_bucket(L, L.h0, 2048, above2, rfx);
            idx = key_index(lkey);
            if (b2 >= 0) {
                const uint64_t *g = group(b2);
                uint64_t c2;
                const uint64_t key2 = smp_select_group(L, g, L.c0[b2], (uint32_t)b2, above2, rfx, lkey, c2);
                if (key2) idx = key_index(key2);
            }
        }
    }

    if (tid == 0) {
        idx = idx < n ? idx : n - 1; // every path yields an element index; never store one past the vocabulary
        if (a.out_index) *a.out_index = idx;
        if (a.ctl) step_advance(a.ctl, a.tokens, a.rope_pos, a.attn_pos, pos, idx);
    }
}

} // namespace ifr

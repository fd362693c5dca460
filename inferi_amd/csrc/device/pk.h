// Persistent layer tail: the GEMV stages between two attentions of a decode
// step (Llama2::launch, crates/inferi/src/models/llama2/transformer.rs:
// 446-469, then :418-445 of the next layer) in ONE launch of one workgroup
// per CU, the stages separated by grid barriers instead of kernel
// boundaries:
//   mode 1:  O (+residual) | gate/up (+SiLU) | down (+residual) | next QKV (+RoPE, +KV store)
//   mode 0:  embedding | QKV of layer 0
// Attention and its merge stay kernels of their own between the launches.
//
// Why: at batch 1 every stage is a short, bandwidth-bound pass, and a kernel
// boundary costs its ramp-up and drain each time.  Here the next stage's
// weights are requested before the grid barrier resolves, so HBM keeps
// streaming across the stage boundary.
//
// Workgroup: PK_WAVES waves.  Wave 0 controls: it runs the stage epilogues
// (RoPE and the KV-cache store, residual adds, SiLU, quantization of the
// next stage's input), writes every output and drives the barrier.  Waves
// 1.. compute the GEMV items.  The stages do the fused kernels' arithmetic
// in their reduction orders, so the results equal theirs bit for bit.
//
// Visibility between workgroups: every value another workgroup reads in the
// same launch is written with agent-scope atomic stores (written through to
// the device-coherent level) into a buffer no workgroup has read earlier in
// the launch, and read after the grid barrier with plain loads.  Before
// arriving, a workgroup waits for its stores to complete (vmcnt 0).  Weights
// are read-only.
//
// The barrier: the last arriver of each of the 8 workgroup classes
// (blockIdx mod 8, one per XCD when workgroups are dealt round robin)
// increments the global counter; every workgroup polls that one.  Counters
// only grow.  A launch reads the epoch word (barriers of earlier launches) at
// its start and waits for epoch + k + 1 rounds at its k-th barrier; after the
// first barrier (when every workgroup has read it) workgroup 0 advances the
// epoch by this launch's barrier count.  Every wait is bounded; a barrier that
// gives up raises the error word, and a launch that finds it raised does
// nothing.  The grid never exceeds what the CUs hold at once (the host checks
// the occupancy), so every workgroup is resident.
#pragma once
#include "attention.h"
#include "elementwise.h"

namespace ifr {

constexpr uint32_t PK_CW = PK_WAVES - 1;          // compute waves
constexpr uint32_t PK_THREADS = PK_WAVES * 64;
constexpr uint32_t PK_SPIN_MAX = 1u << 21;        // polls (with a short sleep) before a barrier gives up

// Row geometry of one GEMV stage.  A unit is GU virtual rows: one RoPE pair
// for QKV, one 16-value output group for RESID (16 rows) and GATEUP (16
// gate/up pairs, 32 virtual rows).  Units are dealt to workgroups in
// contiguous ranges; an item is one row pair times one 64-lane K step.
struct PkGemv {
    const uint8_t *w0, *w1, *w2;
    uint32_t rows0, rows1, total_rows, cols, nb, row_bytes, steps, gu, u0, u1;
    IFR_DEV uint32_t items() const { return (u1 - u0) * (gu / 2) * steps; }
};

template <int MODE>
IFR_DEV const uint8_t *pk_row_ptr(const PkGemv &g, uint32_t v) {
    if constexpr (MODE == GEMV_QKV) {
        if (v < g.rows0) return g.w0 + (size_t)v * g.row_bytes;
        v -= g.rows0;
        if (v < g.rows1) return g.w1 + (size_t)v * g.row_bytes;
        return g.w2 + (size_t)(v - g.rows1) * g.row_bytes;
    } else if constexpr (MODE == GEMV_GATEUP) {
        return ((v & 1u) ? g.w1 : g.w0) + (size_t)(v >> 1) * g.row_bytes;
    } else {
        return g.w0 + (size_t)v * g.row_bytes;
    }
}

template <int FMT>
struct Pk {
    using CH = ChunkI<FMT, 2>;
    static constexpr int LPB = CH::LPB, BPI = 64 / LPB;

    const PkArgs &a;
    uint8_t *lds;
    const int tid, lane;
    const uint32_t wave, b, nwg;
    uint32_t epoch = 0; // barriers of earlier launches
    uint32_t nbar = 0;  // barriers passed in this launch
    uint32_t pos = 0;
    float rs = 1.0f;    // wave 0: RMSNorm scale of the staged input
    CH A, B;            // the compute waves' weight buffers

    IFR_DEV Pk(const PkArgs &args, uint8_t *l)
        : a(args), lds(l), tid((int)threadIdx.x), lane((int)threadIdx.x & 63),
          wave(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)), b(blockIdx.x), nwg(gridDim.x) {}

    IFR_DEV uint32_t xq_off_part() const { return pk_xq_region(max(a.hidden, a.ffn)); }
    IFR_DEV float *part() const { return (float *)(lds + xq_off_part()); } // [PK_PART_ROWS][PK_KSTEPS]

    // ------------------------------------------------------------ barrier
    IFR_DEV bool failed() const { return __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0; }

    // Arrival of this workgroup (thread 0; the caller made every thread's
    // stores complete and synchronised the workgroup).
    IFR_DEV void arrive() {
        const uint32_t x = b % 8u, per = (nwg + 7u - x) / 8u;
        const uint32_t k = epoch + nbar + 1u;
        const uint32_t old =
            __hip_atomic_fetch_add(a.bar + PK_BAR_CLASS + PK_BAR_CLASS * x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1u == k * per) __hip_atomic_fetch_add(a.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    IFR_DEV void wait_all() {
        const uint32_t target = (epoch + nbar + 1u) * min(nwg, 8u);
        uint32_t n = 0;
        while (__hip_atomic_load(a.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++n > PK_SPIN_MAX) {
                __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((n & 255u) == 0 && failed()) break; // another workgroup gave up: do not wait out every barrier
            __builtin_amdgcn_s_sleep(2);
        }
    }

    // The boundary after a stage's items.  The compute waves store nothing
    // (wave 0 writes every output), so once the items' sums are in LDS they
    // request the next stage's first items (pf); wave 0 runs the stage's
    // epilogue (epi) meanwhile, waits
    // for its stores, arrives and waits for every workgroup, then stages
    // the next stage's input into LDS by itself (st: its loads do not queue
    // behind the prefetch, since a wave's loads return in order).
    template <typename PF, typename EPI, typename ST>
    IFR_DEV void stage_boundary(PF &&pf, EPI &&epi, ST &&stage, uint32_t n_total) {
        __syncthreads();
        stamp(4 * nbar + 2);
        // (issuing the prefetch can stall while the memory pipeline is
        // full: the epilogue runs meanwhile)
        if (wave != 0) pf();
        if (wave == 0) {
            epi();
            stamp(4 * nbar + 3);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (lane == 0) {
                arrive();
                wait_all();
                // every workgroup has read the epoch: advance it for the next launch
                if (nbar == 0 && b == 0)
                    __hip_atomic_store(a.bar + PK_BAR_EPOCH, epoch + n_total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            stamp(4 * nbar + 4);
            stage();
        }
        nbar++;
        __syncthreads();
        stamp(4 * nbar + 1);
    }

    // ------------------------------------------------------------ GEMV
    // units of a stage dealt to this workgroup
    IFR_DEV PkGemv with_units(PkGemv g) const {
        const uint32_t units = g.total_rows / g.gu;
        g.u0 = b * units / nwg;
        g.u1 = (b + 1) * units / nwg;
        g.steps = (g.nb + BPI - 1) / BPI;
        return g;
    }
    IFR_DEV PkGemv desc_qkv() const {
        PkGemv g{};
        g.w0 = a.wq; g.w1 = a.wk; g.w2 = a.wv;
        g.rows0 = a.hidden; g.rows1 = a.kv_dim;
        g.total_rows = a.hidden + 2 * a.kv_dim;
        g.gu = 2;
        g.cols = a.hidden; g.nb = a.nb_h; g.row_bytes = a.rb_h;
        return with_units(g);
    }
    IFR_DEV PkGemv desc_o() const {
        PkGemv g{};
        g.w0 = a.wo;
        g.total_rows = a.hidden;
        g.gu = 16;
        g.cols = a.hidden; g.nb = a.nb_h; g.row_bytes = a.rb_h;
        return with_units(g);
    }
    IFR_DEV PkGemv desc_gateup() const {
        PkGemv g{};
        g.w0 = a.wg; g.w1 = a.wu;
        g.total_rows = 2 * a.ffn;
        g.gu = 32;
        g.cols = a.hidden; g.nb = a.nb_h; g.row_bytes = a.rb_h;
        return with_units(g);
    }
    IFR_DEV PkGemv desc_down() const {
        PkGemv g{};
        g.w0 = a.wd;
        g.total_rows = a.hidden;
        g.gu = 16;
        g.cols = a.ffn; g.nb = a.nb_f; g.row_bytes = a.rb_f;
        return with_units(g);
    }

    // weights of item i (clamped into the stage, so every load is valid)
    template <int MODE>
    IFR_DEV void load_item(CH &w, const PkGemv &g, uint32_t i) const {
        const uint32_t n = g.items();
        i = min(i, n - 1u);
        const uint32_t st = i % g.steps, pr = i / g.steps;
        const uint32_t v0 = g.u0 * g.gu + 2u * pr;
        const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
        const uint32_t kb = min(st * BPI + bsub, g.nb - 1u);
        const uint8_t *rowp[2] = {pk_row_ptr<MODE>(g, min(v0, g.total_rows - 1u)),
                                  pk_row_ptr<MODE>(g, min(v0 + 1u, g.total_rows - 1u))};
        w.load(rowp, kb, c);
    }
    // the compute wave's first two items, requested ahead of the stage
    template <int MODE>
    IFR_DEV void prefetch(const PkGemv &g) {
        if (g.items() == 0) return;
        const uint32_t cw = wave - 1u;
        load_item<MODE>(A, g, cw);
        load_item<MODE>(B, g, cw + PK_CW);
    }

    // Wave 0: the input XQ of K values into LDS with LDS-direct loads (1 KB
    // per instruction, none waits on another; the last chunk's lanes past
    // the end re-read the last 16 bytes, the LDS region is whole KBs), and
    // for a normalising stage the RMSNorm scale from the n_ss partial sums
    // of x^2.
    IFR_DEV void stage_xq(const uint8_t *src, uint32_t K, const float *ss, uint32_t n_ss) {
        const uint32_t n16 = xq_bytes(K) / 16, nk = (n16 + 63) / 64;
        const uint4 *s4 = (const uint4 *)src;
        for (uint32_t k = 0; k < nk; k++)
            __builtin_amdgcn_global_load_lds((const void *)(s4 + min(k * 64 + (uint32_t)lane, n16 - 1)),
                                             (__attribute__((address_space(3))) void *)(lds + k * 1024), 16, 0, 0);
        rs = 1.0f;
        if (ss) {
            // the order of gemv_int_body's prologue
            constexpr uint32_t SC = 4;
            float sv[SC];
            const uint32_t last = n_ss - 1u;
#pragma unroll
            for (uint32_t j = 0; j < SC; j++) sv[j] = ss[min((uint32_t)lane + 64 * j, last)];
            float t = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < SC; j++) t += (uint32_t)lane + 64 * j < n_ss ? sv[j] : 0.0f;
            for (uint32_t i = (uint32_t)lane + 64 * SC; i < n_ss; i += 64) t += ss[i];
            t = wave_sum(t);
            rs = 1.0f / sqrtf(t / (float)K + a.eps); // rms_norm.rs:115
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // Compute waves: every item, partial row sums into LDS part[row][step].
    // The two buffers alternate; each item's successor is requested before
    // the other buffer's item is computed.
    template <int MODE>
    IFR_DEV void gemv_items(const PkGemv &g) {
        const uint32_t n = g.items();
        if (wave == 0 || n == 0) return;
        const uint32_t cw = wave - 1u, c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
        const XQ xq(lds, g.cols);
        float *pt = part();
        auto compute = [&](const CH &w, uint32_t i) {
            const uint32_t st = i % g.steps, pr = i / g.steps;
            const uint32_t kb = st * BPI + bsub;
            float acc[2] = {0.0f, 0.0f};
            chunk_step<FMT, 2>(w, xq, min(kb, g.nb - 1u), c, kb < g.nb, acc);
            acc[0] = wave_sum(acc[0]);
            acc[1] = wave_sum(acc[1]);
            if (lane == 0) {
                pt[(2 * pr) * PK_KSTEPS + st] = acc[0];
                pt[(2 * pr + 1) * PK_KSTEPS + st] = acc[1];
            }
        };
        for (uint32_t i = cw; i < n; i += 2 * PK_CW) {
            compute(A, i);
            load_item<MODE>(A, g, i + 2 * PK_CW);
            __builtin_amdgcn_sched_barrier(0);
            if (i + PK_CW >= n) break;
            compute(B, i + PK_CW);
            load_item<MODE>(B, g, i + 3 * PK_CW);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // row value after the K steps, in the fused kernels' order (slices in
    // order, then the RMSNorm scale)
    IFR_DEV float row_val(const PkGemv &g, uint32_t lr) const {
        const float *pt = part();
        float t = pt[lr * PK_KSTEPS];
        for (uint32_t k = 1; k < g.steps; k++) t += pt[lr * PK_KSTEPS + k];
        return t * rs;
    }

    // wave 0 after the items: QKV outputs (RoPE; q, and k, v into the cache
    // row of this position)
    IFR_DEV void epi_qkv(const PkGemv &g) {
        const uint32_t npairs = g.u1 - g.u0;
        for (uint32_t p = (uint32_t)lane; p < npairs; p += 64) {
            const uint32_t v = (g.u0 + p) * 2u;
            float x0 = row_val(g, 2 * p), x1 = row_val(g, 2 * p + 1);
            if (v < g.rows0) {
                rope_pair(x0, x1, v, a.head_size, pos, a.rope_tab);
                st_out<true>(a.q + v, x0);
                st_out<true>(a.q + v + 1, x1);
            } else {
                const bool is_k = v < g.rows0 + g.rows1;
                const uint32_t idx = is_k ? v - g.rows0 : v - g.rows0 - g.rows1;
                if (is_k) rope_pair(x0, x1, idx, a.head_size, pos, a.rope_tab);
                const size_t off = (size_t)pos * a.kv_dim + idx;
                void *cache = is_k ? a.kc : a.vc;
                if (a.kv_f16) {
                    const uint32_t packed = (uint32_t)f32_to_f16(x0) | ((uint32_t)f32_to_f16(x1) << 16);
                    st_out<true>((uint32_t *)((uint16_t *)cache + off), packed);
                } else {
                    st_out<true>((float *)cache + off, x0);
                    st_out<true>((float *)cache + off + 1, x1);
                }
            }
        }
    }
    // wave 0: x_out = x_in + W v; x_out * gamma_next quantized, partial sums of x_out^2
    IFR_DEV void epi_resid(const PkGemv &g, const float *x_in, float *x_out, const float *gamma_next, uint8_t *xq_out,
                           float *ss_out) {
        const uint32_t nu = g.u1 - g.u0;
        for (uint32_t u = (uint32_t)lane / 16; u < ((nu + 3u) & ~3u); u += 4) {
            const uint32_t l16 = (uint32_t)lane & 15u, unit = g.u0 + u, v = unit * 16 + l16;
            const bool ok = u < nu;
            float xn = 0.0f, gn = 1.0f;
            if (ok) {
                xn = x_in[v] + row_val(g, u * 16 + l16);
                st_out<true>(x_out + v, xn);
                if (gamma_next) gn = gamma_next[v];
            }
            quant16<true>(xn * gn, ok, xq_out, g.total_rows, v, lane);
            const float sq = sum16(xn * xn);
            if (ok && l16 == 0) st_out<true>(ss_out + unit, sq);
        }
    }
    // wave 0: h = up * silu(gate), quantized
    IFR_DEV void epi_gateup(const PkGemv &g) {
        const uint32_t nu = g.u1 - g.u0, K = g.total_rows / 2;
        for (uint32_t u = (uint32_t)lane / 16; u < ((nu + 3u) & ~3u); u += 4) {
            const uint32_t l16 = (uint32_t)lane & 15u, v = (g.u0 + u) * 16 + l16;
            const bool ok = u < nu;
            float h = 0.0f;
            if (ok) {
                const float gt = row_val(g, u * 32 + 2 * l16), up = row_val(g, u * 32 + 2 * l16 + 1);
                h = up * (gt / (1.0f + expf(-gt)));
            }
            quant16<true>(h, ok, a.xq_h, K, v, lane);
        }
    }

    // x = token_embd[token] (embed_body's arithmetic: 256 elements per
    // workgroup of the first ceil(hidden/256), partial sums per 256)
    IFR_DEV void embed() {
        float *red = (float *)lds;
        const uint32_t tok = a.tokens[pos];
        const uint8_t *row = a.table + (size_t)tok * a.emb_row_bytes;
        const uint32_t i = b * 256u + (uint32_t)tid;
        const bool mine = tid < 256 && b * 256u < a.hidden;
        const bool ok = mine && i < a.hidden;
        if (mine) {
            const float v = ok ? deq_elem(a.emb_fmt, row, i) : 0.0f;
            if (ok) st_out<true>(a.x + i, v);
            quant16<true>(v * (ok ? a.emb_gamma[i] : 0.0f), ok, a.xq_a, a.hidden, i, lane);
            const float sq = wave_sum(v * v);
            if (lane == 0) red[wave] = sq;
        }
        __syncthreads();
        if (mine && tid == 0) st_out<true>(a.ss_a + b, (red[0] + red[1]) + (red[2] + red[3]));
    }

    // stage timeline (workgroup thread 0), when the host asks for it
    IFR_DEV void stamp(uint32_t e) {
        if (a.ts && tid == 0) a.ts[b * PK_TS_EVENTS + e] = __builtin_amdgcn_s_memrealtime();
    }

    IFR_DEV void qkv_stage(const PkGemv &g) {
        gemv_items<GEMV_QKV>(g);
        __syncthreads();
        stamp(14);
        if (wave == 0) epi_qkv(g);
        stamp(15);
    }

    IFR_DEV void run() {
        if (failed()) return;
        epoch = a.bar[PK_BAR_EPOCH];
        pos = a.ctl->pos;
        const bool has_qkv = a.wq != nullptr;
        auto none = [] {};
        if (a.mode == 0) {
            const PkGemv gq = desc_qkv();
            embed();
            // the embedding's stores are every storing wave's: complete before the arrival
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            stage_boundary([&] { prefetch<GEMV_QKV>(gq); }, none,
                           [&] { stage_xq(a.xq_a, a.hidden, a.ss_a, a.n_ss_a); }, 1u);
            qkv_stage(gq);
            return;
        }
        const uint32_t n_total = has_qkv ? 3u : 2u;
        stamp(0);
        const PkGemv go = desc_o();
        // O: its input comes from the previous kernel
        if (wave != 0) prefetch<GEMV_RESID>(go);
        else stage_xq(a.xq_att, a.hidden, nullptr, 0);
        __syncthreads();
        stamp(1);
        gemv_items<GEMV_RESID>(go);
        const PkGemv gg = desc_gateup();
        stage_boundary([&] { prefetch<GEMV_GATEUP>(gg); },
                       [&] { epi_resid(go, a.x, a.x_mid, a.ffn_norm, a.xq_f, a.ss_f); },
                       [&] { stage_xq(a.xq_f, a.hidden, a.ss_f, a.hidden / 16); }, n_total);
        gemv_items<GEMV_GATEUP>(gg);
        const PkGemv gd = desc_down();
        stage_boundary([&] { prefetch<GEMV_RESID>(gd); }, [&] { epi_gateup(gg); },
                       [&] { stage_xq(a.xq_h, a.ffn, nullptr, 0); }, n_total);
        gemv_items<GEMV_RESID>(gd);
        if (has_qkv) {
            const PkGemv gq = desc_qkv();
            stage_boundary([&] { prefetch<GEMV_QKV>(gq); },
                           [&] { epi_resid(gd, a.x_mid, a.x, a.next_norm, a.xq_a, a.ss_a); },
                           [&] { stage_xq(a.xq_a, a.hidden, a.ss_a, a.hidden / 16); }, n_total);
            qkv_stage(gq);
        } else {
            __syncthreads();
            if (wave == 0) epi_resid(gd, a.x_mid, a.x, a.next_norm, a.xq_a, a.ss_a);
        }
    }
};

template <int FMT>
__device__ void pk_tail_body(const PkArgs &a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t pk_lds[];
    Pk<FMT> k(a, pk_lds);
    k.run();
}

} // namespace ifr

// Dequant-fused GEMV for GGUF blocks on gfx950 (HBM-bound; no MFMA).
//
// Work mapping.  A workgroup is 4 waves of 64 lanes; each wave owns R = 4
// consecutive rows and sweeps the whole K range of those rows, so the x
// values a lane reads from LDS are reused for 4 rows.  Within a wave, a block
// is split over LPB lanes (8 for the 256-element K-quants, so a lane owns one
// 16-byte quant chunk = 32 elements; 2 for Q8_0) and a wave covers 64/LPB
// consecutive blocks per step; every lane issues its R rows' 16-byte loads
// before it touches them.  Partial dots are combined with a DPP butterfly.
// The activation vector is staged in LDS once per workgroup (optionally
// RMS-normalised on the way in), and the workgroups walk row tiles with a
// grid stride so the launch can be sized to the chip.
//
// Arithmetic.  Per 32-element chunk the unsigned quant codes q are
// dotted with x in fp32 and the block scales are applied afterwards:
//   sum_e (d1*q_e - m1) x_e = d1 * sum_e q_e x_e - m1 * sum_e x_e,
// the refactoring the reference kernels use too
// (inferi-shaders/src/gemv_quant_q4_k.rs:47-93).  Accumulation is fp32.
#pragma once
#include "common.h"

namespace ifr {

constexpr int GEMV_R = 4;      // rows per wave
constexpr int GEMV_WAVES = 4;  // waves per workgroup

// Scale/min pair for sub-blocks 2g and 2g+1 of a Q4_K/Q5_K block, branch-free
// (get_scale_min_k4, crates/inferi/src/quantization.rs:394-402).
IFR_DEV void scale_min_pair(uint32_t g, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t &sc0, uint32_t &m0,
                            uint32_t &sc1, uint32_t &m1) {
    uint32_t sh = 16u * (g & 1u);
    if (g < 2) {
        sc0 = (w0 >> sh) & 63u;
        m0 = (w1 >> sh) & 63u;
        sc1 = (w0 >> (sh + 8)) & 63u;
        m1 = (w1 >> (sh + 8)) & 63u;
    } else {
        sc0 = ((w2 >> sh) & 15u) | (((w0 >> (sh + 6)) & 3u) << 4);
        m0 = ((w2 >> (sh + 4)) & 15u) | (((w1 >> (sh + 6)) & 3u) << 4);
        sc1 = ((w2 >> (sh + 8)) & 15u) | (((w0 >> (sh + 14)) & 3u) << 4);
        m1 = ((w2 >> (sh + 12)) & 15u) | (((w1 >> (sh + 14)) & 3u) << 4);
    }
}

IFR_DEV void lds16(const float *p, float *x) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 t = ((const float4 *)p)[i];
        x[4 * i] = t.x;
        x[4 * i + 1] = t.y;
        x[4 * i + 2] = t.z;
        x[4 * i + 3] = t.w;
    }
}

IFR_DEV float sum16v(const float *x) {
    float s0 = (x[0] + x[1]) + (x[2] + x[3]);
    float s1 = (x[4] + x[5]) + (x[6] + x[7]);
    float s2 = (x[8] + x[9]) + (x[10] + x[11]);
    float s3 = (x[12] + x[13]) + (x[14] + x[15]);
    return (s0 + s1) + (s2 + s3);
}

// Dot of 16 unsigned byte codes (four words) with x[0..15].
IFR_DEV float dot16u(uint32_t a, uint32_t b, uint32_t c, uint32_t d, const float *x) {
    float s = 0.0f;
    s = dot4u(a, x, s);
    s = dot4u(b, x + 4, s);
    s = dot4u(c, x + 8, s);
    s = dot4u(d, x + 12, s);
    return s;
}

template <int FMT>
struct QFmt;
template <>
struct QFmt<Q4_K> { static constexpr int QK = 256, BB = 144, LPB = 8; };
template <>
struct QFmt<Q5_K> { static constexpr int QK = 256, BB = 176, LPB = 8; };
template <>
struct QFmt<Q6_K> { static constexpr int QK = 256, BB = 210, LPB = 8; };
template <>
struct QFmt<Q8_0> { static constexpr int QK = 32, BB = 34, LPB = 2; };

// acc[r] += dot(row r, x) over all blocks, for this lane's share.
template <int FMT, int R>
IFR_DEV void gemv_accum(const uint8_t *const *rowp, uint32_t nb, int lane, const float *xs, float *acc) {
    constexpr int LPB = QFmt<FMT>::LPB, BPI = 64 / LPB, BB = QFmt<FMT>::BB, QK = QFmt<FMT>::QK;
    const uint32_t c = (uint32_t)lane % LPB, bsub = (uint32_t)lane / LPB;
    for (uint32_t kb0 = 0; kb0 < nb; kb0 += BPI) {
        const uint32_t kb = kb0 + bsub;
        if (kb >= nb) break;
        if constexpr (FMT == Q4_K) {
            // lane chunk c: qs bytes [16c, 16c+16) = elements 64g+16h+t (low
            // nibbles) and 64g+32+16h+t (high nibbles), g = c/2, h = c%2.
            const uint32_t g = c >> 1, h = c & 1u;
            uint4 hv[R], qv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *b = rowp[r] + (size_t)kb * BB;
                hv[r] = ld16(b);
                qv[r] = ld16(b + 16 + 16 * c);
            }
            float xl[16], xh[16];
            const float *xp = xs + kb * QK + 64 * g + 16 * h;
            lds16(xp, xl);
            lds16(xp + 32, xh);
            const float sl = sum16v(xl), sh = sum16v(xh);
#pragma unroll
            for (int r = 0; r < R; r++) {
                uint32_t sc0, m0, sc1, m1;
                scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
                const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
                const uint4 q = qv[r];
                const float dl = dot16u(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, xl);
                const float dh = dot16u((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                                        (q.w >> 4) & 0x0F0F0F0Fu, xh);
                acc[r] += (d * (float)sc0) * dl - (dm * (float)m0) * sl + (d * (float)sc1) * dh - (dm * (float)m1) * sh;
            }
        } else if constexpr (FMT == Q5_K) {
            const uint32_t g = c >> 1, h = c & 1u;
            uint4 hv[R], qv[R], qhv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *b = rowp[r] + (size_t)kb * BB;
                hv[r] = ld16(b);
                qhv[r] = ld16(b + 16 + 16 * h);
                qv[r] = ld16(b + 48 + 16 * c);
            }
            float xl[16], xh[16];
            const float *xp = xs + kb * QK + 64 * g + 16 * h;
            lds16(xp, xl);
            lds16(xp + 32, xh);
            const float sl = sum16v(xl), sh = sum16v(xh);
            const uint32_t s0 = 2 * g, s1 = 2 * g + 1;
#pragma unroll
            for (int r = 0; r < R; r++) {
                uint32_t sc0, m0, sc1, m1;
                scale_min_pair(g, hv[r].y, hv[r].z, hv[r].w, sc0, m0, sc1, m1);
                const float d = f16_to_f32(hv[r].x & 0xFFFFu), dm = f16_to_f32(hv[r].x >> 16);
                const uint4 q = qv[r], e = qhv[r];
                const uint32_t M = 0x0F0F0F0Fu, B = 0x01010101u;
                const float dl = dot16u((q.x & M) | (((e.x >> s0) & B) << 4), (q.y & M) | (((e.y >> s0) & B) << 4),
                                        (q.z & M) | (((e.z >> s0) & B) << 4), (q.w & M) | (((e.w >> s0) & B) << 4), xl);
                const float dh = dot16u(((q.x >> 4) & M) | (((e.x >> s1) & B) << 4),
                                        ((q.y >> 4) & M) | (((e.y >> s1) & B) << 4),
                                        ((q.z >> 4) & M) | (((e.z >> s1) & B) << 4),
                                        ((q.w >> 4) & M) | (((e.w >> s1) & B) << 4), xh);
                acc[r] += (d * (float)sc0) * dl - (dm * (float)m0) * sl + (d * (float)sc1) * dh - (dm * (float)m1) * sh;
            }
        } else if constexpr (FMT == Q6_K) {
            // lane chunk c: i = c/4 (half), cp = c%4, s = cp%2, u = cp/2.
            // ql bytes [64i+16cp, +16): low nibbles are elements
            // 128i+32u+16s+t, high nibbles +64; qh bytes [32i+16s, +16) give
            // bits 2u..2u+1 (low) and 2u+4..2u+5 (high); scales 8i+s+2u, +4.
            const uint32_t i = c >> 2, cp = c & 3u, s = cp & 1u, u = cp >> 1;
            uint4 qlv[R], qhv[R];
            uint32_t dsc[R], scl[R], sch[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *b = rowp[r] + (size_t)kb * BB;
                qlv[r] = ld16_a2(b + 64 * i + 16 * cp);
                qhv[r] = ld16_a2(b + 128 + 32 * i + 16 * s);
                scl[r] = b[192 + 8 * i + s + 2 * u];
                sch[r] = b[192 + 8 * i + s + 2 * u + 4];
                dsc[r] = ld_u16(b + 208);
            }
            float xl[16], xh[16];
            const float *xp = xs + kb * QK + 128 * i + 32 * u + 16 * s;
            lds16(xp, xl);
            lds16(xp + 64, xh);
            const float sl = sum16v(xl), sh = sum16v(xh);
            const uint32_t s0 = 2 * u, s1 = 2 * u + 4;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint4 q = qlv[r], e = qhv[r];
                const uint32_t M = 0x0F0F0F0Fu, B = 0x03030303u;
                const float dl = dot16u((q.x & M) | (((e.x >> s0) & B) << 4), (q.y & M) | (((e.y >> s0) & B) << 4),
                                        (q.z & M) | (((e.z >> s0) & B) << 4), (q.w & M) | (((e.w >> s0) & B) << 4), xl);
                const float dh = dot16u(((q.x >> 4) & M) | (((e.x >> s1) & B) << 4),
                                        ((q.y >> 4) & M) | (((e.y >> s1) & B) << 4),
                                        ((q.z >> 4) & M) | (((e.z >> s1) & B) << 4),
                                        ((q.w >> 4) & M) | (((e.w >> s1) & B) << 4), xh);
                const float d = f16_to_f32(dsc[r]);
                const float fl = (float)(int)(int8_t)scl[r], fh = (float)(int)(int8_t)sch[r];
                // codes are stored +32: sum (q-32) x = sum q x - 32 sum x
                acc[r] += (d * fl) * (dl - 32.0f * sl) + (d * fh) * (dh - 32.0f * sh);
            }
        } else { // Q8_0: lane half c of block kb: qs bytes [16c, 16c+16)
            uint4 qv[R];
            uint32_t dsc[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint8_t *b = rowp[r] + (size_t)kb * BB;
                dsc[r] = ld_u16(b);
                qv[r] = ld16_a2(b + 2 + 16 * c);
            }
            float xv[16];
            lds16(xs + kb * QK + 16 * c, xv);
            const float sx = sum16v(xv);
#pragma unroll
            for (int r = 0; r < R; r++) {
                // signed codes: (q ^ 0x80) = q + 128 as an unsigned byte
                const uint4 q = qv[r];
                const uint32_t F = 0x80808080u;
                const float dq = dot16u(q.x ^ F, q.y ^ F, q.z ^ F, q.w ^ F, xv);
                acc[r] += f16_to_f32(dsc[r]) * (dq - 128.0f * sx);
            }
        }
    }
}

template <int MODE>
IFR_DEV const uint8_t *gemv_row_ptr(const GemvArgs &a, uint32_t v) {
    if constexpr (MODE == GEMV_QKV) {
        if (v < a.rows0) return a.w0 + (size_t)v * a.row_bytes;
        v -= a.rows0;
        if (v < a.rows1) return a.w1 + (size_t)v * a.row_bytes;
        return a.w2 + (size_t)(v - a.rows1) * a.row_bytes;
    } else if constexpr (MODE == GEMV_GATEUP) {
        return ((v & 1u) ? a.w1 : a.w0) + (size_t)(v >> 1) * a.row_bytes;
    } else {
        return a.w0 + (size_t)v * a.row_bytes;
    }
}

// One RoPE rotation of the adjacent pair at even index idx of a head-strided
// vector (inferi-shaders/src/rope.rs:51-92): theta = base^(-(idx mod hs)/hs)
// read from the state's table (rope_theta_f32 of every pair), angle =
// pos * theta.
IFR_DEV void rope_pair(float &a, float &b, uint32_t idx, uint32_t hs, uint32_t pos, const float *theta_tab) {
    const float theta = theta_tab[(idx % hs) >> 1];
    const float ang = (float)pos * theta;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float x = a, y = b;
    a = cs * x - sn * y;
    b = sn * x + cs * y;
}

template <int FMT, int MODE>
__device__ void gemv_body(const GemvArgs &a) {
    constexpr int R = GEMV_R;
    constexpr bool NORM = (MODE == GEMV_QKV || MODE == GEMV_GATEUP || MODE == GEMV_HEAD);
    extern __shared__ float xs[];
    __shared__ float red[GEMV_WAVES];
    __shared__ uint64_t kred[GEMV_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // Stage x (times gamma when normalising) into LDS.
    float ss = 0.0f;
    for (uint32_t i = (uint32_t)tid * 4; i < a.cols; i += 64 * GEMV_WAVES * 4) {
        float4 v = *(const float4 *)(a.x + i);
        if constexpr (NORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            const float4 g = *(const float4 *)(a.gamma + i);
            v.x *= g.x;
            v.y *= g.y;
            v.z *= g.z;
            v.w *= g.w;
        }
        *(float4 *)(xs + i) = v;
    }
    float rs = 1.0f;
    if constexpr (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    if constexpr (NORM) {
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        // rms_norm.rs:115: 1 / sqrt(sum(x^2)/n + eps)
        rs = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
    }

    uint32_t pos = 0;
    if constexpr (MODE == GEMV_QKV) pos = a.ctl->pos;

    const uint32_t rows_per_wg = GEMV_WAVES * R;
    const uint32_t ntiles = (a.total_rows + rows_per_wg - 1) / rows_per_wg;
    uint64_t best = 0;
    for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const uint32_t v0 = (tile * GEMV_WAVES + (uint32_t)wave) * R;
        if (v0 >= a.total_rows) continue;
        const uint8_t *rowp[R];
#pragma unroll
        for (int r = 0; r < R; r++) rowp[r] = gemv_row_ptr<MODE>(a, min(v0 + r, a.total_rows - 1));
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        gemv_accum<FMT, R>(rowp, a.nb, lane, xs, acc);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]) * rs;

        if constexpr (MODE == GEMV_PLAIN || MODE == GEMV_RESID || MODE == GEMV_HEAD) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (lane == r && v0 + r < a.total_rows) {
                    if constexpr (MODE == GEMV_RESID)
                        a.y[v0 + r] += acc[r];
                    else
                        a.y[v0 + r] = acc[r];
                }
            }
            if constexpr (MODE == GEMV_HEAD) {
#pragma unroll
                for (int r = 0; r < R; r++)
                    if (v0 + r < a.total_rows) {
                        const uint64_t k = argmax_key(acc[r], v0 + r);
                        best = k > best ? k : best;
                    }
            }
        } else if constexpr (MODE == GEMV_GATEUP) {
            // virtual rows 2j (gate j) and 2j+1 (up j): h[j] = up * silu(gate)
#pragma unroll
            for (int p = 0; p < R / 2; p++) {
                if (lane == p && v0 + 2 * p + 1 < a.total_rows) {
                    const float gt = acc[2 * p], up = acc[2 * p + 1];
                    a.y[(v0 >> 1) + p] = up * (gt / (1.0f + expf(-gt)));
                }
            }
        } else if constexpr (MODE == GEMV_QKV) {
#pragma unroll
            for (int p = 0; p < R / 2; p++) {
                const uint32_t v = v0 + 2 * p;
                if (lane == p && v + 1 < a.total_rows) {
                    float x0 = acc[2 * p], x1 = acc[2 * p + 1];
                    if (v < a.rows0) {
                        rope_pair(x0, x1, v, a.head_size, pos, a.rope_tab);
                        a.y[v] = x0;
                        a.y[v + 1] = x1;
                    } else {
                        const bool is_k = v < a.rows0 + a.rows1;
                        const uint32_t idx = is_k ? v - a.rows0 : v - a.rows0 - a.rows1;
                        if (is_k) rope_pair(x0, x1, idx, a.head_size, pos, a.rope_tab);
                        const size_t off = (size_t)pos * a.kv_dim + idx;
                        void *cache = is_k ? a.k_cache : a.v_cache;
                        if (a.kv_f16) {
                            const uint32_t packed = (uint32_t)f32_to_f16(x0) | ((uint32_t)f32_to_f16(x1) << 16);
                            *(uint32_t *)((uint16_t *)cache + off) = packed;
                        } else {
                            ((float *)cache)[off] = x0;
                            ((float *)cache)[off + 1] = x1;
                        }
                    }
                }
            }
        }
    }
    if constexpr (MODE == GEMV_HEAD) {
        if (a.part_keys) {
            if (lane == 0) kred[wave] = best;
            __syncthreads();
            if (tid == 0) {
                uint64_t b = kred[0];
                for (int w = 1; w < GEMV_WAVES; w++) b = kred[w] > b ? kred[w] : b;
                a.part_keys[blockIdx.x] = b;
            }
        }
    }
}

} // namespace ifr

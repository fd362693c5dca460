/* Host-core restatement of the reference's GPU shader decompositions, the
 * CPU baseline of the single-op configs (the GEMV sweep and the decode
 * attention block).  TEST INFRASTRUCTURE ONLY: the product library never
 * loads it; bench.py times it beside the GPU figures, and tests/ pin it
 * against the oracle.
 *
 * The reference runs these shaders on a GPU, or through its khal
 * "cpu-parallel" backend on host threads (crates/inferi/Cargo.toml:17).
 * Each workgroup is restated as one loop nest: its lanes' private sums are
 * arrays, its shared-memory tree reductions run in the shaders' order, and
 * workgroups are spread over POSIX threads.  Element values are the
 * reference's f32 arithmetic (products before sums, no FMA contraction); dot
 * products run left to right as glam's Vec4::dot does.
 *
 *   GEMV Q4_K   crates/inferi-shaders/src/gemv_quant_q4_k.rs:47-182
 *   GEMV Q5_K   crates/inferi-shaders/src/gemv_quant_q5_k.rs:47-196
 *   GEMV Q6_Kx2 crates/inferi-shaders/src/gemv_quant_q6_kx2.rs:41-227
 *   GEMV Q8_0x2 crates/inferi-shaders/src/gemv_quant_q8_0x2.rs:27-175
 *   attention   crates/inferi-shaders/src/fused_attention.rs:66-241
 *               (fused_attention, up to 2048 positions) and :377-617
 *               (flash_attention, longer), chosen as
 *               crates/inferi/src/ops/batched_multiquery_attention.rs:39-76
 *               chooses.  The shaders read an f32 cache; the configs here
 *               hold an f16 cache, decoded to f32 on load.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
    float x, y, z, w;
} v4;

static inline float dot4(v4 a, v4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

static inline float h2f(uint16_t h) { return (float)ifo_decode_f16(h); }

static inline uint32_t rd32(const uint8_t *p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* unpack_scale_and_min, gemv_quant_q4_k.rs:28-43: the 6-bit (scale, min) of
 * sub-block j from the 12 scale bytes */
static void scale_min(uint32_t j, const uint8_t *sc, uint32_t *d, uint32_t *m) {
    if (j < 4) {
        *d = sc[j] & 63u;
        *m = sc[j + 4] & 63u;
    } else {
        *d = (sc[j + 4] & 0xFu) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* ---------------------------------------------------------------- GEMV */

/* Lane k's two Vec4 parts of a Q4_K / Q5_K block (dequantize_q4_k_workgroup,
 * gemv_quant_q4_k.rs:47-93; the Q5_K fifth bit, gemv_quant_q5_k.rs:47-110):
 * elements 64 g + 4 (k % 8) + {0..3} (low nibbles) and + 32 (high), g = k / 8. */
static void parts_k(int fmt, const uint8_t *b, uint32_t k, v4 out[2]) {
    const float d = h2f((uint16_t)rd32(b)), mn = h2f((uint16_t)(rd32(b) >> 16));
    const uint32_t g = k / 8, l = k % 8;
    uint32_t s1, m1s, s2, m2s;
    scale_min(2 * g, b + 4, &s1, &m1s);
    scale_min(2 * g + 1, b + 4, &s2, &m2s);
    const float d1 = d * (float)s1, m1 = mn * (float)m1s, d2 = d * (float)s2, m2 = mn * (float)m2s;
    const uint8_t *qs = fmt == IFO_Q4_K ? b + 16 : b + 48;
    const uint32_t q = rd32(qs + 4 * k);
    uint32_t lo[4], hi[4];
    for (int e = 0; e < 4; e++) {
        lo[e] = (q >> (8 * e)) & 0xFu;
        hi[e] = (q >> (8 * e + 4)) & 0xFu;
    }
    if (fmt == IFO_Q5_K) {
        const uint32_t qh = rd32(b + 16 + 4 * l), u1 = 1u << (2 * g), u2 = 2u << (2 * g);
        for (int e = 0; e < 4; e++) {
            lo[e] += ((qh >> (8 * e)) & u1) ? 16u : 0u;
            hi[e] += ((qh >> (8 * e)) & u2) ? 16u : 0u;
        }
    }
    out[0] = (v4){(float)lo[0] * d1 - m1, (float)lo[1] * d1 - m1, (float)lo[2] * d1 - m1, (float)lo[3] * d1 - m1};
    out[1] = (v4){(float)hi[0] * d2 - m2, (float)hi[1] * d2 - m2, (float)hi[2] * d2 - m2, (float)hi[3] * d2 - m2};
}

/* Lane k's four Vec4 parts of a Q6_K block pair (dequantize_q6_kx2_workgroup,
 * gemv_quant_q6_kx2.rs:41-140): block k / 16 of the pair, half i = (k / 8) % 2,
 * positions l = 4 (k % 8) + {0..3} of the half, elements 128 i + l + {0, 32,
 * 64, 96}, scales of sub-block (k % 8) / 4 (+2, +4, +6). */
static void parts_q6(const uint8_t *pair, uint32_t k, v4 out[4]) {
    const uint8_t *b = pair + (k / 16) * 210;
    const uint32_t i = (k / 8) % 2, lw = k % 8, is = lw / 4;
    const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
    const int8_t *sc = (const int8_t *)(b + 192 + 8 * i);
    const float s[4] = {(1.0f * d) * (float)sc[is], (1.0f * d) * (float)sc[is + 2], (1.0f * d) * (float)sc[4 + is],
                        (1.0f * d) * (float)sc[4 + is + 2]};
    const uint8_t *ql = b + 64 * i, *qh = b + 128 + 32 * i;
    float v[4][4];
    for (int e = 0; e < 4; e++) {
        const uint32_t l = 4 * lw + (uint32_t)e;
        const uint32_t h = qh[l], a = ql[l], c = ql[l + 32];
        const int q1 = (int)((a & 0xFu) | ((h & 3u) << 4)) - 32;
        const int q2 = (int)((c & 0xFu) | (((h >> 2) & 3u) << 4)) - 32;
        const int q3 = (int)((a >> 4) | (((h >> 4) & 3u) << 4)) - 32;
        const int q4 = (int)((c >> 4) | (((h >> 6) & 3u) << 4)) - 32;
        v[0][e] = s[0] * (float)q1;
        v[1][e] = s[1] * (float)q2;
        v[2][e] = s[2] * (float)q3;
        v[3][e] = s[3] * (float)q4;
    }
    for (int p = 0; p < 4; p++) out[p] = (v4){v[p][0], v[p][1], v[p][2], v[p][3]};
}

typedef struct {
    int fmt;
    uint32_t rows, cols;
    const uint8_t *w;
    const float *x;
    float *y;
    uint32_t wg0, wg1; /* workgroups (row quads) of this thread */
} gemv_job;

/* sketch tree reduction of the 32 lane sums (reduce_sum, strides 16..1) */
static void tree32(v4 sk[32], float out[4]) {
    for (int stride = 16; stride >= 1; stride /= 2)
        for (int t = 0; t < stride; t++) {
            sk[t].x += sk[t + stride].x;
            sk[t].y += sk[t + stride].y;
            sk[t].z += sk[t + stride].z;
            sk[t].w += sk[t + stride].w;
        }
    out[0] = sk[0].x, out[1] = sk[0].y, out[2] = sk[0].z, out[3] = sk[0].w;
}

static void *gemv_run(void *arg) {
    const gemv_job *J = (const gemv_job *)arg;
    const v4 *xv = (const v4 *)J->x;
    const size_t rb = (size_t)(J->cols / (uint32_t)ifo_block_elems(J->fmt)) * (size_t)ifo_block_bytes(J->fmt);
    for (uint32_t wg = J->wg0; wg < J->wg1; wg++) {
        v4 sum[32];
        memset(sum, 0, sizeof sum);
        const uint8_t *row[4];
        for (int r = 0; r < 4; r++) row[r] = J->w + (size_t)(4 * wg + (uint32_t)r) * rb;
        if (J->fmt == IFO_Q4_K || J->fmt == IFO_Q5_K) {
            const uint32_t nb = J->cols / 256, bb = J->fmt == IFO_Q4_K ? 144 : 176;
            for (uint32_t j = 0; j < nb; j++)
                for (uint32_t k = 0; k < 32; k++) {
                    v4 p[4][2];
                    for (int r = 0; r < 4; r++) parts_k(J->fmt, row[r] + (size_t)j * bb, k, p[r]);
                    const size_t jb = (size_t)j * 64, jj = k & ~7u;
                    const v4 va = xv[jb + k + jj], vb = xv[jb + k + jj + 8];
                    sum[k].x += dot4(p[0][0], va), sum[k].y += dot4(p[1][0], va);
                    sum[k].z += dot4(p[2][0], va), sum[k].w += dot4(p[3][0], va);
                    sum[k].x += dot4(p[0][1], vb), sum[k].y += dot4(p[1][1], vb);
                    sum[k].z += dot4(p[2][1], vb), sum[k].w += dot4(p[3][1], vb);
                }
        } else if (J->fmt == IFO_Q6_K) {
            const uint32_t npair = J->cols / 512;
            for (uint32_t j = 0; j < npair; j++)
                for (uint32_t k = 0; k < 32; k++) {
                    v4 p[4][4];
                    for (int r = 0; r < 4; r++) parts_q6(row[r] + (size_t)j * 420, k, p[r]);
                    const size_t jb = (size_t)j * 128, jj = (k / 16) * 64 + ((k / 8) % 2) * 32 + (k % 8);
                    const v4 vv[4] = {xv[jb + jj], xv[jb + jj + 8], xv[jb + jj + 16], xv[jb + jj + 24]};
                    /* Mat4::transpose() * v, column by column: component r is
                     * dot(parts_r[c], v) (glam's mul_vec4), summed over c */
                    float t[4][4];
                    for (int c = 0; c < 4; c++)
                        for (int r = 0; r < 4; r++) t[c][r] = dot4(p[r][c], vv[c]);
                    sum[k].x += ((t[0][0] + t[1][0]) + t[2][0]) + t[3][0];
                    sum[k].y += ((t[0][1] + t[1][1]) + t[2][1]) + t[3][1];
                    sum[k].z += ((t[0][2] + t[1][2]) + t[2][2]) + t[3][2];
                    sum[k].w += ((t[0][3] + t[1][3]) + t[2][3]) + t[3][3];
                }
        } else { /* Q8_0 pairs: lane k takes block (k / 8) of the iteration's four, bytes 4 (k % 8) .. */
            const uint32_t niter = J->cols / 128;
            for (uint32_t j = 0; j < niter; j++)
                for (uint32_t k = 0; k < 32; k++) {
                    const v4 vj = xv[(size_t)j * 32 + k];
                    float dd[4];
                    for (int r = 0; r < 4; r++) {
                        const uint8_t *b = row[r] + ((size_t)j * 4 + k / 8) * 34;
                        const float s = h2f((uint16_t)(b[0] | (b[1] << 8)));
                        const int8_t *q = (const int8_t *)(b + 2 + 4 * (k % 8));
                        const v4 w = {(float)q[0] * s, (float)q[1] * s, (float)q[2] * s, (float)q[3] * s};
                        dd[r] = dot4(w, vj);
                    }
                    sum[k].x += dd[0], sum[k].y += dd[1], sum[k].z += dd[2], sum[k].w += dd[3];
                }
        }
        tree32(sum, J->y + 4 * (size_t)wg);
    }
    return NULL;
}

int ifo_ref_gemv(int32_t dtype, uint32_t rows, uint32_t cols, const void *w, const float *x, float *y, int nthreads) {
    if (rows % 4) return -1;
    if ((dtype == IFO_Q4_K || dtype == IFO_Q5_K) && cols % 256) return -1;
    if (dtype == IFO_Q6_K && cols % 512) return -1;
    if (dtype == IFO_Q8_0 && cols % 128) return -1;
    if (dtype != IFO_Q4_K && dtype != IFO_Q5_K && dtype != IFO_Q6_K && dtype != IFO_Q8_0) return -1;
    if (nthreads <= 0) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    const uint32_t wgs = rows / 4;
    pthread_t th[64];
    gemv_job jobs[64];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (gemv_job){dtype, rows, cols, (const uint8_t *)w, x, y, (uint32_t)((uint64_t)wgs * t / nthreads),
                             (uint32_t)((uint64_t)wgs * (t + 1) / nthreads)};
        pthread_create(&th[t], NULL, gemv_run, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    return 0;
}

/* ----------------------------------------------------------- attention */

#define ATT_WG 128    /* threads per workgroup without subgroup ops */
#define ATT_MAX 2048  /* fused_attention's score buffer */
#define ATT_BLOCK 32  /* flash_attention's BLOCK_KV */

typedef struct {
    const float *q;
    const uint16_t *k, *v; /* f16 cache [seq][kv_dim] */
    float *out;
    uint32_t n_heads, n_kv_heads, hs, pos;
    uint32_t h0, h1;
} att_job;

static float tree_max128(float *ws) {
    for (int stride = 64; stride >= 1; stride /= 2)
        for (int t = 0; t < stride; t++) ws[t] = fmaxf(ws[t], ws[t + stride]);
    return ws[0];
}
static float tree_sum128(float *ws) {
    for (int stride = 64; stride >= 1; stride /= 2)
        for (int t = 0; t < stride; t++) ws[t] += ws[t + stride];
    return ws[0];
}

static void *att_run(void *arg) {
    const att_job *A = (const att_job *)arg;
    const uint32_t hs = A->hs, kv_dim = A->n_kv_heads * hs, kv_mul = A->n_heads / A->n_kv_heads;
    const size_t seq = (size_t)A->pos + 1;
    const float sq = sqrtf((float)hs);
    float *scores = (float *)malloc(seq * sizeof(float));
    float ws[ATT_WG];
    for (uint32_t h = A->h0; h < A->h1; h++) {
        const float *q = A->q + (size_t)h * hs;
        const size_t kvb = (size_t)(h / kv_mul) * hs;
        float *out = A->out + (size_t)h * hs;
        if (seq <= ATT_MAX) {
            /* fused_attention, fused_attention.rs:66-241 */
            for (int t = 0; t < ATT_WG; t++) ws[t] = -1.0e38f;
            for (size_t i = 0; i < seq; i++) {
                const uint16_t *kr = A->k + i * kv_dim + kvb;
                float dot = 0.0f;
                for (uint32_t d = 0; d < hs; d++) dot += q[d] * h2f(kr[d]);
                scores[i] = dot / sq;
                ws[i % ATT_WG] = fmaxf(ws[i % ATT_WG], scores[i]);
            }
            const float mx = tree_max128(ws);
            for (int t = 0; t < ATT_WG; t++) ws[t] = 0.0f;
            for (size_t i = 0; i < seq; i++) {
                scores[i] = expf(scores[i] - mx);
                ws[i % ATT_WG] += scores[i];
            }
            const float inv = 1.0f / tree_sum128(ws);
            for (size_t i = 0; i < seq; i++) scores[i] = scores[i] * inv;
            for (uint32_t d = 0; d < hs; d++) {
                float acc = 0.0f;
                for (size_t i = 0; i < seq; i++) acc += scores[i] * h2f(A->v[i * kv_dim + kvb + d]);
                out[d] = acc;
            }
        } else {
            /* flash_attention, fused_attention.rs:377-617: blocks of 32
             * positions with a running maximum and sum */
            float rmax = -1.0e38f, rsum = 0.0f, acc[128], sc[ATT_BLOCK];
            for (uint32_t d = 0; d < hs; d++) acc[d] = 0.0f;
            for (size_t b0 = 0; b0 < seq; b0 += ATT_BLOCK) {
                const size_t bl = seq - b0 < ATT_BLOCK ? seq - b0 : ATT_BLOCK;
                for (int t = 0; t < ATT_WG; t++) ws[t] = -1.0e38f;
                for (size_t p = 0; p < bl; p++) {
                    const uint16_t *kr = A->k + (b0 + p) * kv_dim + kvb;
                    float dot = 0.0f;
                    for (uint32_t d = 0; d < hs; d++) dot += q[d] * h2f(kr[d]);
                    sc[p] = dot / sq;
                    ws[p] = sc[p];
                }
                const float bmax = tree_max128(ws);
                for (int t = 0; t < ATT_WG; t++) ws[t] = 0.0f;
                for (size_t p = 0; p < bl; p++) {
                    sc[p] = expf(sc[p] - bmax);
                    ws[p] = sc[p];
                }
                const float bsum = tree_sum128(ws);
                const float nmax = fmaxf(rmax, bmax);
                const float r_old = expf(rmax - nmax), r_new = expf(bmax - nmax);
                rmax = nmax;
                rsum = rsum * r_old + bsum * r_new;
                for (uint32_t d = 0; d < hs; d++) {
                    const float old = acc[d] * r_old;
                    float add = 0.0f;
                    for (size_t p = 0; p < bl; p++) add += (sc[p] * r_new) * h2f(A->v[(b0 + p) * kv_dim + kvb + d]);
                    acc[d] = old + add;
                }
            }
            for (uint32_t d = 0; d < hs; d++) out[d] = acc[d] / rsum;
        }
    }
    free(scores);
    return NULL;
}

int ifo_ref_attention(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, uint32_t n_heads,
                      uint32_t n_kv_heads, uint32_t head_size, uint32_t pos, float *out, int nthreads) {
    if (!n_kv_heads || n_heads % n_kv_heads || head_size > 128 || head_size == 0) return -1;
    if (nthreads <= 0) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    if ((uint32_t)nthreads > n_heads) nthreads = (int)n_heads;
    pthread_t th[64];
    att_job jobs[64];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (att_job){q, k_cache, v_cache, out, n_heads, n_kv_heads, head_size, pos,
                            (uint32_t)((uint64_t)n_heads * t / nthreads), (uint32_t)((uint64_t)n_heads * (t + 1) / nthreads)};
        pthread_create(&th[t], NULL, att_run, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    return 0;
}

// Small per-token kernels: RMSNorm, RoPE, SiLU*mul, residual add, argmax,
// token embedding, KV-row store, dequant/quantize of whole tensors and the
// synthetic-weight generator.
#pragma once
#include "gemv.h"

namespace ifr {

// The operands are views: element i of a sits at a.a[i * a.sa] (likewise b,
// w, k), as the reference shaders index through their tensor layouts
// (shape.it(..), rms_norm.rs:118-119, rope.rs:81-87, silu.rs:46-47).

// RMSNorm with one 1024-thread workgroup (inferi-shaders/src/rms_norm.rs:81-121):
// rms = 1 / sqrt(sum(x^2)/n + eps); out = (x * rms) * w.
__device__ void rms_norm_body(const EltArgs &a) {
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float eps = ((const ifr_rms_cfg_dev *)a.cfg)->nudge_factor;
    float ss = 0.0f;
    for (uint32_t i = tid; i < a.n; i += blockDim.x) ss = fmaf(a.b[i * a.sb], a.b[i * a.sb], ss);
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    if (tid < 64) {
        float v = tid < (int)(blockDim.x >> 6) ? red[tid] : 0.0f;
        v = wave_sum(v);
        if (tid == 0) red[0] = v;
    }
    __syncthreads();
    const float rms = 1.0f / sqrtf(red[0] / (float)a.n + eps);
    for (uint32_t i = tid; i < a.n; i += blockDim.x) a.a[i * a.sa] = (a.b[i * a.sb] * rms) * a.w[i * a.sw];
}

// RoPE (inferi-shaders/src/rope.rs:51-92 Original, :97-141 NeoX).  Thread i
// rotates pair i of q and, while 2i < kv_dim, the same pair of k.  Through a
// view, the pair's first element is the view's element iq and its second
// lies `shift` elements after it in memory (rope.rs:81-84, 129-132: the
// partner is at it(..) + 1, or + head_size / 2).
__device__ void rope_body(const EltArgs &a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n / 2) return;
    const ifr_rope_cfg_dev c = *(const ifr_rope_cfg_dev *)a.cfg;
    const float head_dim = (float)((i * 2) % c.head_size);
    const float theta = rope_theta_f32(c.base_freq, head_dim, (float)c.head_size);
    const float ang = (float)c.pos * theta;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    uint32_t iq, shift;
    if (a.variant == 1) { // NeoX: pairs (i, i + hs/2) within each head
        const uint32_t head_id = (i * 2) / c.head_size;
        iq = i + head_id * c.head_size / 2;
        shift = c.head_size / 2;
    } else {
        iq = 2 * i;
        shift = 1;
    }
    if (iq + shift >= a.n) return;
    float *q0 = a.a + iq * a.sa;
    float x = q0[0], y = q0[shift];
    q0[0] = cs * x - sn * y;
    q0[shift] = sn * x + cs * y;
    if (i * 2 < c.kv_dim && iq + shift < a.n2) {
        float *k0 = a.k + iq * a.sk;
        x = k0[0];
        y = k0[shift];
        k0[0] = cs * x - sn * y;
        k0[shift] = sn * x + cs * y;
    }
}

// h1 <- h2 * (h1 / (1 + exp(-h1)))  (inferi-shaders/src/silu.rs:14-53)
__device__ void silu_body(const EltArgs &a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.n) return;
    const float h = a.a[i * a.sa];
    a.a[i * a.sa] = a.b[i * a.sb] * (h / (1.0f + expf(-h)));
}

__device__ void add_body(const EltArgs &a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.a[i * a.sa] = a.a[i * a.sa] + a.b[i * a.sb];
}

// Per-workgroup best key over a grid-stride range of v.
__device__ void argmax_part_body(const ArgmaxArgs &a) {
    __shared__ uint64_t red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t best = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + tid; i < a.n; i += gridDim.x * blockDim.x) {
        const uint64_t k = argmax_key(a.div != 0.0f ? a.v[i] / a.div : a.v[i], i);
        best = k > best ? k : best;
    }
    for (int sh = 1; sh < 64; sh <<= 1) {
        const uint64_t o = __shfl_xor(best, sh, 64);
        best = o > best ? o : best;
    }
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = red[0];
        for (uint32_t w = 1; w < (blockDim.x >> 6); w++) b = red[w] > b ? red[w] : b;
        a.part_keys[blockIdx.x] = b;
    }
}

// End of a decode step at position p with next token idx (one thread): store
// the token unless position p+1 is forced, advance the device position and
// the position fields of the op configs.  The position saturates at
// max_pos - 1, so a step run past the end of the cache rewrites the last row
// instead of leaving it.
IFR_DEV void step_advance(StepCtl *ctl, uint32_t *tokens, uint32_t *rope_pos, uint32_t *attn_pos, uint32_t p,
                          uint32_t idx) {
    if (p + 1 < ctl->max_pos) {
        if (p + 1 >= ctl->n_forced) tokens[p + 1] = idx;
        ctl->pos = p + 1;
        if (rope_pos) *rope_pos = p + 1;
        if (attn_pos) *attn_pos = p + 1;
    }
}

// One workgroup: reduce the partial keys to the winning index; optionally
// finish a decode step (store the next token unless it is forced, advance
// the device position and the position fields of the op configs).
// Launched as one workgroup of ARGMAX_FINAL_THREADS threads (a constant:
// blockDim.x would be one more scalar round trip, to the hidden arguments).
constexpr uint32_t ARGMAX_FINAL_THREADS = 1024;
__device__ void argmax_final_body(const ArgmaxArgs &a) {
    __shared__ uint64_t red[ARGMAX_FINAL_THREADS / 64];
    // the arguments in one batch of scalar loads; an empty asm that emits nothing
    asm volatile("" ::"s"(a.n_parts), "s"(a.part_keys), "s"(a.out_index), "s"(a.ctl), "s"(a.tokens), "s"(a.rope_pos),
                 "s"(a.attn_pos));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t best = 0;
    for (uint32_t i = tid; i < a.n_parts; i += ARGMAX_FINAL_THREADS)
        best = a.part_keys[i] > best ? a.part_keys[i] : best;
    for (int sh = 1; sh < 64; sh <<= 1) {
        const uint64_t o = __shfl_xor(best, sh, 64);
        best = o > best ? o : best;
    }
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (tid == 0) {
        uint64_t b = red[0];
        for (uint32_t w = 1; w < ARGMAX_FINAL_THREADS / 64; w++) b = red[w] > b ? red[w] : b;
        const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu);
        if (a.out_index) *a.out_index = idx;
        if (a.ctl) step_advance(a.ctl, a.tokens, a.rope_pos, a.attn_pos, a.ctl->pos, idx);
    }
}

// x <- dequant(table)[tokens[pos], :]  (transformer.rs:366-374 dequantizes the
// table at load; chat_llama2.rs:217-219 copies the row).  Bit-exact.  Also
// quantizes x * gamma for the first GEMV and writes per-workgroup partial
// sums of x^2 (one element per thread: launch ceil(hidden/256) x 256).
__device__ void embed_body(const EmbedArgs &a) {
    __shared__ float red[4];
    // the arguments in one batch of scalar loads, so the position's load
    // (then the token's, then the row's) starts after one round trip; an
    // empty asm that emits nothing
    asm volatile("" ::"s"(a.x), "s"(a.table), "s"(a.tokens), "s"(a.ctl), "s"(a.xq_out), "s"(a.ss_out), "s"(a.gamma),
                 "s"(a.hidden), "s"(a.row_bytes), "s"(a.fmt));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tok = a.tokens[a.ctl->pos];
    const uint8_t *row = a.table + (size_t)tok * a.row_bytes;
    const uint32_t i = blockIdx.x * 256u + (uint32_t)tid; // launched with 256 threads (red[] holds 4 waves)
    const bool ok = i < a.hidden;
    const float v = ok ? deq_elem(a.fmt, row, i) : 0.0f;
    if (ok) a.x[i] = v;
    if (a.xq_out) {
        quant16(v * (ok ? a.gamma[i] : 0.0f), ok, a.xq_out, a.hidden, i, lane);
        const float sq = wave_sum(v * v);
        if (lane == 0) red[wave] = sq;
        __syncthreads();
        if (tid == 0) a.ss_out[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
    }
}

// XQ of x (times gamma when given), one element per thread, 256 threads per
// workgroup; partial sums of x^2 per workgroup.
__device__ void quant_act_body(const QActArgs &a) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t i = blockIdx.x * blockDim.x + (uint32_t)tid;
    const bool ok = i < a.n;
    const float v = ok ? a.x[i] : 0.0f;
    const float g = (ok && a.gamma) ? a.gamma[i] : 1.0f;
    quant16(v * g, ok, a.xq_out, a.n, i, lane);
    const float sq = wave_sum(v * v);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (tid == 0 && a.ss_out) a.ss_out[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// cache[pos] <- k, v (rounded to binary16 when kv_f16).
__device__ void kv_store_body(const KvStoreArgs &a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.kv_dim) return;
    const size_t off = (size_t)a.ctl->pos * a.kv_dim + i;
    if (a.kv_f16) {
        ((uint16_t *)a.k_cache)[off] = f32_to_f16(a.k[i]);
        ((uint16_t *)a.v_cache)[off] = f32_to_f16(a.v[i]);
    } else {
        ((float *)a.k_cache)[off] = a.k[i];
        ((float *)a.v_cache)[off] = a.v[i];
    }
}

__device__ void dequant_body(const DequantArgs &a) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n_elems;
         i += (uint64_t)gridDim.x * blockDim.x)
        a.out[i] = deq_elem(a.fmt, a.blocks, i);
}

// One thread per block.
__device__ void quantize_body(const QuantArgs &a) {
    const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= a.n_blocks) return;
    const int qk = fmt_qk(a.fmt), bb = fmt_bytes(a.fmt);
    const float *x = a.x + b * (uint64_t)qk;
    uint8_t *out = a.out + b * (uint64_t)bb;
    switch (a.fmt) {
    case F32: *(float *)out = x[0]; break;
    case F16: wr16(out, f32_to_f16(x[0])); break;
    case Q4_0: quant_q4_0(x, out); break;
    case Q4_1: quant_q4_1(x, out); break;
    case Q5_0: quant_q5_0(x, out); break;
    case Q5_1: quant_q5_1(x, out); break;
    case Q8_0: quant_q8_0(x, out); break;
    case Q4_K: quant_q4_k(x, out); break;
    case Q5_K: quant_q5_k(x, out); break;
    case Q8_K: quant_q8_k(x, out); break;
    default: quant_q6_k(x, out); break;
    }
}

// out[i] = mean + std * z_i; z from Box-Muller on two 24-bit uniforms drawn
// from mix64(key + pair index).  Counter-based: any element can be generated
// independently of the others.
__device__ void fill_normal_body(const FillArgs &a) {
    for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * p < a.n;
         p += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = mix64(a.key + p * 0x9E3779B97F4A7C15ull);
        const float u1 = ((float)(uint32_t)(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
        const float u2 = (float)(uint32_t)((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        const float rad = sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.283185307179586f * u2, &sn, &cs);
        a.out[2 * p] = a.mean + a.std * (rad * cs);
        if (2 * p + 1 < a.n) a.out[2 * p + 1] = a.mean + a.std * (rad * sn);
    }
}

} // namespace ifr

/*
 * CPU oracle for the inferi batch-1 GGUF decode token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libinferi_hip.so) never
 * links, loads or calls it, and there is no CPU fallback built from it.
 *
 * Every function restates the reference's algorithm (dimforge/inferi, Rust)
 * and cites the file:line it follows, relative to the reference root.  Where
 * the reference's CPU path and its GPU path disagree (eps, RoPE theta, softmax
 * normalisation), the GPU path's semantics are used, because that is the path
 * being replaced.  Accumulations use double precision, as the reference's own
 * GEMV test oracle does (crates/inferi/src/ops/gemv_quant.rs:444-456).
 *
 * Parity pins (each checked by tests/test_oracle_*.py):
 *   decode_f16          exhaustive vs numpy float16->float32 (all 65536 codes)
 *   encode_f16          vs numpy float32->float16 (RNE) on 2^20 values + edges
 *   get_scale_min_k4    round trip through an independent 12-byte packer
 *   dequant_*           hand-built known-answer blocks with closed forms
 *   quantize_*          round-trip error bounds; bytes decode to the input grid
 *   gemv_*              x = e_k selects column k exactly; numpy f64 matmul
 *   rms_norm            constant-vector closed form; scale invariance
 *   rope                pos 0 identity; norm preservation; cos/sin closed form
 *   silu_mul            scipy.special.expit closed form
 *   attention           pos 0 -> v0; equal keys -> mean(V); numpy brute force
 *   argmax              lowest index among equal maxima
 *   forward             numpy f64 re-derivation on a tiny model; zero-layer
 *                       model reduces to head(rmsnorm(embedding))
 */
#ifndef INFERI_ORACLE_H
#define INFERI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (crates/inferi/src/gguf.rs:74-104). */
enum {
    IFO_F32 = 0,
    IFO_F16 = 1,
    IFO_Q4_0 = 2,
    IFO_Q4_1 = 3,
    IFO_Q5_0 = 6,
    IFO_Q5_1 = 7,
    IFO_Q8_0 = 8,
    IFO_Q4_K = 12,
    IFO_Q5_K = 13,
    IFO_Q6_K = 14,
    IFO_Q8_K = 15,
};

/* Elements and bytes per block (quantization.rs:42-45, 217-222, 262-268, 335-340). */
int ifo_block_elems(int dtype);
int ifo_block_bytes(int dtype);

/* quantization.rs:405-422 */
float ifo_decode_f16(uint16_t h);
/* Round-to-nearest-even binary32 -> binary16 (not in the reference; the
 * quantizers and the f16 KV cache need it). */
uint16_t ifo_encode_f16(float f);
void ifo_decode_f16_array(const uint16_t *h, float *out, size_t n);
void ifo_encode_f16_array(const float *f, uint16_t *out, size_t n);

/* quantization.rs:394-402 */
void ifo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);

/* One block each: quantization.rs:47-55, 287-330, 224-257, 358-392. */
void ifo_dequant_q8_0(const uint8_t *blk, float *y);
void ifo_dequant_q4_k(const uint8_t *blk, float *y);
void ifo_dequant_q5_k(const uint8_t *blk, float *y);
void ifo_dequant_q6_k(const uint8_t *blk, float *y);
void ifo_dequant_q4_0(const uint8_t *blk, float *y);
void ifo_dequant_q4_1(const uint8_t *blk, float *y);
void ifo_dequant_q5_0(const uint8_t *blk, float *y);
void ifo_dequant_q5_1(const uint8_t *blk, float *y);
void ifo_dequant_q8_k(const uint8_t *blk, float *y);
/* n_elems must be a multiple of the block size; F32/F16 are accepted too. */
int ifo_dequant(int dtype, const void *data, size_t n_elems, float *y);

/* Quantizers (the reference has none: see oracle.c for the algorithm). */
int ifo_quantize(int dtype, const float *x, size_t n_elems, void *out);

/* y = W x, f64 accumulation over a dense f32 matrix (gemv_quant.rs:444-456). */
void ifo_gemv_f64(const float *w, int rows, int cols, const float *x, float *y);
/* y = deq(W) x over GGUF blocks, f64 accumulation, row-parallel over threads. */
int ifo_gemv_quant(int dtype, const void *w, int rows, int cols, const float *x,
                   float *y, int nthreads);

/* rms_norm shader (inferi-shaders/src/rms_norm.rs:112-120); eps from config. */
void ifo_rms_norm(float *out, const float *x, const float *w, int n, float eps);
/* rope shader (inferi-shaders/src/rope.rs:51-92), Original (adjacent pairs)
 * and NeoX (rope.rs:97-141) variants.  k may be NULL when k_len == 0. */
void ifo_rope(int neox, float *q, int q_len, float *k, int k_len, int head_size,
              int pos, float base_freq);
/* silu shader (inferi-shaders/src/silu.rs:24-53): h1 <- h2 * h1/(1+exp(-h1)). */
void ifo_silu_mul(float *h1, const float *h2, int n);
/* x += b (vortx OpAssign::Add, context.rs:516-530). */
void ifo_add(float *x, const float *b, int n);

/* Decode attention for one token (ops/batched_multiquery_attention.rs:191-245,
 * fused_attention.rs:66-241).  Caches are [max_pos][kv_dim] row-major; kv_f16
 * selects binary16 storage (as uint16_t) instead of f32. */
typedef struct {
    uint32_t seq_len, kv_dim, kv_mul, n_heads, head_size, pos;
} ifo_attn_params;
void ifo_attention(const ifo_attn_params *p, const float *q, const void *k_cache,
                   const void *v_cache, int kv_f16, float *out);

/* GEMV accumulation of ifo_gemv_quant and the model forward: 0 (default)
 * f64 rounded once; 1 f32 left to right (the reference CPU path's order). */
void ifo_set_f32_accum(int on);

/* models/sampler.rs:54-56: index of the maximum, lowest index on ties. */
int ifo_argmax(const float *v, int n);

/* SoftMax::run_cpu (ops/softmax.rs:130-143), in place, f32 left-to-right. */
void ifo_softmax(float *v, int n);
/* Sampler::sample_mult (models/sampler.rs:60-76). */
int ifo_sample_mult(const float *p, int n, float coin);
/* Sampler::sample_topp (models/sampler.rs:83-131) with vocab_size = n.
 * Returns -1 where the reference has no candidate to sort (it panics);
 * *last and *cum (when not NULL) receive the truncation position in the
 * sorted list and the cumulative probability the coin is scaled by. */
int ifo_sample_topp(const float *p, int n, float topp, float coin, int *last, float *cum);
/* Sampler::sample (models/sampler.rs:32-52) with the coin given instead of
 * drawn; logits are overwritten as the reference overwrites them. */
int ifo_sample(float *logits, int n, float temperature, float topp, float coin);

/* ---- Llama-style model forward (models/llama2/transformer.rs:409-481) ---- */
typedef struct {
    int hidden, ffn, n_layers, n_heads, n_kv_heads, vocab, max_pos;
    float rope_theta, rms_eps;
    int kv_f16; /* 1: K/V rounded to binary16 at store time */
    int rope_neox; /* 1: NeoX pairs (LlamaModelType::Qwen2, models/llama2/mod.rs:25-30) */
} ifo_config;

typedef struct {
    int dtype;        /* GGUF type id */
    const void *data; /* GGUF blocks, row-major [rows][cols/QK] */
    int rows, cols;
} ifo_tensor;

typedef struct {
    ifo_tensor attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down;
    const float *attn_norm, *ffn_norm;
    /* Qwen2's QKV biases (transformer.rs:434-442); NULL when absent */
    const float *q_bias, *k_bias, *v_bias;
} ifo_layer;

typedef struct {
    ifo_config cfg;
    ifo_tensor token_embd; /* [vocab][hidden] */
    ifo_tensor output;     /* [vocab][hidden] */
    const float *output_norm;
    const ifo_layer *layers; /* n_layers entries */
} ifo_model;

typedef struct ifo_state ifo_state;
ifo_state *ifo_state_new(const ifo_config *cfg);
void ifo_state_free(ifo_state *s);
/* One decode step; writes vocab logits.  nthreads <= 0 uses all cores. */
int ifo_forward(const ifo_model *m, ifo_state *s, int token, int pos, float *logits,
                int nthreads);
/* Access to the state for checks: which = 0 x, 1 k_cache layer, 2 v_cache layer. */
const void *ifo_state_buffer(const ifo_state *s, int which, int layer);

/* CPU baseline (oracle/ref_shaders.c): the reference's GEMV and decode
 * attention shader decompositions restated on host threads.  ifo_ref_gemv:
 * y[rows] = W x for Q4_K, Q5_K (cols % 256), Q6_K (block pairs, cols % 512)
 * or Q8_0 (block pairs, cols % 128), rows % 4 == 0.  ifo_ref_attention:
 * one query head per workgroup over cache rows 0..pos (f16 caches
 * [pos + 1][n_kv_heads * head_size]), out[n_heads * head_size].  Return 0,
 * or -1 for a shape the shaders do not take. */
int ifo_ref_gemv(int32_t dtype, uint32_t rows, uint32_t cols, const void *w, const float *x, float *y, int nthreads);
int ifo_ref_attention(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, uint32_t n_heads,
                      uint32_t n_kv_heads, uint32_t head_size, uint32_t pos, float *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif

/*
 * inferi_hip — C ABI of the MI355X (gfx950) backend for inferi's batch-1
 * GGUF decode token loop.
 *
 * This header is the drop-in boundary.  Every entry point below replaces one
 * call of the reference's op/model API (dimforge/inferi, Rust); the comment on
 * each names the reference function (file:line, relative to the reference
 * root) whose arguments and semantics it keeps.
 *
 * Conventions (mirroring crates/inferi/src/context.rs:106-130):
 *   - Every call returns an ifr_status; on failure ifr_last_error() says why.
 *     Contract violations that the reference assert!s on (shape, rank,
 *     contiguity: ops/gemv_quant.rs:197-201, ops/rope.rs:39-44) return
 *     IFR_EINVAL instead of aborting.
 *   - Op calls are asynchronous: they enqueue kernels on the context's one
 *     HIP stream, in call order, and complete at ifr_sync() or at an
 *     ifr_download(), which waits for everything queued before it.
 *   - Pointers named dev_* or documented as device pointers are device
 *     memory owned by the caller (allocate with ifr_alloc or any hipMalloc);
 *     the library never frees what it did not allocate.
 *   - One context per thread; a context is not thread-safe.
 */
#ifndef INFERI_HIP_H
#define INFERI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFR_API __attribute__((visibility("default")))

typedef int32_t ifr_status;
#define IFR_OK 0
#define IFR_EINVAL 1       /* bad argument: shape, alignment, dtype, null pointer */
#define IFR_EUNSUPPORTED 2 /* valid for the reference, not implemented here */
#define IFR_EHIP 3         /* a HIP runtime call failed */
#define IFR_ENOMEM 4       /* device allocation failed */

/* GGUF tensor type ids (crates/inferi/src/gguf.rs:74-104). */
#define IFR_F32 0
#define IFR_F16 1
#define IFR_Q4_0 2
#define IFR_Q4_1 3
#define IFR_Q5_0 6
#define IFR_Q5_1 7
#define IFR_Q8_0 8
#define IFR_Q4_K 12
#define IFR_Q5_K 13
#define IFR_Q6_K 14
#define IFR_Q8_K 15

/* RoPEVariant (crates/inferi/src/ops/rope.rs:7-13). */
#define IFR_ROPE_ORIGINAL 0
#define IFR_ROPE_NEOX 1

/* Device-resident op parameter structs; same field order and types as the
 * reference's #[repr(C)] structs, so a buffer written for one is valid for
 * the other. */
typedef struct { float nudge_factor; } ifr_rms_norm_config; /* RmsNormConfig, inferi-shaders/src/rms_norm.rs:24-26 */
typedef struct {
    uint32_t head_size, kv_dim, pos;
    float base_freq;
} ifr_rope_config; /* RoPEConfig, inferi-shaders/src/rope.rs:21-26 */
typedef struct {
    uint32_t seq_len, kv_dim, kv_mul, n_heads, head_size, pos;
} ifr_attn_params; /* AttentionParams, inferi-shaders/src/batched_multiquery_attention.rs:18-31 */

typedef struct ifr_ctx ifr_ctx;

/* ---------------------------------------------------------------- context */

/* Opens device `device`, creates the context's stream and loads the gfx950
 * code object (`code_object_path`, or NULL for inferi_kernels.hsaco beside
 * this library).  Replaces LlmOps::new (crates/inferi/src/context.rs:58-85),
 * which loads every compiled kernel of the backend. */
IFR_API ifr_status ifr_create(int32_t device, const char *code_object_path, ifr_ctx **out);
IFR_API void ifr_destroy(ifr_ctx *ctx);
/* Message of the last failed call on this context (or, when ctx is NULL, of
 * the last failed call made without a context on this thread: ifr_create,
 * ifr_gguf_*). */
IFR_API const char *ifr_last_error(const ifr_ctx *ctx);
/* Device name and compute-unit count, for reports. */
IFR_API ifr_status ifr_device_info(ifr_ctx *ctx, char *name, size_t name_len, int32_t *n_cu);

/* Knobs (no reference counterpart): "gemv_max_grid" sets the number of GEMV
 * workgroups (0 = chosen by shape, the default); "gemv_waves" caps the
 * waves per GEMV workgroup (1, 2, 4, 8 or 16; 0 = chosen by shape); either
 * one also turns off the one-item GEMV forms.  "gemv_exact" = 1
 * makes every GEMV keep x in fp32 and use fp32 FMAs, instead of the default
 * path that takes x as 22-bit fixed point per 16 elements and multiplies
 * with int8 dot products (see ifr_quantize_activation).  "gemv_grp" selects
 * the one-item forms of the grouped decode GEMVs (bit 0 attention output,
 * a default; bit 1 FFN down; bit 2 gate/up, bit 3 with 16 waves of two
 * rows; bit 4 the output head; bit 5, a default, gate/up with h in f32 and
 * the FFN down GEMV quantizing h itself; bit 6, a default, the Q6_K output
 * head in 4-wave workgroups of up to 256 VGPRs, two per CU; bit 7, a
 * default, four rows per wave in the Q4_K one-item gate/up form; bit 8 four
 * rows per wave in the Q4_K one-item plain and QKV forms).  Default 225.
 * "pf_chunk"
 * sets the prompt tokens per ifr_llama2_prefill pass (a multiple of 64, at
 * most 16384; 0 = 4096), read at a state's first prefill.  "pf_tile"
 * selects the prefill GEMM's tiles: 0 (the default) 256 x 256 tiles where a
 * product has at least 128 of them, else 128 x 128 tiles; 128 or 256 forces
 * one form.  "pf_ws" = 1 (the default) runs the Q4_K products on 256 x 256
 * tiles in the warp-specialized form (eight MFMA waves and four waves that
 * load and dequantize the tiles), 0 in the eight-wave form where every wave
 * does both.  Every form sums each output element's products in the same
 * order, so the results do not depend on the form or the pass length.
 * "pf_rope_fuse" = 1 (the default) lets the warp-specialized Q/K/V product
 * add the biases, apply RoPE and store k and v to the cache in its epilogue
 * (pairs (2i, 2i + 1) only), 0 leaves that to a kernel of its own; both
 * give the same results bit for bit.
 * A captured decode step is captured again after any option change. */
IFR_API ifr_status ifr_set_option(ifr_ctx *ctx, const char *key, int64_t value);
/* Reads an option (no reference counterpart): any key ifr_set_option takes. */
IFR_API ifr_status ifr_get_option(ifr_ctx *ctx, const char *key, int64_t *value);

/* ----------------------------------------------------------------- memory */

/* Device buffers (vortx Tensor storage in the reference).  Allocations are
 * 256-byte aligned. */
IFR_API ifr_status ifr_alloc(ifr_ctx *ctx, size_t bytes, void **dev_ptr);
IFR_API ifr_status ifr_free(ifr_ctx *ctx, void *dev_ptr);
/* Host -> device; returns once the host buffer may be reused
 * (GpuBackend::write_buffer in crates/inferi-chat/src/chat_llama2.rs:210-216). */
IFR_API ifr_status ifr_upload(ifr_ctx *ctx, void *dev_dst, const void *host_src, size_t bytes);
/* Device -> host after all queued work (GpuBackend::read_buffer,
 * crates/inferi-chat/src/chat_llama2.rs:250-252). */
IFR_API ifr_status ifr_download(ifr_ctx *ctx, void *host_dst, const void *dev_src, size_t bytes);
IFR_API ifr_status ifr_memset(ifr_ctx *ctx, void *dev_dst, int32_t byte_value, size_t bytes);
/* Waits for all queued work (LlmContext::submit + synchronize,
 * crates/inferi/src/context.rs:117-130). */
IFR_API ifr_status ifr_sync(ifr_ctx *ctx);
/* Timing on the context's stream: records event `slot` (0..15) and returns
 * the milliseconds between two recorded slots (waits for the later one). */
IFR_API ifr_status ifr_event_record(ifr_ctx *ctx, int32_t slot);
IFR_API ifr_status ifr_event_elapsed(ifr_ctx *ctx, int32_t start_slot, int32_t end_slot, float *ms);

/* -------------------------------------------------------------------- ops */

/* out[0..n_elems) = dequantize(blocks), bit-exact with the reference's
 * Block*::dequantize (crates/inferi/src/quantization.rs:47-55, 66-82,
 * 94-112, 123-143, 155-177, 204-212, 224-257, 287-330, 358-392) and
 * decode_f16 (:405-422).  dtype: any IFR_* above;
 * n_elems a multiple of the block size. */
IFR_API ifr_status ifr_dequant(ifr_ctx *ctx, float *out, const void *blocks, int32_t dtype, uint64_t n_elems);

/* out[rows] = dequant(W)[rows x cols] . v[cols], fp32 accumulation.
 * W is `rows` rows of cols/QK consecutive GGUF blocks, exactly as a GGUF file
 * stores them.  Replaces LlmContext::matmul_quant_assign
 * (crates/inferi/src/context.rs:441-456) -> GemvQuant::launch
 * (crates/inferi/src/ops/gemv_quant.rs:183-340).
 * The product runs on the integer path (see ifr_quantize_activation) unless
 * the "gemv_exact" option is set; on it the GEMV kernel quantizes v into its
 * LDS itself (one launch, nothing allocated).
 * Requirements: cols % QK == 0; cols <= 18432 (integer path; 16320 with
 * "gemv_exact"), as x is staged in one workgroup's LDS; W 16-byte aligned
 * for Q4_K and Q5_K, 4-byte aligned for the other formats (GGUF data is
 * 32-aligned).  dtype Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K or
 * Q8_K (the reference's GEMV shaders, crates/inferi-shaders/src/gemv_quant_*.rs). */
IFR_API ifr_status ifr_matmul_quant(ifr_ctx *ctx, float *out, const void *w, int32_t dtype, uint32_t rows,
                                    uint32_t cols, const float *v);

/* ifr_matmul_quant without allocation (no counterpart in the reference): for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments and results as ifr_matmul_quant, computed in two launches (the
 * activation quantization, then the GEMV on it) whose quantized copy of v
 * lives in a fixed device array of 65536 bytes (one per GPU, held until the
 * process ends); the call makes no hipMalloc, hipFree or other allocating
 * call.  cols whose
 * quantized input would not fit (cols > 18724 on the integer path) return
 * IFR_EINVAL.  Every call on one GPU shares that array: calls that overlap
 * on one GPU (two streams, two contexts) race; calls queued on one context's
 * stream are ordered and safe. */
IFR_API ifr_status ifr_matmul_quant_noalloc(ifr_ctx *ctx, float *out, const void *w, int32_t dtype, uint32_t rows,
                                            uint32_t cols, const float *v);

/* Activation pre-quantization (no reference counterpart: the reference
 * multiplies f32 vectors).  A caller that multiplies several matrices by the
 * same vector quantizes it once into `xq` (ifr_activation_bytes(n) bytes,
 * 16-byte aligned): 16-value groups of 22-bit fixed point held as three int8
 * digit planes, x rounded by at most max|x| of its group * 2.4e-7 (about
 * the rounding of an f32 significand at the group's largest value); x is multiplied
 * by gamma first when gamma is not NULL, and ss_out (when not NULL) receives
 * ceil(n/256) partial sums of x^2.  ifr_matmul_quant_xq is then
 * ifr_matmul_quant on the quantized vector (the kernel the decode step uses);
 * ifr_matmul_quant itself quantizes v and calls it.  n, cols: multiples of 32. */
IFR_API uint64_t ifr_activation_bytes(uint32_t n);
IFR_API ifr_status ifr_quantize_activation(ifr_ctx *ctx, void *xq, const float *x, const float *gamma, uint32_t n,
                                           float *ss_out);
IFR_API ifr_status ifr_matmul_quant_xq(ifr_ctx *ctx, float *out, const void *w, int32_t dtype, uint32_t rows,
                                       uint32_t cols, const void *xq);

/* out = (value * (1/sqrt(sum(value^2)/n + cfg.nudge_factor))) * weight, with
 * cfg a device pointer.  LlmContext::rms_norm_assign
 * (crates/inferi/src/context.rs:336-353) -> rms_norm shader
 * (inferi-shaders/src/rms_norm.rs:81-121). */
IFR_API ifr_status ifr_rms_norm(ifr_ctx *ctx, const ifr_rms_norm_config *dev_cfg, float *out, const float *value,
                                const float *weight, uint32_t n);

/* in_out_a += b.  LlmContext::add_assign (crates/inferi/src/context.rs:516-530). */
IFR_API ifr_status ifr_add(ifr_ctx *ctx, float *in_out_a, const float *b, uint32_t n);

/* Rotary embedding in place on q[0..q_len) and, for pair starts 2i < cfg.kv_dim,
 * on k.  cfg is a device pointer (pos is device-resident, as in the
 * reference).  LlmContext::rope (crates/inferi/src/context.rs:687-704) ->
 * RoPE::launch (crates/inferi/src/ops/rope.rs:25-95). q_len even. */
IFR_API ifr_status ifr_rope(ifr_ctx *ctx, int32_t variant, const ifr_rope_config *dev_cfg, float *q,
                            uint32_t q_len, float *k, uint32_t k_len);

/* in_out_h1 <- h2 * (h1 / (1 + exp(-h1))).  LlmContext::silu
 * (crates/inferi/src/context.rs:706-719) -> silu shader
 * (inferi-shaders/src/silu.rs:24-53). */
IFR_API ifr_status ifr_silu(ifr_ctx *ctx, float *in_out_h1, const float *h2, uint32_t n);

/* Strided views of the same four ops.  The reference's op shaders index
 * every operand through its tensor layout (shape.it(..): rms_norm.rs:118-119,
 * rope.rs:81-87 and 129-132, silu.rs:46-47), so an operand may be a view of
 * a larger buffer.  Here a view is (offset, stride) in elements: element i
 * of the operand is base[offset + i * stride].  As in the reference, a RoPE
 * pair's second element lies 1 (Original) or head_size / 2 (NeoX) elements
 * after its first in memory, whatever the stride.  The caller sizes the
 * buffers; the library cannot check views against them. */
typedef struct {
    int64_t offset;
    int64_t stride;
} ifr_view;
IFR_API ifr_status ifr_rms_norm_view(ifr_ctx *ctx, const ifr_rms_norm_config *dev_cfg, float *out, ifr_view out_v,
                                     const float *value, ifr_view value_v, const float *weight, ifr_view weight_v,
                                     uint32_t n);
IFR_API ifr_status ifr_add_view(ifr_ctx *ctx, float *in_out_a, ifr_view a_v, const float *b, ifr_view b_v, uint32_t n);
IFR_API ifr_status ifr_rope_view(ifr_ctx *ctx, int32_t variant, const ifr_rope_config *dev_cfg, float *q, ifr_view q_v,
                                 uint32_t q_len, float *k, ifr_view k_v, uint32_t k_len);
IFR_API ifr_status ifr_silu_view(ifr_ctx *ctx, float *in_out_h1, ifr_view h1_v, const float *h2, ifr_view h2_v,
                                 uint32_t n);

/* Decode attention of one token over the KV cache:
 * xb[h] = softmax_t((q[h] . k_t[h/kv_mul]) / sqrt(head_size)) . v_t, t in [0, pos].
 * Caches are [seq_len][kv_dim] row-major, kv_dtype IFR_F32 (the reference's
 * layout) or IFR_F16.  `params` (host) sizes the launch; `dev_params` is the
 * device copy the kernel reads.  BatchedMultiqueryAttention::launch
 * (crates/inferi/src/ops/batched_multiquery_attention.rs:87-110) ->
 * FusedAttention::launch (:27-76), which, like this call, takes any kv_mul.
 * head_size is a multiple of 8, at most 128; pos below 2^30. */
IFR_API ifr_status ifr_attention(ifr_ctx *ctx, const ifr_attn_params *params, const ifr_attn_params *dev_params,
                                 const float *q, const void *key_cache, const void *value_cache, int32_t kv_dtype,
                                 float *xb);

/* dev_index[0] = index of the largest of v[0..n), lowest index on ties.
 * Replaces the host-side Sampler::sample_argmax
 * (crates/inferi/src/models/sampler.rs:54-56) so the logits never leave
 * the device. */
IFR_API ifr_status ifr_argmax(ifr_ctx *ctx, const float *v, uint32_t n, uint32_t *dev_index);

/* Sampler::sample (crates/inferi/src/models/sampler.rs:32-52) on the device,
 * with the coin passed in instead of drawn by rand::random() (:41):
 *   temperature == 0: dev_index[0] = argmax(logits) (sample_argmax, :54-56);
 *   otherwise probs = softmax(logits / temperature) (:38-39 and
 *   SoftMax::run_cpu, crates/inferi/src/ops/softmax.rs:130-143; probs may
 *   alias logits, which is what the reference does to its logits), then
 *   dev_index[0] = sample_mult(probs, coin) (:60-76) when topp <= 0 or
 *   topp >= 1, else sample_topp(probs, coin) (:83-131).
 * dev_coin points to one float in [0, 1) in device memory.  The running sums
 * the choice compares are exact (probabilities truncated to multiples of
 * 2^-40), so the result is deterministic; it can differ from the reference's
 * f32 running sums only for a coin within their rounding of a boundary.
 * When no probability reaches the top-p cutoff (1 - topp) / (n - 1), where
 * the reference fails, the most probable token is returned.
 * n <= 262144; logits and probs 16-byte aligned. */
IFR_API ifr_status ifr_sample(ifr_ctx *ctx, const float *logits, float *probs, uint32_t n, float temperature,
                              float topp, const float *dev_coin, uint32_t *dev_index);

/* Prompt-path GEMM (no reference counterpart; the reference multiplies
 * the prompt one token at a time through GemvQuant,
 * crates/inferi/src/ops/gemv_quant.rs:183-340):
 * y[m][rows] (+)= x[m][cols] . dequant(W)[rows x cols]^T, x f16 (IEEE
 * binary16, row-major, 16-byte aligned), W rows of any quantized GGUF type
 * (Q4_0 .. Q8_K) or F16/F32 as a GGUF file stores them (16-byte aligned for
 * Q4_K, Q5_K, F16 and F32, 4 otherwise; cols a multiple of 64 and of the
 * block size), y f32 row-major with leading dimension `rows`.  The weights
 * are dequantized tile by tile with the reference's arithmetic to f16 inside
 * the kernel (nothing is allocated) and multiplied on the matrix cores with
 * f32 accumulation (option pf_tile picks the tile size).  accumulate != 0
 * adds to y. */
IFR_API ifr_status ifr_gemm_quant(ifr_ctx *ctx, float *y, const void *w, int32_t dtype, uint32_t rows, uint32_t cols,
                                  const void *x_f16, uint32_t m, int32_t accumulate);

/* GGUF blocks from f32 values on the device: the deterministic min/max
 * quantizer used for the synthetic models (the reference only dequantizes;
 * crates/inferi/src/quantization.rs:1-426).  dtype any IFR_* type above. */
IFR_API ifr_status ifr_quantize(ifr_ctx *ctx, void *out_blocks, const float *x, int32_t dtype, uint64_t n_elems);

/* Synthetic weights: out[i] = mean + std * z_i, z_i ~ N(0,1) from a
 * counter-based generator keyed by (seed, stream), so a tensor is reproducible
 * from its seed alone. */
IFR_API ifr_status ifr_fill_normal(ifr_ctx *ctx, float *out, uint64_t n, uint64_t seed, uint64_t stream, float mean,
                                   float std);

/* ------------------------------------------------------------ llama model */

/* Llama2Config (crates/inferi/src/models/llama2/cpu.rs:78-141) plus the two
 * choices the reference fixes elsewhere: the KV-cache element type (the
 * reference uses F32, transformer.rs:85-104) and the RoPE variant
 * (models/llama2/mod.rs:25-30). */
typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, vocab, max_pos;
    float rope_theta, rms_eps;
    int32_t kv_dtype;     /* IFR_F16 or IFR_F32 */
    int32_t rope_variant; /* IFR_ROPE_ORIGINAL (llama) */
} ifr_llama2_config;
/* Accepted shapes: head size (hidden / n_heads) a multiple of 8, at most
 * 128; n_heads / n_kv_heads (kv_mul) at most 64; hidden and ffn multiples of
 * 32; max_pos up to 2^30 (the cache is sized to it, as transformer.rs:85-104
 * sizes it to context_length). */

typedef struct ifr_llama2_weights ifr_llama2_weights;
typedef struct ifr_llama2_state ifr_llama2_state;

/* Llama2Weights (crates/inferi/src/models/llama2/transformer.rs:176-196,
 * 294-393): a table of device tensors keyed by GGUF name.  The tensors stay
 * owned by the caller. */
IFR_API ifr_status ifr_llama2_weights_create(ifr_ctx *ctx, const ifr_llama2_config *cfg, ifr_llama2_weights **out);
/* Binds one GGUF tensor ("token_embd.weight", "output_norm.weight",
 * "output.weight", "blk.N.{attn_norm,attn_q,attn_k,attn_v,attn_output,
 * ffn_norm,ffn_gate,ffn_up,ffn_down}.weight", and Qwen2's
 * "blk.N.attn_{q,k,v}.bias") already in device memory.
 * rows/cols follow gguf.rs:591-593 (dims reversed: rows = ne1, cols = ne0);
 * norms and biases are F32 vectors with rows = 1.  A layer with biases adds
 * them to q, k and v before RoPE (transformer.rs:434-442).  Every call
 * starts a new generation of the table: captured decode graphs made before
 * it are rebuilt.  The decode and prefill kernels read the bound buffers
 * directly, so bytes rewritten in place are used by the next call. */
IFR_API ifr_status ifr_llama2_weights_set(ifr_llama2_weights *w, const char *gguf_name, int32_t dtype,
                                          const void *dev_data, uint32_t rows, uint32_t cols);
IFR_API void ifr_llama2_weights_destroy(ifr_llama2_weights *w);

/* Llama2State (crates/inferi/src/models/llama2/transformer.rs:46-137):
 * activations, logits, the KV cache, the device-resident position counter
 * and the token sequence.  Owned by the library. */
IFR_API ifr_status ifr_llama2_state_create(ifr_ctx *ctx, const ifr_llama2_config *cfg, ifr_llama2_state **out);
IFR_API void ifr_llama2_state_destroy(ifr_llama2_state *s);
/* Sets the token sequence to `prompt` (forced tokens, chat_llama2.rs:137-160)
 * and the device position counter to `pos`. */
IFR_API ifr_status ifr_llama2_state_reset(ifr_llama2_state *s, const uint32_t *prompt, uint32_t n_prompt,
                                          uint32_t pos);

/* One decode step at the state's device position p: embeds token[p], runs
 * every layer, the final norm and the output head into the logits, stores
 * argmax(logits) as token[p+1] unless p+1 is a forced prompt position, and
 * advances the position.  Llama2::launch
 * (crates/inferi/src/models/llama2/transformer.rs:409-481) plus the
 * embedding copy and greedy sampling of ChatLlama2::forward_logits
 * (crates/inferi-chat/src/chat_llama2.rs:191-255).  `fused` selects the fused
 * kernels (6 launches per layer) instead of the one-kernel-per-reference-op
 * sequence (14 per layer). */
IFR_API ifr_status ifr_llama2_launch(ifr_ctx *ctx, ifr_llama2_state *s, const ifr_llama2_weights *w, int32_t fused);
/* n_steps decode steps; with use_graph the step is captured once into a HIP
 * graph and replayed (the position lives on the device, so one graph serves
 * every step).  The graph is captured again when it was made for another
 * weights object or before an ifr_llama2_weights_set on this one, or when
 * the options or the sampler changed; a caller that frees or overwrites a
 * bound tensor's memory in place must rebind it (ifr_llama2_weights_set) or
 * pass use_graph = 0. */
IFR_API ifr_status ifr_llama2_generate(ifr_ctx *ctx, ifr_llama2_state *s, const ifr_llama2_weights *w,
                                       uint32_t n_steps, int32_t use_graph);
/* Prompt prefill (the reference runs a prompt through Llama2::launch one
 * token at a time, crates/inferi-chat/src/chat_llama2.rs:137-160): the
 * n_tokens forced prompt tokens at device positions [pos, pos + n_tokens)
 * go through every layer in chunks, with their matrix products as GEMMs on
 * the matrix cores (ifr_gemm_quant) and causal attention over the cache;
 * their KV-cache rows are written and the position advances by n_tokens.
 * No logits are formed: the next decode step, at the prompt's last token,
 * produces them (so the last layer's attention and FFN, whose outputs feed
 * nothing else, are not run).  Waits for queued work (it reads the position).  The
 * attention and FFN matrices may be of any quantized GGUF type that
 * ifr_gemm_quant takes; both RoPE variants and QKV biases are handled. */
IFR_API ifr_status ifr_llama2_prefill(ifr_ctx *ctx, ifr_llama2_state *s, const ifr_llama2_weights *w,
                                      uint32_t n_tokens);
/* Measurement hook (no reference counterpart): enqueues one stage of the
 * fused decode step ("qkv", "attention" = split + merge, "attn_output",
 * "ffn_gate_up", "ffn_down") for every layer in turn, `iters` times, on the
 * context's stream between two HIP events, and returns the average time of
 * one layer's stage in microseconds.  The launches are the decode step's
 * own; they overwrite the state's activations and this position's KV rows,
 * so reset the state before decoding on.  Blocks until done. */
IFR_API ifr_status ifr_llama2_time_stage(ifr_ctx *ctx, ifr_llama2_state *state, const ifr_llama2_weights *weights,
                                         const char *stage, uint32_t iters, float *us_per_launch);

/* Sampling at the end of each decode step, as sample_next_token does
 * (crates/inferi-chat/src/sampler.rs:91-111, with Sampler::new(vocab, 0.7,
 * 0.95)): with temperature != 0 the step chooses token[p+1] by ifr_sample's
 * algorithm instead of the argmax, its probabilities going to the state's
 * "probs" buffer and its coin drawn on the device from (seed, p + 1); forced
 * prompt positions are not sampled.  temperature 0 (the default) restores
 * the argmax.  A captured decode step is captured again. */
IFR_API ifr_status ifr_llama2_set_sampler(ifr_llama2_state *s, float temperature, float topp, uint64_t seed);
/* Copies tokens[start, start+n) of the sequence to the host (waits). */
IFR_API ifr_status ifr_llama2_read_tokens(ifr_llama2_state *s, uint32_t *host, uint32_t start, uint32_t n);
/* Device pointer and size of a state buffer: "x", "logits", "probs", "pos", "tokens",
 * "key_cache" / "value_cache" (of `layer`), "q", "att". */
IFR_API ifr_status ifr_llama2_state_buffer(ifr_llama2_state *s, const char *name, int32_t layer, void **dev_ptr,
                                           size_t *bytes);

/* ------------------------------------------------------------------ GGUF */

/* Gguf::from_bytes (crates/inferi/src/gguf.rs:516-692).  The file is
 * memory-mapped; metadata and tensor infos are parsed as the reference does:
 * the magic in either byte order, typed metadata (MetadataValueType,
 * gguf.rs:388-511), tensor dimensions reversed from GGUF's order into
 * [rows, cols, ...] with unused dimensions 1 (gguf.rs:620-626), tensor data
 * at the aligned end of the infos plus the tensor's offset, the alignment
 * being general.alignment when it is a U32, else 32.  Where the reference
 * panics (a read past the end, rank > 4) or errs (bad magic, unknown value
 * or tensor type) the call returns IFR_EINVAL (ifr_last_error(NULL)).
 * Tensor data pointers point into the mapping and live until ifr_gguf_close. */
typedef struct ifr_gguf ifr_gguf;
/* Metadata value types (gguf.rs MetadataValueType). */
#define IFR_GGUF_U8 0
#define IFR_GGUF_I8 1
#define IFR_GGUF_U16 2
#define IFR_GGUF_I16 3
#define IFR_GGUF_U32 4
#define IFR_GGUF_I32 5
#define IFR_GGUF_F32 6
#define IFR_GGUF_BOOL 7
#define IFR_GGUF_STRING 8
#define IFR_GGUF_ARRAY 9
#define IFR_GGUF_U64 10
#define IFR_GGUF_I64 11
#define IFR_GGUF_F64 12

IFR_API ifr_status ifr_gguf_open(const char *path, ifr_gguf **out);
/* Parses a copy of bytes[0..len) (Gguf::from_bytes on an in-memory file). */
IFR_API ifr_status ifr_gguf_from_bytes(const void *bytes, size_t len, ifr_gguf **out);
IFR_API void ifr_gguf_close(ifr_gguf *g);
IFR_API uint32_t ifr_gguf_version(const ifr_gguf *g);
IFR_API uint32_t ifr_gguf_alignment(const ifr_gguf *g);
/* Metadata keys in file order (a repeated key keeps its first position and
 * its last value, as the reference's map insert does). */
IFR_API uint64_t ifr_gguf_metadata_count(const ifr_gguf *g);
IFR_API const char *ifr_gguf_metadata_key(const ifr_gguf *g, uint64_t i);
/* The value type of key (-1 when absent); for an array, its element type
 * and length; for a string, its byte length. */
IFR_API int32_t ifr_gguf_metadata_type(const ifr_gguf *g, const char *key, int32_t *elem_type, uint64_t *len);
/* A scalar of exactly `type` (the reference's unwrap_u32 / as_f32 are
 * strict): its 1, 2, 4 or 8 little-endian bytes to *out (BOOL: one byte). */
IFR_API ifr_status ifr_gguf_get_scalar(const ifr_gguf *g, const char *key, int32_t type, void *out);
/* A STRING value (not NUL-terminated in the file; the pointer here is). */
IFR_API ifr_status ifr_gguf_get_string(const ifr_gguf *g, const char *key, const char **s, uint64_t *len);
/* An ARRAY: element type and length; for scalar elements, *data points at
 * the packed little-endian elements in the file (unaligned). */
IFR_API ifr_status ifr_gguf_get_array(const ifr_gguf *g, const char *key, int32_t *elem_type, uint64_t *len,
                                      const void **data);
IFR_API ifr_status ifr_gguf_get_array_string(const ifr_gguf *g, const char *key, uint64_t i, const char **s,
                                             uint64_t *len);
/* Tensors in file order; info by name: type id (gguf.rs:74-104), dims in
 * the reference's order, rank, the data in the file and its byte size (NULL
 * and 0 for the types whose data the reference does not read). */
IFR_API uint64_t ifr_gguf_tensor_count(const ifr_gguf *g);
IFR_API const char *ifr_gguf_tensor_name(const ifr_gguf *g, uint64_t i);
IFR_API ifr_status ifr_gguf_tensor_info(const ifr_gguf *g, const char *name, int32_t *dtype, uint64_t dims[4],
                                        uint32_t *rank, const void **data, uint64_t *bytes);

/* GGUF writer (no reference counterpart: the reference only reads).  Writes
 * version 3 with metadata and tensor infos in insertion order and each
 * tensor's data at the next multiple of general.alignment (32 unless set),
 * zero-padded, so the files read back through ifr_gguf_open and the
 * reference's Gguf::from_bytes alike.  Tensor dims are given in the
 * reference's order ([rows, cols, ...]); data is copied. */
typedef struct ifr_gguf_writer ifr_gguf_writer;
IFR_API ifr_status ifr_gguf_writer_create(ifr_gguf_writer **out);
IFR_API void ifr_gguf_writer_destroy(ifr_gguf_writer *w);
/* A scalar (value points at its bytes) or a STRING (value is a C string);
 * setting a key again replaces its value in place. */
IFR_API ifr_status ifr_gguf_writer_set(ifr_gguf_writer *w, const char *key, int32_t type, const void *value);
/* An array of scalars (packed elements) or of STRINGs (const char *const *). */
IFR_API ifr_status ifr_gguf_writer_set_array(ifr_gguf_writer *w, const char *key, int32_t elem_type,
                                             const void *data, uint64_t len);
IFR_API ifr_status ifr_gguf_writer_add_tensor(ifr_gguf_writer *w, const char *name, int32_t dtype, uint32_t rank,
                                              const uint64_t *dims, const void *data, uint64_t bytes);
IFR_API ifr_status ifr_gguf_writer_save(ifr_gguf_writer *w, const char *path);

/* Llama2Config::from_gguf_with_model_type (crates/inferi/src/models/llama2/
 * cpu.rs:74-107): with M = "qwen2" when general.architecture names qwen2
 * (ChatLlm::from_gguf, inferi-chat/src/llm.rs:71-92), else "llama":
 * M.{embedding_length, feed_forward_length, block_count,
 * attention.head_count, attention.head_count_kv, context_length} as U32,
 * vocab = the length of tokenizer.ggml.tokens, M.rope.freq_base (F32,
 * default 10000) and M.attention.layer_norm_rms_epsilon (F32, default 1e-6);
 * max_pos = context_length.  kv_dtype is set to IFR_F32 (the reference's
 * cache), rope_variant to NeoX for qwen2 and the original otherwise
 * (models/llama2/mod.rs:25-30); a caller may change kv_dtype before creating
 * a state. */
IFR_API ifr_status ifr_llama2_config_from_gguf(const ifr_gguf *g, ifr_llama2_config *cfg);
/* Llama2Weights::from_gguf (crates/inferi/src/models/llama2/transformer.rs:
 * 294-393): every tensor the model uses is copied verbatim (GGUF blocks) to
 * device memory that the weights own and free at ifr_llama2_weights_destroy,
 * including blk.N.attn_{q,k,v}.bias when present (Qwen2); output.weight
 * falls back to token_embd.weight when absent (:376-382). */
IFR_API ifr_status ifr_llama2_weights_from_gguf(ifr_ctx *ctx, const ifr_gguf *g, const ifr_llama2_config *cfg,
                                                ifr_llama2_weights **out);

#ifdef __cplusplus
}
#endif
#endif

// Kernel argument blocks shared by the host library and the gfx950 kernels.
// Each kernel takes one of these structs by value; the host passes it through
// hipModuleLaunchKernel's argument buffer, so the layout must be identical on
// both sides (plain C types only).
#pragma once
#include <stdint.h>

namespace ifr {

// GGUF tensor type ids (ggml_type)
enum Fmt : int32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15 };

// GEMV epilogue/prologue modes.
enum GemvMode : int32_t {
    GEMV_PLAIN = 0,  // y[r] = W x
    GEMV_RESID = 1,  // y[r] += W x                       (attention-out / down + residual)
    GEMV_QKV = 2,    // rmsnorm(x) -> [Wq;Wk;Wv] -> RoPE -> q, k/v cache row pos
    GEMV_GATEUP = 3, // rmsnorm(x) -> [Wgate;Wup] interleaved -> h = silu(g) * u
    GEMV_HEAD = 4,   // rmsnorm(x) -> logits = W x, per-workgroup argmax keys
};

// Exact-path GEMV launch geometry per mode, shared by the kernels and the
// host: R rows per wave, W waves per workgroup (a workgroup tile is W*R
// rows).  RESID and GATEUP tiles hold exactly one 16-value output activation
// group (GATEUP's 32 virtual rows are 16 gate/up pairs).
struct GemvGeomT {
    int R, W;
};
constexpr GemvGeomT gemv_geom(int mode) {
    return mode == GEMV_RESID ? GemvGeomT{2, 8} : mode == GEMV_GATEUP ? GemvGeomT{2, 16} : GemvGeomT{2, 4};
}

// Device copies of the C ABI's op configs (same layout as ifr_rms_norm_config
// and ifr_rope_config in include/inferi_hip.h).
struct ifr_rms_cfg_dev {
    float nudge_factor;
};
struct ifr_rope_cfg_dev {
    uint32_t head_size, kv_dim, pos;
    float base_freq;
};

// Device-side control block of a decode state: the position and the number
// of forced (prompt) tokens.
struct StepCtl {
    uint32_t pos;
    uint32_t n_forced;
    uint32_t max_pos;
    uint32_t pad;
};

// Integer-path GEMV, one-item form (device/gemv.h gemv_one_body): waves per
// workgroup (two rows each).
constexpr uint32_t GEMV_ONE_WAVES = 4;

// Integer-path GEMV: at most this many K-slices and 16 waves per workgroup.
constexpr uint32_t GEMV_KS_MAX = 4;
constexpr uint32_t GEMV_INT_MAX_WAVES = 16;

struct GemvArgs {
    const uint8_t *w0, *w1, *w2; // matrices: PLAIN/RESID/HEAD w0; QKV q,k,v; GATEUP gate,up
    uint32_t rows0, rows1, rows2; // rows of each matrix
    uint32_t total_rows;          // virtual rows covered by the launch
    uint32_t cols;                // K
    uint32_t nb;                  // blocks per row
    uint32_t row_bytes;           // bytes per row
    uint32_t n_ss;                // integer path + RMSNorm: number of partial sums in ss_part
    const float *x;      // exact path: input vector [cols]
    const float *gamma;  // exact path: RMSNorm weight [cols]
    const uint8_t *xq;   // integer path: the input, quantized (XQ layout, device/gemv.h)
    const float *ss_part; // integer path + RMSNorm: partial sums of x^2 of the input
    float eps;           // RMSNorm epsilon
    uint32_t ks;         // integer path: K-slices per workgroup (1, 2 or 4)
    float *y;            // PLAIN/HEAD: out[rows]; RESID: x (+=); QKV: q; GATEUP: h
    uint8_t *xq_out;     // RESID/GATEUP: the output quantized for the next GEMV (may be null)
    float *ss_out;       // RESID: per-tile partial sums of x^2 of the output
    const float *gamma_next; // RESID: RMSNorm weight of the next GEMV, applied before quantizing
    const float *rope_tab; // QKV: theta of each pair within a head [head_size/2]
    void *k_cache;       // QKV: cache base of this layer, [max_pos][kv_dim]
    void *v_cache;
    const StepCtl *ctl;  // QKV: position
    uint32_t kv_dim, head_size;
    int32_t kv_f16;      // QKV: cache element type
    uint32_t nwaves;     // integer path: waves per workgroup (blockDim.x / 64)
    uint64_t *part_keys; // HEAD: one argmax key per workgroup (may be null)
    const float *q_bias, *k_bias, *v_bias; // QKV: Qwen2 biases (may be null)
    int32_t neox;        // QKV: RoPE pairs (j, j + hs/2) instead of (2j, 2j+1)
};

struct AttnArgs {
    const float *q;           // [n_heads * head_size]
    const void *k_cache;      // [seq_len][kv_dim]
    const void *v_cache;
    float *out;               // [n_heads * head_size]
    uint8_t *xq_out;          // merge: the output quantized for the next GEMV (may be null)
    float *part_o;            // [n_heads][n_splits][head_size]
    float *part_ml;           // [n_heads][n_splits][2]
    const uint32_t *pos;      // device position
    uint32_t kv_dim;
    uint32_t n_splits;        // gridDim.y
    uint32_t seq_cap;         // positions attended never exceed this (cache rows)
    uint32_t spec_rows;       // the host's bound on pos + 1: the first batch is loaded before pos is read
                              // when n_splits batches cover it (any pos stays correct, a larger one is slower)
    uint32_t n_out;           // n_heads * head_size (length of out and xq_out)
    uint32_t head_size;       // a multiple of 8, at most 128
    uint32_t kv_mul;          // query heads per KV head
    uint32_t n_sub;           // workgroups per KV head and split (gridDim.x / n_kv_heads)
};

struct EltArgs {
    float *a;
    const float *b;
    const float *w;
    const void *cfg; // op-specific device config
    float *k;
    uint32_t n, n2;
    int32_t variant;
    uint32_t pad;
    // element strides of the views a, b, w and k (the pointers already at
    // the views' first elements); 1 for contiguous vectors
    int64_t sa = 1, sb = 1, sw = 1, sk = 1;
};

struct DequantArgs {
    float *out;
    const uint8_t *blocks;
    uint64_t n_elems;
    int32_t fmt;
    uint32_t pad;
};

struct QuantArgs {
    uint8_t *out;
    const float *x;
    uint64_t n_blocks;
    int32_t fmt;
    uint32_t pad;
};

struct FillArgs {
    float *out;
    uint64_t n;
    uint64_t key;
    float mean, std;
};

struct ArgmaxArgs {
    const float *v;
    uint32_t n;
    uint32_t n_parts;
    uint64_t *part_keys;
    uint32_t *out_index;
    StepCtl *ctl;        // step_end: advance the position
    uint32_t *tokens;    // step_end: token sequence
    uint32_t *rope_pos;  // step_end: pos field of the state's RoPE config (may be null)
    uint32_t *attn_pos;  // step_end: pos field of the state's attention params (may be null)
    float div;           // part keys of v / div when non-zero
};

// Token sampling: temperature, softmax, multinomial or top-p selection in
// up to four kernels (exp sums, probabilities and the grouping of the top-p
// candidates over many workgroups, the selection in one), optionally ending
// a decode step as ArgmaxArgs does.
constexpr uint32_t SAMPLE_MAX_N = 262144;     // vocabulary limit (1024 chunks of 256)
constexpr uint32_t SAMPLE_GROUP_ELEMS = 2048; // elements per workgroup of the exp / prob kernels
// Scratch the three kernels share (byte offsets from SampleArgs::work).
constexpr uint32_t SMPW_PART = 0;                       // float[128]: per-workgroup sums of exp(y - max)
constexpr uint32_t SMPW_MASS = 512;                     // uint64[2048]: candidate mass per level-0 bucket
constexpr uint32_t SMPW_CNT = SMPW_MASS + 2048 * 8;     // uint32[2048]: candidates per level-0 bucket
constexpr uint32_t SMPW_CHUNK = SMPW_CNT + 2048 * 4;    // uint64[1024]: mass per chunk of 256 (multinomial)
constexpr uint32_t SMPW_N0 = SMPW_CHUNK + 1024 * 8;     // uint32: candidates
constexpr uint32_t SMPW_KMIN = SMPW_N0 + 8;             // uint64: smallest candidate key
constexpr uint32_t SMPW_CUR = SMPW_KMIN + 8;            // uint32[2048]: fill cursor per bucket
constexpr uint32_t SMPW_KEYS = SMPW_CUR + 2048 * 4;     // uint64[SAMPLE_MAX_N]: candidate keys grouped by bucket
constexpr uint32_t SAMPLE_WORK_BYTES = SMPW_KEYS + SAMPLE_MAX_N * 8;
struct SampleArgs {
    const float *logits;        // n logits
    float *probs;               // n probabilities out (may alias logits)
    uint32_t n;
    float temperature;          // != 0
    float topp;                 // top-p mass; <= 0 or >= 1 samples from the whole distribution
    uint32_t n_parts;           // argmax keys giving the maximum (> 0)
    const uint64_t *part_keys;
    int32_t keys_of_y;          // 1: keys of logits / T; 0: keys of the logits (T > 0)
    const float *coin;          // device coin in [0, 1); null: drawn from (seed, position)
    uint64_t seed;
    uint8_t *work;              // SAMPLE_WORK_BYTES of scratch
    uint32_t *out_index;        // may be null
    StepCtl *ctl;               // step end (may be null), as ArgmaxArgs
    uint32_t *tokens;
    uint32_t *rope_pos;
    uint32_t *attn_pos;
};

struct EmbedArgs {
    float *x;
    const uint8_t *table;
    const uint32_t *tokens;
    const StepCtl *ctl;
    uint8_t *xq_out;          // x * gamma quantized for the first GEMV (may be null)
    float *ss_out;            // per-workgroup partial sums of x^2
    const float *gamma;       // RMSNorm weight of the first GEMV
    uint32_t hidden;
    uint32_t row_bytes;
    int32_t fmt;
    uint32_t pad;
};

// Quantizes an activation vector (XQ layout), optionally times gamma, with
// per-workgroup partial sums of x^2.
struct QActArgs {
    const float *x;
    const float *gamma;
    uint8_t *xq_out;
    float *ss_out;
    uint32_t n;
    uint32_t pad;
};

struct KvStoreArgs {
    const float *k;
    const float *v;
    void *k_cache;
    void *v_cache;
    const StepCtl *ctl;
    uint32_t kv_dim;
    int32_t kv_f16;
};

// Prefill GEMM: Y[m][n] (+)= sum_k X[m][k] * deq(W)[n][k]; X f16 (as raw
// halves), W rows of GGUF blocks, Y f32 (or f16 h for the SwiGLU form).
// The n rows are those of up to three matrices of one type stacked one after
// another: n < n1 from w0, n1 <= n < n2 from w1, the rest from w2.  SwiGLU:
// w0 gate and w1 up, n1 = their row count, N = 2 n1.
struct PfGemmArgs {
    const void *x;       // f16 [M][ldx], rows 16-byte aligned
    const uint8_t *w0, *w1, *w2; // rows of K/QK GGUF blocks
    void *y;             // f32 [M][ldy] (f16 for SwiGLU)
    uint32_t M, N, K, ldx, ldy, row_bytes;
    uint32_t n1, n2;     // stacked matrix boundaries
    uint32_t tiles_n, tiles_m; // tile grid (pf_gemm: 256 x 256 tiles)
    // warp-specialized form: tiles at or past tiles_full run as two 256 x
    // 128 halves, one workgroup each (tiles_full = tiles_n * tiles_m: none)
    uint32_t tiles_full;
    // warp-specialized store product of stacked Q | K | V with rope != 0:
    // the epilogue adds the biases, rotates q and k (pairs (2i, 2i+1)) with
    // the pass's (cos, sin) table and stores q to Y and k, v to the cache
    // rows of positions p0 + m (the work of pf_rope_kv_k)
    const float *rope_cs;          // [M][head_size / 2][2]
    const float *q_bias, *k_bias, *v_bias;
    void *k_cache, *v_cache;
    uint32_t head_size, p0, rope;
    int32_t kv_f16;
};

// Prefill pointwise and attention kernels (one chunk of M prompt tokens at
// positions p0 .. p0+M-1).
struct PfArgs {
    void *x;             // f32 [M][hidden] residual stream
    void *xh;            // f16 [M][ldh] GEMM input / attention output / h
    uint32_t ldh, hidden;
    const float *gamma;  // RMSNorm weight
    float eps;
    uint32_t M, p0;
    const uint32_t *tokens; // token sequence (embedding)
    const uint8_t *table;   // token_embd rows
    uint32_t row_bytes;
    int32_t fmt;
    void *qkv;           // f32 [M][ld_qkv]: q | k | v
    uint32_t ld_qkv, q_dim, kv_dim, head_size;
    const float *rope_tab;
    void *k_cache, *v_cache; // this layer's cache base
    int32_t kv_f16;
    uint32_t ffn;
    void *gu;            // f32 [M][2*ffn]: gate | up (layers whose gate and up types differ)
    void *h;             // f16 [M][ffn]: silu(gate) * up, the down product's input
    const float *q_bias, *k_bias, *v_bias; // QKV biases (may be null)
    int32_t neox;        // RoPE pairs (j, j + hs/2) instead of (2j, 2j+1)
    uint32_t kv_mul;     // attention: query heads per KV head
    float *rope_cs;      // [M][head_size / 2][2]: cos, sin of (p0 + m) * theta_j
};

} // namespace ifr

// inferi_hip host library: the C ABI of include/inferi_hip.h over the HIP
// runtime.  Kernels live in a gfx950 code object loaded with hipModuleLoad
// and are launched with hipModuleLaunchKernel on the context's stream.
//
// The model layer mirrors the reference's Llama2 (crates/inferi/src/models/
// llama2/transformer.rs): Llama2Weights is a table of caller-owned device
// tensors, Llama2State owns the activations and the KV cache, and one decode
// step is Llama2::launch (:409-481) plus the embedding copy and greedy
// sampling of ChatLlama2::forward_logits (crates/inferi-chat/src/
// chat_llama2.rs:191-255), with the position, the token sequence and the
// argmax all on the device.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/inferi_hip.h"
#include "kargs.h"
#include "noalloc.h"

using namespace ifr;

// Message of the last failed call made without a context on this thread
// (ifr_create, the GGUF reader and writer of gguf.cpp).
static thread_local std::string g_create_error;
std::string &ifr_free_error() { return g_create_error; }

namespace {

constexpr uint32_t GEMV_MAX_LDS = 65536 - 256;

// Bytes of a quantized activation vector of n values (XQ layout,
// device/gemv.h): three int8 digit planes plus a scale and a sum per 16 values.
uint64_t xq_bytes(uint64_t n) { return 3 * n + n / 2; }

// Dynamic LDS of a GEMV launch: x as f32, or its XQ copy.
constexpr uint32_t ATTN_SPLITS_MAX = 256; // attention splits per KV head (at most)
constexpr uint32_t ATTN_GT_MAX = 8;       // device/attention.h: query heads per workgroup
constexpr uint32_t MAX_PARTS = 1024;      // argmax partial keys per launch
constexpr uint32_t PF_GEMM_TILE = 128;    // device/prefill.h: PF_BM = PF_BN
constexpr uint32_t PF_BIG_TILE = 256;     // device/pf_gemm.h: PG_BM = PG_BN
constexpr uint32_t PF_BIG_THREADS = 512;  // device/pf_gemm.h: PG_THREADS
constexpr uint32_t PF_WS_THREADS = 768;   // device/pf_gemm.h: PGW_THREADS
constexpr uint32_t PF_WS_ROUND = 256;     // workgroups of one round (one per CU on MI355X)
constexpr uint32_t PF_CHUNK = 4096;       // prompt tokens per prefill pass (at most)

int qk_of(int32_t dt) {
    switch (dt) {
    case IFR_F32: case IFR_F16: return 1;
    case IFR_Q4_0: case IFR_Q4_1: case IFR_Q5_0: case IFR_Q5_1: case IFR_Q8_0: return 32;
    case IFR_Q4_K: case IFR_Q5_K: case IFR_Q6_K: case IFR_Q8_K: return 256;
    default: return 0;
    }
}
int bytes_of(int32_t dt) {
    switch (dt) {
    case IFR_F32: return 4;
    case IFR_F16: return 2;
    case IFR_Q4_0: return 18;
    case IFR_Q4_1: return 20;
    case IFR_Q5_0: return 22;
    case IFR_Q5_1: return 24;
    case IFR_Q8_0: return 34;
    case IFR_Q4_K: return 144;
    case IFR_Q5_K: return 176;
    case IFR_Q6_K: return 210;
    case IFR_Q8_K: return 292;
    default: return 0;
    }
}
const char *gemv_fmt_name(int32_t dt) {
    switch (dt) {
    case IFR_Q4_0: return "q4_0";
    case IFR_Q4_1: return "q4_1";
    case IFR_Q5_0: return "q5_0";
    case IFR_Q5_1: return "q5_1";
    case IFR_Q8_0: return "q8_0";
    case IFR_Q4_K: return "q4_k";
    case IFR_Q5_K: return "q5_k";
    case IFR_Q6_K: return "q6_k";
    case IFR_Q8_K: return "q8_k";
    case IFR_F16: return "f16";
    case IFR_F32: return "f32";
    default: return nullptr;
    }
}
// The GEMV kernels' block: the GGUF block, or a virtual block of 32
// elements for the unquantized types (device/gemv.h QFmt).
int gemv_qk(int32_t dt) { return qk_of(dt) == 1 ? 32 : qk_of(dt); }
uint32_t gemv_block_bytes(int32_t dt) { return (uint32_t)(qk_of(dt) == 1 ? 32 * bytes_of(dt) : bytes_of(dt)); }
// Row alignment the GEMV and prefill tile loads need: 16 bytes for the
// formats read with 16-byte loads, 4 (or the field alignment) otherwise.
uintptr_t gemv_align(int32_t dt) {
    return (dt == IFR_Q4_K || dt == IFR_Q5_K || dt == IFR_F16 || dt == IFR_F32) ? 16 : 4;
}
// Blocks one 64-lane step of the integer GEMV covers: 32 for the 32-element
// formats (2 lanes per block), 16 for the 256-element ones (4 lanes).
uint32_t int_blocks_per_step(int32_t dt) { return gemv_qk(dt) == 32 ? 32u : 16u; }

} // namespace

struct ifr_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    std::map<std::string, hipFunction_t> fns;
    std::string err;
    char dev_name[256] = {0};
    int n_cu = 0;
    hipEvent_t events[16] = {};
    // scratch for the op-level attention and argmax
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // quantized activation of the op-level GEMV
    void *xq_scratch = nullptr;
    size_t xq_scratch_bytes = 0;
    // tuning: cap on GEMV workgroups (0 = one per row tile)
    uint32_t gemv_max_grid = 0;
    uint32_t gemv_waves = 0; // integer-path waves per workgroup (0: by shape)
    // GEMV arithmetic: 0 = x as 16-bit fixed point with int8 dot products,
    // 1 = exact fp32 x and FMAs
    int gemv_exact = 0;
    // one-item GEMV forms in use: bit 0 resid with one K step (O), bit 1
    // resid with K-slices (down), bit 2 gateup, bit 3 gateup as 16 waves of
    // two rows (else 8 waves of four), bit 4 the output head, bit 5 gateup
    // with h in f32 and the down GEMV quantizing it, bit 6 the Q6_K head in
    // 256-VGPR workgroups, bit 7 gateup with four rows per wave, bit 8 plain
    // and qkv with four rows per wave (default: bits 0, 5, 6 and 7)
    int gemv_grp = 225;
    // prompt tokens per prefill pass (0: PF_CHUNK), read at a state's first prefill
    uint32_t pf_chunk = 0;
    // this device's fixed scratch of ifr_matmul_quant_noalloc (noalloc.hip)
    void *noalloc_scratch = nullptr;
    // prefill GEMM tiles: 0 = by shape (256 x 256 tiles where the product
    // has enough of them, else 128 x 128), 128 or 256 to force one (option
    // pf_tile)
    uint32_t pf_tile = 0;
    // Q4_K products on 256 x 256 tiles in the warp-specialized form (option
    // pf_ws, default on; 0 = the eight-wave form; device/pf_gemm.h
    // pf_gemm_ws_body)
    int pf_ws = 1;
    // the Q/K/V product's epilogue applies RoPE and stores k, v to the cache
    // (warp-specialized form, pairs (2i, 2i + 1)) instead of pf_rope_kv_k
    // (option pf_rope_fuse, default on)
    int pf_rope_fuse = 1;
    // bumped by every option change: a captured decode step is captured
    // again when it differs
    uint64_t opt_gen = 0;

    ifr_status fail(ifr_status st, const char *fmt, ...) {
        char buf[1024];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        err = buf;
        return st;
    }
    ifr_status hip(hipError_t e, const char *what) {
        if (e == hipSuccess) return IFR_OK;
        return fail(e == hipErrorOutOfMemory ? IFR_ENOMEM : IFR_EHIP, "%s: %s", what, hipGetErrorString(e));
    }
    hipFunction_t fn(const std::string &name) {
        auto it = fns.find(name);
        if (it != fns.end()) return it->second;
        hipFunction_t f = nullptr;
        if (hipModuleGetFunction(&f, module, name.c_str()) != hipSuccess) f = nullptr;
        fns[name] = f;
        return f;
    }
    template <class A>
    ifr_status launch(const std::string &name, dim3 grid, dim3 block, uint32_t shmem, const A &args) {
        hipFunction_t f = fn(name);
        if (!f) return fail(IFR_EUNSUPPORTED, "kernel %s not in the code object", name.c_str());
        // every kernel takes one struct argument: kernelParams[0] points at it
        A copy = args;
        void *params[] = {&copy};
        return hip(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem, stream, params,
                                         nullptr),
                   name.c_str());
    }
    ifr_status ensure_xq_scratch(size_t bytes) {
        if (bytes <= xq_scratch_bytes) return IFR_OK;
        if (xq_scratch) {
            hipStreamSynchronize(stream);
            hipFree(xq_scratch);
            xq_scratch = nullptr;
            xq_scratch_bytes = 0;
        }
        ifr_status st = hip(hipMalloc(&xq_scratch, bytes), "hipMalloc(xq scratch)");
        if (st) return st;
        xq_scratch_bytes = bytes;
        return IFR_OK;
    }
    ifr_status ensure_scratch(size_t bytes) {
        if (bytes <= scratch_bytes) return IFR_OK;
        if (scratch) {
            hipStreamSynchronize(stream);
            hipFree(scratch);
            scratch = nullptr;
            scratch_bytes = 0;
        }
        ifr_status st = hip(hipMalloc(&scratch, bytes), "hipMalloc(scratch)");
        if (st) return st;
        scratch_bytes = bytes;
        return IFR_OK;
    }
};

// ------------------------------------------------------------------ GEMV --

struct GemvPlan {
    const char *fmt;
    uint32_t nb, row_bytes;
    uint32_t bpi; // blocks per integer-path step (int_blocks_per_step)
};

static ifr_status check_gemv(ifr_ctx *c, int32_t dtype, uint32_t cols, const void *w, GemvPlan &p) {
    p.fmt = gemv_fmt_name(dtype);
    if (!p.fmt) return c->fail(IFR_EUNSUPPORTED, "matmul_quant: dtype %d has no GEMV kernel", dtype);
    const int qk = gemv_qk(dtype);
    if (cols == 0 || cols % (uint32_t)qk) return c->fail(IFR_EINVAL, "matmul_quant: cols %u not a multiple of %d", cols, qk);
    if ((c->gemv_exact ? (uint64_t)cols * 4 : xq_bytes(cols)) > GEMV_MAX_LDS)
        return c->fail(IFR_EUNSUPPORTED, "matmul_quant: cols %u too large for one workgroup's LDS", cols);
    const uintptr_t need = gemv_align(dtype);
    if ((uintptr_t)w % need) return c->fail(IFR_EINVAL, "matmul_quant: weights not %u-byte aligned", (unsigned)need);
    p.nb = cols / (uint32_t)qk;
    p.row_bytes = p.nb * gemv_block_bytes(dtype);
    p.bpi = int_blocks_per_step(dtype);
    return IFR_OK;
}

// Exact-path launch geometry per mode (kargs.h gemv_geom): rows per
// workgroup tile and threads per workgroup.
static GemvGeomT geom_of(const char *mode) {
    return gemv_geom(!strcmp(mode, "gateup") ? GEMV_GATEUP : !strcmp(mode, "resid") ? GEMV_RESID : GEMV_PLAIN);
}

// Integer-path geometry (device/gemv.h, gemv_int_body): K-slices KS by the
// number of 64-lane steps a row takes, as many row waves as the output
// group allows (16 virtual rows, 32 for gateup, two per wave) up to 16
// waves, and one resident workgroup set (16 waves per CU) looping over the
// groups unless a cap is given.
struct IntGeom {
    uint32_t ks, waves, grid;
};
static IntGeom int_geom(const ifr_ctx *c, uint32_t bpi, const char *mode, const GemvArgs &a, uint32_t cap) {
    const uint32_t steps = (a.nb + bpi - 1) / bpi;
    IntGeom g;
    g.ks = steps <= 1 ? 1 : steps <= 2 ? 2 : 4;
    const uint32_t gr = !strcmp(mode, "gateup") ? 32 : 16;
    // gateup: 8 waves (two sub-tiles per group) and three workgroups per CU
    // measured fastest; the others: as many row waves as a group allows
    const bool gateup = !strcmp(mode, "gateup");
    // waves that finish their own rows (one K-slice, no quantized output):
    // four waves of two rows per workgroup, one workgroup per 8 rows, every
    // workgroup resident at once (measured fastest); the groups are then
    // the workgroups' 8 rows
    const bool local = g.ks == 1 && (!strcmp(mode, "plain") || !strcmp(mode, "qkv") || !strcmp(mode, "head"));
    uint32_t rw = gateup ? 8 / g.ks : local ? 4 : std::min(GEMV_INT_MAX_WAVES / g.ks, gr / 2);
    if (c->gemv_waves) rw = std::max(1u, std::min(std::min(GEMV_INT_MAX_WAVES / g.ks, gr / 2), c->gemv_waves / g.ks));
    g.waves = g.ks * rw;
    const uint32_t gr_eff = local ? rw * 2 : gr;
    const uint32_t ngroups = (a.total_rows + gr_eff - 1) / gr_eff;
    uint32_t grid = gateup ? c->n_cu * 3 : local ? ngroups : c->n_cu * (GEMV_INT_MAX_WAVES / g.waves);
    if (c->gemv_max_grid) grid = c->gemv_max_grid;
    if (cap) grid = std::min(grid, cap);
    g.grid = std::max(std::min(grid, ngroups), 1u);
    return g;
}

// xf (plain mode only): a.x is f32 and the kernel quantizes it into its LDS
// itself (the `_xf` forms), instead of reading a.xq.
static ifr_status launch_gemv(ifr_ctx *c, const GemvPlan &p, const char *mode, GemvArgs &a, uint32_t cap = 0,
                              uint32_t *grid_out = nullptr, bool xf = false) {
    const bool exact = c->gemv_exact != 0;
    std::string name = std::string("gemv_") + p.fmt + "_" + mode + (exact ? "_f32" : "");
    if (exact) {
        const GemvGeomT ge = geom_of(mode);
        const uint32_t tr = (uint32_t)(ge.R * ge.W);
        uint32_t g = (a.total_rows + tr - 1) / tr;
        if (c->gemv_max_grid) g = std::min(g, c->gemv_max_grid);
        if (cap) g = std::min(g, cap);
        g = std::max(g, 1u);
        if (grid_out) *grid_out = g;
        return c->launch(name, dim3(g), dim3((uint32_t)ge.W * 64u), a.cols * 4, a);
    }
    if ((!xf && !a.xq) || (a.total_rows && a.cols % 16))
        return c->fail(IFR_EINVAL, "gemv: integer path needs a quantized input");
    // plain and qkv rows of one 64-lane step: the one-item kernel, every
    // workgroup launched at once
    const bool one_mode = !strcmp(mode, "plain") || !strcmp(mode, "qkv");
    if (one_mode && a.nb <= p.bpi && !c->gemv_waves && !c->gemv_max_grid && a.total_rows) {
        // four rows per wave where the code object has that form (bit 8;
        // slower for the QKV launch's 6144 rows, whose 384 workgroups of
        // four-row waves do not fill the chip)
        const bool four = !xf && (c->gemv_grp & 256) && c->fn(name + "_one4");
        const uint32_t rows_per = GEMV_ONE_WAVES * (four ? 4 : 2), g = (a.total_rows + rows_per - 1) / rows_per;
        a.ks = 1;
        a.nwaves = GEMV_ONE_WAVES;
        if (grid_out) *grid_out = g;
        return c->launch(name + (four ? "_one4" : xf ? "_one_xf" : "_one"), dim3(g), dim3(GEMV_ONE_WAVES * 64),
                         (uint32_t)xq_bytes(a.cols), a);
    }
    // resid and gateup: one output group per workgroup, one item per wave,
    // where the code object has the form for this format and K
    const bool resid = !strcmp(mode, "resid"), gateup = !strcmp(mode, "gateup");
    if ((resid || gateup) && !c->gemv_waves && !c->gemv_max_grid && a.total_rows) {
        const uint32_t steps = (a.nb + p.bpi - 1) / p.bpi;
        char kn[96] = {0};
        const bool alt = c->gemv_grp & 8;
        if (resid && steps == 1 && (c->gemv_grp & 1)) snprintf(kn, sizeof kn, "gemv_%s_resid_r2w8k1", p.fmt);
        else if (resid && steps > 1 && steps <= 4 && (c->gemv_grp & 2)) snprintf(kn, sizeof kn, "gemv_%s_resid_r4w4k4", p.fmt);
        else if (gateup && steps == 1 && (c->gemv_grp & 4))
            snprintf(kn, sizeof kn, alt ? "gemv_%s_gateup_r2w16k1" : "gemv_%s_gateup_r4w8k1", p.fmt);
        hipFunction_t f = kn[0] ? c->fn(kn) : nullptr;
        if (f) {
            const uint32_t gr = gateup ? 32 : 16, g = (a.total_rows + gr - 1) / gr;
            const uint32_t waves = resid && steps == 1 ? 8 : resid ? 16 : alt ? 16 : 8;
            a.ks = steps;
            a.nwaves = waves;
            if (grid_out) *grid_out = g;
            return c->launch(kn, dim3(g), dim3(waves * 64), (uint32_t)xq_bytes(a.cols), a);
        }
    }
    const IntGeom g = int_geom(c, p.bpi, mode, a, cap);
    a.ks = g.ks;
    a.nwaves = g.waves;
    if (grid_out) *grid_out = g.grid;
    // the head's form with up to 256 VGPRs, where the code object has it:
    // two workgroups per CU, each looping over its share of the row groups
    // (measured fastest: 3 or 4 per CU and the 128-VGPR form are slower)
    if (!strcmp(mode, "head") && (c->gemv_grp & 64) && g.waves <= 4 && !c->gemv_max_grid && c->fn(name + "_w2")) {
        const uint32_t gg = std::min(g.grid, (uint32_t)c->n_cu * 2);
        if (grid_out) *grid_out = gg;
        return c->launch(name + "_w2", dim3(gg), dim3(g.waves * 64), (uint32_t)xq_bytes(a.cols), a);
    }
    return c->launch(name + (xf ? "_xf" : ""), dim3(g.grid), dim3(g.waves * 64), (uint32_t)xq_bytes(a.cols), a);
}

// x (times gamma) -> XQ with per-256 partial sums of x^2.
static ifr_status launch_quant_act(ifr_ctx *c, const float *x, const float *gamma, uint32_t n, uint8_t *xq,
                                   float *ss_out, uint32_t *n_parts = nullptr) {
    QActArgs q{x, gamma, xq, ss_out, n, 0};
    const uint32_t g = (n + 255) / 256;
    if (n_parts) *n_parts = g;
    return c->launch("quant_act_k", dim3(g), dim3(256), 0, q);
}

// out = W v for a plain f32 v: quantizes v into `xq` first on the integer path.
static ifr_status gemv_plain(ifr_ctx *c, float *out, const void *w, int32_t dtype, uint32_t rows, uint32_t cols,
                             const float *v, uint8_t *xq, bool allow_xf = true) {
    GemvPlan p;
    ifr_status st = check_gemv(c, dtype, cols, w, p);
    if (st) return st;
    GemvArgs a{};
    a.w0 = (const uint8_t *)w;
    a.total_rows = rows;
    a.cols = cols;
    a.nb = p.nb;
    a.row_bytes = p.row_bytes;
    a.x = v;
    a.y = out;
    if (!c->gemv_exact) {
        // the GEMV kernel quantizes the f32 x into its LDS itself (the same
        // bytes as the quantize launch): one launch instead of two
        const std::string one = std::string("gemv_") + p.fmt + "_plain_one_xf", loop = std::string("gemv_") + p.fmt + "_plain_xf";
        if (allow_xf && cols % 16 == 0 && c->fn(one) && c->fn(loop)) return launch_gemv(c, p, "plain", a, 0, nullptr, true);
        if (!xq) {
            if ((st = c->ensure_xq_scratch(xq_bytes(cols)))) return st;
            xq = (uint8_t *)c->xq_scratch;
        }
        if ((st = launch_quant_act(c, v, nullptr, cols, xq, nullptr))) return st;
        a.xq = xq;
    }
    return launch_gemv(c, p, "plain", a);
}

// ------------------------------------------------------------- attention --

// Head sizes run on kernels for 64 or 128 dims (device/attention.h pads the
// head to them).
static uint32_t attn_hsp(uint32_t head_size) { return head_size <= 64 ? 64u : 128u; }
// Splits of the attention over the sequence for T positions: one batch of
// the split kernel each (8192/HSP positions, device/attention.h
// attn_quantum), at most ATTN_SPLITS_MAX; longer chunks beyond that.
static uint32_t attn_splits_for(uint32_t T, uint32_t head_size) {
    const uint32_t q = 8192u / attn_hsp(head_size);
    return std::max(1u, std::min(ATTN_SPLITS_MAX, (uint32_t)(((uint64_t)T + q - 1) / q)));
}
// A KV head's query heads go to n_sub workgroups of gt heads each (gt <= 8,
// the last workgroup holding the rest).
static void attn_groups(uint32_t kv_mul, uint32_t &n_sub, uint32_t &gt) {
    n_sub = (kv_mul + ATTN_GT_MAX - 1) / ATTN_GT_MAX;
    gt = (kv_mul + n_sub - 1) / n_sub;
}

// Positions come in buckets of ATTN_BUCKET: steps at positions p of bucket
// b = p / ATTN_BUCKET assume pos + 1 <= (b + 1) * ATTN_BUCKET (capped at
// max_pos), so the attention splits cover the positions in use, not the
// whole cache.
constexpr uint32_t ATTN_BUCKET = 256;
static uint32_t attn_spec_for(uint32_t pos, uint32_t max_pos) {
    return (uint32_t)std::min<uint64_t>(max_pos, ((uint64_t)pos / ATTN_BUCKET + 1) * ATTN_BUCKET);
}

// Split pass over the KV sequence, then the merge of the partials.  `a`
// carries head_size, kv_mul, n_splits and n_out; n_sub is set here.
static ifr_status launch_attn(ifr_ctx *c, int32_t kv_dtype, AttnArgs &a, uint32_t n_kv_heads) {
    uint32_t n_sub, gt;
    attn_groups(a.kv_mul, n_sub, gt);
    a.n_sub = n_sub;
    char name[64];
    snprintf(name, sizeof name, "attn_%s_h%u_g%u", kv_dtype == IFR_F16 ? "f16" : "f32", attn_hsp(a.head_size), gt);
    ifr_status st = c->launch(name, dim3(n_kv_heads * n_sub, a.n_splits), dim3(256), 0, a);
    if (st) return st;
    return c->launch("attn_merge", dim3((a.n_out + 15) / 16), dim3(64), 0, a);
}

// ----------------------------------------------------------------- model --

struct Tens {
    int32_t dtype = -1;
    const uint8_t *data = nullptr;
    uint32_t rows = 0, cols = 0;
};

struct LayerW {
    Tens attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down;
    Tens q_bias, k_bias, v_bias; // Qwen2 (transformer.rs:434-442); data null when absent
};

struct ifr_llama2_weights {
    ifr_ctx *ctx;
    ifr_llama2_config cfg;
    // identity of the tensor table for captured decode graphs: a process-wide
    // id (never reused) and a generation every ifr_llama2_weights_set bumps
    uint64_t id = 0, gen = 0;
    Tens token_embd, output_norm, output;
    std::vector<LayerW> layers;
    std::vector<void *> owned; // device copies made by ifr_llama2_weights_from_gguf
};

struct ifr_llama2_state {
    ifr_ctx *ctx;
    ifr_llama2_config cfg;
    uint32_t kv_dim, head_size, kv_mul, n_splits;
    // the device position as the host knows it (every step advances it by
    // one, up to max_pos - 1), and the bound on pos + 1 the steps being
    // enqueued assume (the attention splits are sized for it)
    uint32_t host_pos = 0, step_spec = 0;
    std::vector<void *> allocs;
    float *x, *xb, *xb2, *q, *ktmp, *vtmp, *hb, *hb2, *att, *logits, *probs;
    uint8_t *smp_work;
    uint32_t *tokens;
    StepCtl *ctl;
    ifr_rms_norm_config *rms_cfg;
    ifr_rope_config *rope_cfg;
    ifr_attn_params *attn_params;
    uint64_t *part_keys;
    uint32_t part_keys_cap = 0; // entries of part_keys
    float *part_o, *part_ml;
    float *rope_tab;
    // quantized activations passed between the fused kernels, and the
    // partial sums of x^2 the RMSNorm consumers reduce:
    //   xq_a: x * attn_norm (or output_norm), input of QKV / the head
    //   xq_f: x * ffn_norm, input of gate/up;  xq_att: attention output;
    //   xq_h: silu(gate) * up;  xq_u: scratch of the one-op-per-kernel path
    uint8_t *xq_a, *xq_f, *xq_att, *xq_h, *xq_u;
    float *ss_a, *ss_f;
    uint8_t *kcache, *vcache;
    size_t layer_kv_bytes;
    // prefill scratch (allocated at the first prefill): a chunk of pf_chunk tokens
    uint32_t pf_chunk = 0, pf_ldh = 0;
    float *pf_x = nullptr, *pf_qkv = nullptr, *pf_gu = nullptr;
    float *pf_rope_cs = nullptr; // [pf_chunk][head_size / 2][2]: the pass's RoPE (cos, sin)
    uint16_t *pf_xh = nullptr, *pf_h = nullptr;
    // sampler of the step end: temperature 0 takes the argmax
    float temperature = 0.0f, topp = 0.0f;
    uint64_t seed = 0;
    uint32_t sampler_gen = 0;
    // captured decode step
    hipGraphExec_t graph = nullptr;
    uint64_t graph_opt = ~0ull; // the context's option generation the graph was captured with
    uint32_t graph_sampler = 0;
    uint32_t graph_spec = 0; // step_spec the graph was captured with
    // graphs replaced while their launches may still run: destroyed once the
    // event recorded after their last launch has completed
    std::vector<std::pair<hipGraphExec_t, hipEvent_t>> retired;
    uint64_t graph_wid = 0, graph_wgen = 0; // weights id and generation the graph was captured with
    int graph_fused = -1;
};

static ifr_status validate_cfg(ifr_ctx *c, const ifr_llama2_config *cfg) {
    if (!cfg) return c->fail(IFR_EINVAL, "null config");
    if (!cfg->n_layers || !cfg->hidden || !cfg->n_heads || !cfg->n_kv_heads || !cfg->vocab || !cfg->max_pos || !cfg->ffn)
        return c->fail(IFR_EINVAL, "config has a zero dimension");
    if (cfg->hidden % cfg->n_heads || cfg->n_heads % cfg->n_kv_heads)
        return c->fail(IFR_EINVAL, "hidden %% n_heads or n_heads %% n_kv_heads != 0");
    const uint32_t hs = cfg->hidden / cfg->n_heads, kv_mul = cfg->n_heads / cfg->n_kv_heads;
    if (hs % 8 || hs > 128) return c->fail(IFR_EUNSUPPORTED, "head_size %u (a multiple of 8, at most 128)", hs);
    if (kv_mul > 64) return c->fail(IFR_EUNSUPPORTED, "kv_mul %u (at most 64 query heads per KV head)", kv_mul);
    if (cfg->hidden % 32 || cfg->ffn % 32) return c->fail(IFR_EUNSUPPORTED, "hidden and ffn must be multiples of 32");
    if (cfg->kv_dtype != IFR_F16 && cfg->kv_dtype != IFR_F32) return c->fail(IFR_EINVAL, "kv_dtype must be F16 or F32");
    if (cfg->rope_variant != IFR_ROPE_ORIGINAL && cfg->rope_variant != IFR_ROPE_NEOX)
        return c->fail(IFR_EINVAL, "bad rope_variant");
    if (cfg->max_pos > (1u << 30)) return c->fail(IFR_EUNSUPPORTED, "max_pos %u too large", cfg->max_pos);
    return IFR_OK;
}

// Enqueues one decode step.  Fused: per layer QKV+RoPE+KV store, attention
// (split + merge), O + residual, gate/up + SiLU, down + residual; activations
// travel between them quantized (integer path) and in f32 (exact path and the
// residual stream).  Unfused: one kernel per reference op (transformer.rs:418-469).
// Sampler::sample with T != 0: exp sums, probabilities and (top-p) the
// candidates grouped by bucket over many workgroups, the choice in one.  The
// maximum of y = logits / T comes from argmax keys: `parts` keys of the
// logits when keys_of_y is 0 (T > 0 only), of y when 1.
static ifr_status launch_sample(ifr_ctx *c, SampleArgs a) {
    const uint32_t groups = (a.n + SAMPLE_GROUP_ELEMS - 1) / SAMPLE_GROUP_ELEMS;
    ifr_status st;
    if ((st = c->launch("sample_exp_k", dim3(groups), dim3(256), 0, a))) return st;
    if ((st = c->launch("sample_prob_k", dim3(groups), dim3(256), 0, a))) return st;
    const bool nucleus = !(a.topp <= 0.0f || a.topp >= 1.0f); // sampler.rs:44
    if (nucleus && (st = c->launch("sample_group_k", dim3(groups), dim3(256), 0, a))) return st;
    return c->launch("sample_select_k", dim3(1), dim3(1024), 0, a);
}

// Argmax keys of logits / T into keys (the maximum the sampler subtracts).
static ifr_status launch_keys_of_y(ifr_ctx *c, const float *logits, uint32_t n, float T, uint64_t *keys,
                                   uint32_t &parts) {
    ArgmaxArgs k{};
    k.v = logits;
    k.n = n;
    k.part_keys = keys;
    k.div = T;
    parts = std::min((n + 255) / 256, MAX_PARTS);
    return c->launch("argmax_part_k", dim3(parts), dim3(256), 0, k);
}

static ifr_status enqueue_head(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, int fused, uint32_t n_ss_a);

// Decode stages of one layer, in order (a mask selects which run: the step
// runs them all; ifr_llama2_time_stage repeats one).  n_ss_a: partial sums of
// x^2 in ss_a, read by the fused QKV and set by the fused down GEMV.
enum : uint32_t { ST_QKV = 1, ST_ATTN = 2, ST_O = 4, ST_GATEUP = 8, ST_DOWN = 16, ST_LAYER = 31 };

static ifr_status enqueue_layer(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, int fused, uint32_t l,
                                uint32_t stages, uint32_t &n_ss_a) {
    const ifr_llama2_config &cfg = s->cfg;
    const uint32_t hidden = cfg.hidden, kv_dim = s->kv_dim, ffn = cfg.ffn, L = cfg.n_layers;
    const uint32_t n_ss_res = hidden / 16; // partial sums written by a RESID GEMV (one per 16-row tile)
    ifr_status st;
    const LayerW &Lw = w->layers[l];
    uint8_t *kc = s->kcache + (size_t)l * s->layer_kv_bytes;
    uint8_t *vc = s->vcache + (size_t)l * s->layer_kv_bytes;
    const bool fuse_qkv = fused != 0;
    const bool fuse_ffn = fused && Lw.ffn_gate.dtype == Lw.ffn_up.dtype;
    // gate/up as one item per wave with h in f32, quantized by the down
    // GEMV itself (Q4_K, rows of one K step; option gemv_grp bit 5)
    const bool h32 = fuse_ffn && (c->gemv_grp & 32) && !c->gemv_exact && !c->gemv_waves && !c->gemv_max_grid &&
                     Lw.ffn_gate.dtype == IFR_Q4_K && Lw.ffn_down.dtype == IFR_Q4_K && hidden <= 4096 &&
                     hidden % 256 == 0 && c->fn("gemv_q4_k_gateup_one") && c->fn("gemv_q4_k_resid_xf");
    const float *next_norm = (const float *)(l + 1 < L ? w->layers[l + 1].attn_norm.data : w->output_norm.data);
    GemvPlan p;

    if (stages & ST_QKV) {
        // ---- attention block
        if (fuse_qkv) {
            // one launch per run of consecutive matrices of one GGUF type
            // (q, k, v in that order; a Q4_K_M file keeps v in Q6_K on some
            // layers): the launch's rows are those matrices' rows, the others
            // counted as zero rows so the epilogue still tells q, k and v apart
            const Tens *m3[3] = {&Lw.attn_q, &Lw.attn_k, &Lw.attn_v};
            const uint32_t r3[3] = {hidden, kv_dim, kv_dim};
            for (uint32_t g0 = 0; g0 < 3;) {
                uint32_t g1 = g0 + 1;
                while (g1 < 3 && m3[g1]->dtype == m3[g0]->dtype) g1++;
                if ((st = check_gemv(c, m3[g0]->dtype, hidden, m3[g0]->data, p))) return st;
                GemvArgs a{};
                a.w0 = Lw.attn_q.data;
                a.w1 = Lw.attn_k.data;
                a.w2 = Lw.attn_v.data;
                a.rows0 = g0 <= 0 && 0 < g1 ? r3[0] : 0;
                a.rows1 = g0 <= 1 && 1 < g1 ? r3[1] : 0;
                a.rows2 = g0 <= 2 && 2 < g1 ? r3[2] : 0;
                a.total_rows = a.rows0 + a.rows1 + a.rows2;
                a.cols = hidden;
                a.nb = p.nb;
                a.row_bytes = p.row_bytes;
                a.x = s->x;
                a.gamma = (const float *)Lw.attn_norm.data;
                a.xq = s->xq_a;
                a.ss_part = s->ss_a;
                a.n_ss = n_ss_a;
                a.eps = cfg.rms_eps;
                a.rope_tab = s->rope_tab;
                a.y = s->q;
                a.k_cache = kc;
                a.v_cache = vc;
                a.ctl = s->ctl;
                a.kv_dim = kv_dim;
                a.head_size = s->head_size;
                a.kv_f16 = cfg.kv_dtype == IFR_F16;
                a.q_bias = (const float *)Lw.q_bias.data;
                a.k_bias = (const float *)Lw.k_bias.data;
                a.v_bias = (const float *)Lw.v_bias.data;
                a.neox = cfg.rope_variant == IFR_ROPE_NEOX;
                if ((st = launch_gemv(c, p, "qkv", a))) return st;
                g0 = g1;
            }
        } else {
            EltArgs n{};
            n.a = s->xb;
            n.b = s->x;
            n.w = (const float *)Lw.attn_norm.data;
            n.cfg = s->rms_cfg;
            n.n = hidden;
            if ((st = c->launch("rms_norm_k", dim3(1), dim3(1024), 0, n))) return st;
            const Tens *mats[3] = {&Lw.attn_q, &Lw.attn_k, &Lw.attn_v};
            float *outs[3] = {s->q, s->ktmp, s->vtmp};
            for (int m = 0; m < 3; m++)
                if ((st = gemv_plain(c, outs[m], mats[m]->data, mats[m]->dtype, mats[m]->rows, hidden, s->xb, s->xq_u)))
                    return st;
            // Qwen2: q += q_bias, k += k_bias, v += v_bias before RoPE (transformer.rs:434-442)
            const Tens *bias[3] = {&Lw.q_bias, &Lw.k_bias, &Lw.v_bias};
            for (int m = 0; m < 3; m++) {
                if (!bias[m]->data) continue;
                EltArgs e{};
                e.a = outs[m];
                e.b = (const float *)bias[m]->data;
                e.n = mats[m]->rows;
                if ((st = c->launch("add_k", dim3((e.n + 255) / 256), dim3(256), 0, e))) return st;
            }
            EltArgs r{};
            r.a = s->q;
            r.k = s->ktmp;
            r.cfg = s->rope_cfg;
            r.n = hidden;
            r.n2 = kv_dim;
            r.variant = cfg.rope_variant;
            if ((st = c->launch("rope_k", dim3((hidden / 2 + 255) / 256), dim3(256), 0, r))) return st;
            KvStoreArgs kv{};
            kv.k = s->ktmp;
            kv.v = s->vtmp;
            kv.k_cache = kc;
            kv.v_cache = vc;
            kv.ctl = s->ctl;
            kv.kv_dim = kv_dim;
            kv.kv_f16 = cfg.kv_dtype == IFR_F16;
            if ((st = c->launch("kv_store_k", dim3((kv_dim + 255) / 256), dim3(256), 0, kv))) return st;
        }
    }
    if (stages & ST_ATTN) {
        {
            AttnArgs a{};
            a.q = s->q;
            a.k_cache = kc;
            a.v_cache = vc;
            a.out = s->att;
            a.xq_out = fused ? s->xq_att : nullptr;
            a.part_o = s->part_o;
            a.part_ml = s->part_ml;
            a.pos = &s->ctl->pos;
            a.kv_dim = kv_dim;
            a.n_splits = attn_splits_for(s->step_spec, s->head_size);
            a.seq_cap = cfg.max_pos;
            a.spec_rows = s->step_spec;
            a.n_out = hidden;
            a.head_size = s->head_size;
            a.kv_mul = s->kv_mul;
            if ((st = launch_attn(c, cfg.kv_dtype, a, cfg.n_kv_heads))) return st;
        }
    }
    if (stages & ST_O) {
        if (fused) {   // x += Wo att; x * ffn_norm quantized for gate/up
            if ((st = check_gemv(c, Lw.attn_output.dtype, hidden, Lw.attn_output.data, p))) return st;
            GemvArgs a{};
            a.w0 = Lw.attn_output.data;
            a.total_rows = hidden;
            a.cols = hidden;
            a.nb = p.nb;
            a.row_bytes = p.row_bytes;
            a.x = s->att;
            a.xq = s->xq_att;
            a.y = s->x;
            a.xq_out = s->xq_f;
            a.ss_out = s->ss_f;
            a.gamma_next = (const float *)Lw.ffn_norm.data;
            if ((st = launch_gemv(c, p, "resid", a))) return st;
        } else {
            if ((st = gemv_plain(c, s->xb2, Lw.attn_output.data, Lw.attn_output.dtype, hidden, hidden, s->att, s->xq_u)))
                return st;
            EltArgs e{};
            e.a = s->x;
            e.b = s->xb2;
            e.n = hidden;
            if ((st = c->launch("add_k", dim3((hidden + 255) / 256), dim3(256), 0, e))) return st;
        }
    }

    if (stages & ST_GATEUP) {
        // ---- feed-forward block
        if (fuse_ffn) {
            if ((st = check_gemv(c, Lw.ffn_gate.dtype, hidden, Lw.ffn_gate.data, p))) return st;
            GemvArgs a{};
            a.w0 = Lw.ffn_gate.data;
            a.w1 = Lw.ffn_up.data;
            a.total_rows = 2 * ffn;
            a.cols = hidden;
            a.nb = p.nb;
            a.row_bytes = p.row_bytes;
            a.x = s->x;
            a.gamma = (const float *)Lw.ffn_norm.data;
            a.xq = s->xq_f;
            a.ss_part = s->ss_f;
            a.n_ss = n_ss_res;
            a.eps = cfg.rms_eps;
            a.y = s->hb;
            a.xq_out = s->xq_h;
            if (h32) {
                a.xq_out = nullptr;
                a.ks = 1;
                a.nwaves = GEMV_ONE_WAVES;
                const bool four = (c->gemv_grp & 128) && c->fn("gemv_q4_k_gateup_one4");
                const uint32_t rows_per = GEMV_ONE_WAVES * (four ? 4 : 2), g = (a.total_rows + rows_per - 1) / rows_per;
                if ((st = c->launch(four ? "gemv_q4_k_gateup_one4" : "gemv_q4_k_gateup_one", dim3(g),
                                    dim3(GEMV_ONE_WAVES * 64), (uint32_t)xq_bytes(a.cols), a)))
                    return st;
            } else if ((st = launch_gemv(c, p, "gateup", a))) {
                return st;
            }
        } else {
            EltArgs n{};
            n.a = s->xb;
            n.b = s->x;
            n.w = (const float *)Lw.ffn_norm.data;
            n.cfg = s->rms_cfg;
            n.n = hidden;
            if ((st = c->launch("rms_norm_k", dim3(1), dim3(1024), 0, n))) return st;
            const Tens *mats[2] = {&Lw.ffn_gate, &Lw.ffn_up};
            float *outs[2] = {s->hb, s->hb2};
            for (int m = 0; m < 2; m++)
                if ((st = gemv_plain(c, outs[m], mats[m]->data, mats[m]->dtype, ffn, hidden, s->xb, s->xq_u))) return st;
            EltArgs e{};
            e.a = s->hb;
            e.b = s->hb2;
            e.n = ffn;
            if ((st = c->launch("silu_k", dim3((ffn + 255) / 256), dim3(256), 0, e))) return st;
            if (fused && (st = launch_quant_act(c, s->hb, nullptr, ffn, s->xq_h, nullptr))) return st;
        }
    }
    if (stages & ST_DOWN) {
        if (fused) {   // x += Wdown h; x * next norm quantized for the next QKV / the head
            if ((st = check_gemv(c, Lw.ffn_down.dtype, ffn, Lw.ffn_down.data, p))) return st;
            GemvArgs a{};
            a.w0 = Lw.ffn_down.data;
            a.total_rows = hidden;
            a.cols = ffn;
            a.nb = p.nb;
            a.row_bytes = p.row_bytes;
            a.x = s->hb;
            a.xq = s->xq_h;
            a.y = s->x;
            a.xq_out = s->xq_a;
            a.ss_out = s->ss_a;
            a.gamma_next = next_norm;
            if (h32) {
                a.xq = nullptr; // h arrives in f32 (a.x) and is quantized in LDS
                const IntGeom g = int_geom(c, p.bpi, "resid", a, 0);
                a.ks = g.ks;
                a.nwaves = g.waves;
                if ((st = c->launch("gemv_q4_k_resid_xf", dim3(g.grid), dim3(g.waves * 64), (uint32_t)xq_bytes(a.cols), a)))
                    return st;
            } else if ((st = launch_gemv(c, p, "resid", a))) {
                return st;
            }
            n_ss_a = n_ss_res;
        } else {
            if ((st = gemv_plain(c, s->xb2, Lw.ffn_down.data, Lw.ffn_down.dtype, hidden, ffn, s->hb, s->xq_u))) return st;
            EltArgs e{};
            e.a = s->x;
            e.b = s->xb2;
            e.n = hidden;
            if ((st = c->launch("add_k", dim3((hidden + 255) / 256), dim3(256), 0, e))) return st;
        }
    }
    return IFR_OK;
}

static ifr_status enqueue_step(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, int fused) {
    const ifr_llama2_config &cfg = s->cfg;
    const uint32_t hidden = cfg.hidden, L = cfg.n_layers;
    ifr_status st;

    uint32_t n_ss_a;
    {   // x <- token_embd[tokens[pos]], and x * attn_norm(0) quantized
        EmbedArgs e{};
        e.x = s->x;
        e.table = w->token_embd.data;
        e.tokens = s->tokens;
        e.ctl = s->ctl;
        e.xq_out = s->xq_a;
        e.ss_out = s->ss_a;
        e.gamma = (const float *)w->layers[0].attn_norm.data;
        e.hidden = hidden;
        e.row_bytes = hidden / (uint32_t)qk_of(w->token_embd.dtype) * (uint32_t)bytes_of(w->token_embd.dtype);
        e.fmt = w->token_embd.dtype;
        n_ss_a = (hidden + 255) / 256;
        if ((st = c->launch("embed_k", dim3(n_ss_a), dim3(256), 0, e))) return st;
    }

    for (uint32_t l = 0; l < L; l++)
        if ((st = enqueue_layer(c, s, w, fused, l, ST_LAYER, n_ss_a))) return st;
    return enqueue_head(c, s, w, fused, n_ss_a);
}

// Final RMSNorm, output head, then the argmax (or the sampler) that writes
// the next token and advances the position.  n_ss_a: partial sums of x^2 in
// ss_a (fused path).
static ifr_status enqueue_head(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, int fused, uint32_t n_ss_a) {
    const ifr_llama2_config &cfg = s->cfg;
    const uint32_t hidden = cfg.hidden;
    ifr_status st;
    // ---- final norm, output head, argmax, advance
    const Tens &out = w->output.data ? w->output : w->token_embd; // transformer.rs:376-382
    GemvPlan p;
    if ((st = check_gemv(c, out.dtype, hidden, out.data, p))) return st;
    uint32_t n_parts = 0;
    if (fused) {
        GemvArgs a{};
        a.w0 = out.data;
        a.total_rows = cfg.vocab;
        a.cols = hidden;
        a.nb = p.nb;
        a.row_bytes = p.row_bytes;
        a.x = s->x;
        a.gamma = (const float *)w->output_norm.data;
        a.xq = s->xq_a;
        a.ss_part = s->ss_a;
        a.n_ss = n_ss_a;
        a.eps = cfg.rms_eps;
        a.y = s->logits;
        a.part_keys = s->part_keys;
        // one item per wave and a key per workgroup when the state holds them
        const uint32_t one_grid = (cfg.vocab + GEMV_ONE_WAVES * 2 - 1) / (GEMV_ONE_WAVES * 2);
        const std::string one = std::string("gemv_") + p.fmt + "_head_one";
        if ((c->gemv_grp & 16) && !c->gemv_exact && p.nb <= p.bpi && one_grid <= s->part_keys_cap && c->fn(one)) {
            a.ks = 1;
            a.nwaves = GEMV_ONE_WAVES;
            if ((st = c->launch(one, dim3(one_grid), dim3(GEMV_ONE_WAVES * 64), (uint32_t)xq_bytes(a.cols), a))) return st;
            n_parts = one_grid;
        } else if ((st = launch_gemv(c, p, "head", a, MAX_PARTS, &n_parts))) {
            return st;
        }
    } else {
        EltArgs n{};
        n.a = s->xb;
        n.b = s->x;
        n.w = (const float *)w->output_norm.data;
        n.cfg = s->rms_cfg;
        n.n = hidden;
        if ((st = c->launch("rms_norm_k", dim3(1), dim3(1024), 0, n))) return st;
        if ((st = gemv_plain(c, s->logits, out.data, out.dtype, cfg.vocab, hidden, s->xb, s->xq_u))) return st;
        ArgmaxArgs m{};
        m.v = s->logits;
        m.n = cfg.vocab;
        m.part_keys = s->part_keys;
        n_parts = std::min((cfg.vocab + 255) / 256, MAX_PARTS);
        if ((st = c->launch("argmax_part_k", dim3(n_parts), dim3(256), 0, m))) return st;
    }
    if (s->temperature != 0.0f) {
        // sample_next_token -> Sampler::sample (crates/inferi-chat/src/sampler.rs:91-111)
        SampleArgs a{};
        a.logits = s->logits;
        a.probs = s->probs;
        a.n = cfg.vocab;
        a.temperature = s->temperature;
        a.topp = s->topp;
        a.n_parts = n_parts; // the head's keys of the logits
        a.part_keys = s->part_keys;
        if (s->temperature < 0.0f) { // the order reverses: keys of y itself
            if ((st = launch_keys_of_y(c, s->logits, cfg.vocab, s->temperature, s->part_keys, a.n_parts))) return st;
            a.keys_of_y = 1;
        }
        a.seed = s->seed;
        a.work = s->smp_work;
        a.ctl = s->ctl;
        a.tokens = s->tokens;
        a.rope_pos = &s->rope_cfg->pos;
        a.attn_pos = &s->attn_params->pos;
        return launch_sample(c, a);
    }
    ArgmaxArgs m{};
    m.n_parts = n_parts;
    m.part_keys = s->part_keys;
    m.ctl = s->ctl;
    m.tokens = s->tokens;
    m.rope_pos = &s->rope_cfg->pos;
    m.attn_pos = &s->attn_params->pos;
    return c->launch("argmax_final_k", dim3(1), dim3(1024), 0, m);
}

// =================================================================== C ABI

extern "C" {

IFR_API ifr_status ifr_create(int32_t device, const char *code_object_path, ifr_ctx **out) {
    if (!out) return IFR_EINVAL;
    *out = nullptr;
    auto *c = new ifr_ctx();
    c->device = device;
    auto bail = [&](ifr_status st) {
        g_create_error = c->err;
            if (c->module) hipModuleUnload(c->module);
        if (c->stream) hipStreamDestroy(c->stream);
        delete c;
        return st;
    };
    ifr_status st;
    if ((st = c->hip(hipSetDevice(device), "hipSetDevice"))) return bail(st);
    hipDeviceProp_t prop;
    if ((st = c->hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"))) return bail(st);
    snprintf(c->dev_name, sizeof c->dev_name, "%s (%s)", prop.name, prop.gcnArchName);
    c->n_cu = prop.multiProcessorCount;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return bail(c->fail(IFR_EUNSUPPORTED, "device %d is %s; this build targets gfx950", device, prop.gcnArchName));
    // default-priority stream (no priority argument anywhere)
    if ((st = c->hip(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate"))) return bail(st);
    std::string path;
    if (code_object_path && *code_object_path) {
        path = code_object_path;
    } else {
        Dl_info info;
        if (!dladdr((void *)&ifr_create, &info) || !info.dli_fname)
            return bail(c->fail(IFR_EINVAL, "cannot locate the library to find inferi_kernels.hsaco"));
        path = info.dli_fname;
        size_t slash = path.rfind('/');
        path = (slash == std::string::npos ? std::string(".") : path.substr(0, slash)) + "/inferi_kernels.hsaco";
    }
    if ((st = c->hip(hipModuleLoad(&c->module, path.c_str()), ("hipModuleLoad(" + path + ")").c_str())))
        return bail(st);
    for (auto &e : c->events)
        if ((st = c->hip(hipEventCreate(&e), "hipEventCreate"))) return bail(st);
    if ((st = c->hip(ifr_noalloc_init(device, &c->noalloc_scratch), "hipGetSymbolAddress(scratch)"))) return bail(st);
    *out = c;
    return IFR_OK;
}

IFR_API void ifr_destroy(ifr_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    if (c->scratch) hipFree(c->scratch);
    if (c->xq_scratch) hipFree(c->xq_scratch);
    for (auto &e : c->events)
        if (e) hipEventDestroy(e);
    if (c->module) hipModuleUnload(c->module);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

IFR_API const char *ifr_last_error(const ifr_ctx *c) { return c ? c->err.c_str() : g_create_error.c_str(); }

IFR_API ifr_status ifr_device_info(ifr_ctx *c, char *name, size_t name_len, int32_t *n_cu) {
    if (!c) return IFR_EINVAL;
    if (name && name_len) snprintf(name, name_len, "%s", c->dev_name);
    if (n_cu) *n_cu = c->n_cu;
    return IFR_OK;
}

IFR_API ifr_status ifr_set_option(ifr_ctx *c, const char *key, int64_t value) {
    if (!c || !key) return IFR_EINVAL;
    c->opt_gen++;
    if (!strcmp(key, "gemv_max_grid")) {
        c->gemv_max_grid = (uint32_t)std::max<int64_t>(0, value);
        return IFR_OK;
    }
    if (!strcmp(key, "gemv_exact")) {
        c->gemv_exact = value ? 1 : 0;
        return IFR_OK;
    }
    if (!strcmp(key, "pf_chunk")) {
        if (value < 0 || value > 16384 || value % 64) return c->fail(IFR_EINVAL, "pf_chunk must be a multiple of 64 in [0, 16384]");
        c->pf_chunk = (uint32_t)value;
        return IFR_OK;
    }
    if (!strcmp(key, "pf_tile")) {
        if (value != 0 && value != 128 && value != 256) return c->fail(IFR_EINVAL, "pf_tile must be 0, 128 or 256");
        c->pf_tile = (uint32_t)value;
        return IFR_OK;
    }
    if (!strcmp(key, "pf_ws")) {
        c->pf_ws = value ? 1 : 0;
        return IFR_OK;
    }
    if (!strcmp(key, "pf_rope_fuse")) {
        c->pf_rope_fuse = value ? 1 : 0;
        return IFR_OK;
    }
    if (!strcmp(key, "gemv_grp")) {
        c->gemv_grp = (int)value;
        return IFR_OK;
    }
    if (!strcmp(key, "gemv_waves")) {
        // a power of two, so that the row waves always tile a 16-row group
        if (value < 0 || value > (int64_t)GEMV_INT_MAX_WAVES || (value & (value - 1)))
            return c->fail(IFR_EINVAL, "gemv_waves must be 0, 1, 2, 4, 8 or 16");
        c->gemv_waves = (uint32_t)value;
        return IFR_OK;
    }
    return c->fail(IFR_EINVAL, "unknown option %s", key);
}

IFR_API ifr_status ifr_get_option(ifr_ctx *c, const char *key, int64_t *value) {
    if (!c || !key || !value) return IFR_EINVAL;
    const std::string k = key;
    if (k == "gemv_max_grid") *value = c->gemv_max_grid;
    else if (k == "gemv_exact") *value = c->gemv_exact;
    else if (k == "pf_chunk") *value = c->pf_chunk;
    else if (k == "pf_tile") *value = c->pf_tile;
    else if (k == "pf_ws") *value = c->pf_ws;
    else if (k == "pf_rope_fuse") *value = c->pf_rope_fuse;
    else if (k == "gemv_grp") *value = c->gemv_grp;
    else if (k == "gemv_waves") *value = c->gemv_waves;
    else return c->fail(IFR_EINVAL, "unknown option %s", key);
    return IFR_OK;
}

IFR_API ifr_status ifr_alloc(ifr_ctx *c, size_t bytes, void **p) {
    if (!c || !p) return IFR_EINVAL;
    *p = nullptr;
    return c->hip(hipMalloc(p, std::max<size_t>(bytes, 1)), "hipMalloc");
}

IFR_API ifr_status ifr_free(ifr_ctx *c, void *p) {
    if (!c) return IFR_EINVAL;
    if (!p) return IFR_OK;
    ifr_status st = c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (st) return st;
    return c->hip(hipFree(p), "hipFree");
}

IFR_API ifr_status ifr_upload(ifr_ctx *c, void *dst, const void *src, size_t n) {
    if (!c || (!dst && n) || (!src && n)) return IFR_EINVAL;
    if (!n) return IFR_OK;
    ifr_status st = c->hip(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    if (st) return st;
    return c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

IFR_API ifr_status ifr_download(ifr_ctx *c, void *dst, const void *src, size_t n) {
    if (!c || (!dst && n) || (!src && n)) return IFR_EINVAL;
    if (!n) return IFR_OK;
    ifr_status st = c->hip(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    if (st) return st;
    return c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

IFR_API ifr_status ifr_memset(ifr_ctx *c, void *dst, int32_t v, size_t n) {
    if (!c || (!dst && n)) return IFR_EINVAL;
    return c->hip(hipMemsetAsync(dst, v, n, c->stream), "hipMemsetAsync");
}

IFR_API ifr_status ifr_sync(ifr_ctx *c) {
    if (!c) return IFR_EINVAL;
    return c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

IFR_API ifr_status ifr_event_record(ifr_ctx *c, int32_t slot) {
    if (!c || slot < 0 || slot >= 16) return IFR_EINVAL;
    return c->hip(hipEventRecord(c->events[slot], c->stream), "hipEventRecord");
}

IFR_API ifr_status ifr_event_elapsed(ifr_ctx *c, int32_t a, int32_t b, float *ms) {
    if (!c || a < 0 || a >= 16 || b < 0 || b >= 16 || !ms) return IFR_EINVAL;
    ifr_status st = c->hip(hipEventSynchronize(c->events[b]), "hipEventSynchronize");
    if (st) return st;
    return c->hip(hipEventElapsedTime(ms, c->events[a], c->events[b]), "hipEventElapsedTime");
}

// ------------------------------------------------------------------- ops --

IFR_API ifr_status ifr_dequant(ifr_ctx *c, float *out, const void *blocks, int32_t dtype, uint64_t n) {
    if (!c) return IFR_EINVAL;
    const int qk = qk_of(dtype);
    if (!qk) return c->fail(IFR_EINVAL, "dequant: unknown dtype %d", dtype);
    if (n % (uint64_t)qk) return c->fail(IFR_EINVAL, "dequant: %llu elements not a multiple of %d", (unsigned long long)n, qk);
    if (!n) return IFR_OK;
    if (!out || !blocks) return c->fail(IFR_EINVAL, "dequant: null pointer");
    // f32 fields (F32, Q8_K's d) need 4-byte alignment, f16 fields 2
    if ((uintptr_t)blocks % ((dtype == IFR_F32 || dtype == IFR_Q8_K) ? 4 : 2)) return c->fail(IFR_EINVAL, "dequant: misaligned blocks");
    DequantArgs a{out, (const uint8_t *)blocks, n, dtype, 0};
    const uint64_t g = std::min<uint64_t>((n + 255) / 256, 65536);
    return c->launch("dequant_k", dim3((uint32_t)g), dim3(256), 0, a);
}

IFR_API ifr_status ifr_matmul_quant(ifr_ctx *c, float *out, const void *w, int32_t dtype, uint32_t rows, uint32_t cols,
                                    const float *v) {
    if (!c) return IFR_EINVAL;
    if (!out || !w || !v) return c->fail(IFR_EINVAL, "matmul_quant: null pointer");
    if (!rows) return IFR_OK;
    if ((uintptr_t)v % 16) return c->fail(IFR_EINVAL, "matmul_quant: v not 16-byte aligned");
    // the GEMV quantizes v itself where the code object has that form; the
    // context's scratch is allocated only for the two-launch form
    return gemv_plain(c, out, w, dtype, rows, cols, v, nullptr);
}

IFR_API ifr_status ifr_matmul_quant_noalloc(ifr_ctx *c, float *out, const void *w, int32_t dtype, uint32_t rows,
                                            uint32_t cols, const float *v) {
    if (!c) return IFR_EINVAL;
    if (!out || !w || !v) return c->fail(IFR_EINVAL, "matmul_quant_noalloc: null pointer");
    if (!rows) return IFR_OK;
    if ((uintptr_t)v % 16) return c->fail(IFR_EINVAL, "matmul_quant_noalloc: v not 16-byte aligned");
    if (!c->gemv_exact && xq_bytes(cols) > IFR_NOALLOC_SCRATCH_BYTES)
        return c->fail(IFR_EINVAL, "matmul_quant_noalloc: cols %u needs %llu bytes of scratch, above the fixed %u", cols,
                       (unsigned long long)xq_bytes(cols), (unsigned)IFR_NOALLOC_SCRATCH_BYTES);
    // ifr_matmul_quant's two-launch form (the activation quantization, then
    // the GEMV on it), with the quantized input in the device's fixed array
    // (shared by every call on this device); the same bytes and results as
    // the form that quantizes inside the GEMV
    return gemv_plain(c, out, w, dtype, rows, cols, v, (uint8_t *)c->noalloc_scratch, false);
}

IFR_API uint64_t ifr_activation_bytes(uint32_t n) { return xq_bytes(n); }

IFR_API ifr_status ifr_quantize_activation(ifr_ctx *c, void *xq, const float *x, const float *gamma, uint32_t n,
                                           float *ss_out) {
    if (!c) return IFR_EINVAL;
    if (!xq || !x) return c->fail(IFR_EINVAL, "quantize_activation: null pointer");
    if (n % 32) return c->fail(IFR_EINVAL, "quantize_activation: n must be a multiple of 32");
    if ((uintptr_t)xq % 16) return c->fail(IFR_EINVAL, "quantize_activation: xq not 16-byte aligned");
    if (!n) return IFR_OK;
    return launch_quant_act(c, x, gamma, n, (uint8_t *)xq, ss_out);
}

IFR_API ifr_status ifr_matmul_quant_xq(ifr_ctx *c, float *out, const void *w, int32_t dtype, uint32_t rows,
                                       uint32_t cols, const void *xq) {
    if (!c) return IFR_EINVAL;
    if (!out || !w || !xq) return c->fail(IFR_EINVAL, "matmul_quant_xq: null pointer");
    if (c->gemv_exact) return c->fail(IFR_EINVAL, "matmul_quant_xq: needs the integer path (gemv_exact = 0)");
    if ((uintptr_t)xq % 16) return c->fail(IFR_EINVAL, "matmul_quant_xq: xq not 16-byte aligned");
    if (cols % 32) return c->fail(IFR_EINVAL, "matmul_quant_xq: cols must be a multiple of 32");
    if (!rows) return IFR_OK;
    GemvPlan p;
    ifr_status st = check_gemv(c, dtype, cols, w, p);
    if (st) return st;
    GemvArgs a{};
    a.w0 = (const uint8_t *)w;
    a.total_rows = rows;
    a.cols = cols;
    a.nb = p.nb;
    a.row_bytes = p.row_bytes;
    a.xq = (const uint8_t *)xq;
    a.y = out;
    return launch_gemv(c, p, "plain", a);
}

IFR_API ifr_status ifr_rms_norm(ifr_ctx *c, const ifr_rms_norm_config *cfg, float *out, const float *value,
                                const float *weight, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!cfg || !out || !value || !weight) return c->fail(IFR_EINVAL, "rms_norm: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = out;
    a.b = value;
    a.w = weight;
    a.cfg = cfg;
    a.n = n;
    return c->launch("rms_norm_k", dim3(1), dim3(1024), 0, a);
}

IFR_API ifr_status ifr_add(ifr_ctx *c, float *x, const float *b, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!x || !b) return c->fail(IFR_EINVAL, "add: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = x;
    a.b = b;
    a.n = n;
    return c->launch("add_k", dim3((n + 255) / 256), dim3(256), 0, a);
}

IFR_API ifr_status ifr_rope(ifr_ctx *c, int32_t variant, const ifr_rope_config *cfg, float *q, uint32_t q_len, float *k,
                            uint32_t k_len) {
    if (!c) return IFR_EINVAL;
    if (!cfg || !q) return c->fail(IFR_EINVAL, "rope: null pointer");
    if (variant != IFR_ROPE_ORIGINAL && variant != IFR_ROPE_NEOX) return c->fail(IFR_EINVAL, "rope: bad variant");
    if (q_len % 2) return c->fail(IFR_EINVAL, "rope: q_len must be even (ops/rope.rs:39-44)");
    if (k_len % 2) return c->fail(IFR_EINVAL, "rope: k_len must be even");
    if (k_len && !k) return c->fail(IFR_EINVAL, "rope: null k");
    if (!q_len) return IFR_OK;
    EltArgs a{};
    a.a = q;
    a.k = k;
    a.cfg = cfg;
    a.n = q_len;
    a.n2 = k_len;
    a.variant = variant;
    return c->launch("rope_k", dim3((q_len / 2 + 255) / 256), dim3(256), 0, a);
}

IFR_API ifr_status ifr_silu(ifr_ctx *c, float *h1, const float *h2, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!h1 || !h2) return c->fail(IFR_EINVAL, "silu: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = h1;
    a.b = h2;
    a.n = n;
    return c->launch("silu_k", dim3((n + 255) / 256), dim3(256), 0, a);
}

// ------------------------------------------------- strided operand views

IFR_API ifr_status ifr_rms_norm_view(ifr_ctx *c, const ifr_rms_norm_config *cfg, float *out, ifr_view ov,
                                     const float *value, ifr_view vv, const float *weight, ifr_view wv, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!cfg || !out || !value || !weight) return c->fail(IFR_EINVAL, "rms_norm_view: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = out + ov.offset;
    a.b = value + vv.offset;
    a.w = weight + wv.offset;
    a.sa = ov.stride;
    a.sb = vv.stride;
    a.sw = wv.stride;
    a.cfg = cfg;
    a.n = n;
    return c->launch("rms_norm_k", dim3(1), dim3(1024), 0, a);
}

IFR_API ifr_status ifr_add_view(ifr_ctx *c, float *x, ifr_view xv, const float *b, ifr_view bv, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!x || !b) return c->fail(IFR_EINVAL, "add_view: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = x + xv.offset;
    a.b = b + bv.offset;
    a.sa = xv.stride;
    a.sb = bv.stride;
    a.n = n;
    return c->launch("add_k", dim3((n + 255) / 256), dim3(256), 0, a);
}

IFR_API ifr_status ifr_rope_view(ifr_ctx *c, int32_t variant, const ifr_rope_config *cfg, float *q, ifr_view qv,
                                 uint32_t q_len, float *k, ifr_view kv, uint32_t k_len) {
    if (!c) return IFR_EINVAL;
    if (!cfg || !q) return c->fail(IFR_EINVAL, "rope_view: null pointer");
    if (variant != IFR_ROPE_ORIGINAL && variant != IFR_ROPE_NEOX) return c->fail(IFR_EINVAL, "rope_view: bad variant");
    if (q_len % 2 || k_len % 2) return c->fail(IFR_EINVAL, "rope_view: q_len and k_len must be even (ops/rope.rs:39-44)");
    if (k_len && !k) return c->fail(IFR_EINVAL, "rope_view: null k");
    if (!q_len) return IFR_OK;
    EltArgs a{};
    a.a = q + qv.offset;
    a.k = k ? k + kv.offset : nullptr;
    a.sa = qv.stride;
    a.sk = kv.stride;
    a.cfg = cfg;
    a.n = q_len;
    a.n2 = k_len;
    a.variant = variant;
    return c->launch("rope_k", dim3((q_len / 2 + 255) / 256), dim3(256), 0, a);
}

IFR_API ifr_status ifr_silu_view(ifr_ctx *c, float *h1, ifr_view av, const float *h2, ifr_view bv, uint32_t n) {
    if (!c) return IFR_EINVAL;
    if (!h1 || !h2) return c->fail(IFR_EINVAL, "silu_view: null pointer");
    if (!n) return IFR_OK;
    EltArgs a{};
    a.a = h1 + av.offset;
    a.b = h2 + bv.offset;
    a.sa = av.stride;
    a.sb = bv.stride;
    a.n = n;
    return c->launch("silu_k", dim3((n + 255) / 256), dim3(256), 0, a);
}

IFR_API ifr_status ifr_attention(ifr_ctx *c, const ifr_attn_params *p, const ifr_attn_params *dev_p, const float *q,
                                 const void *kc, const void *vc, int32_t kv_dtype, float *xb) {
    if (!c) return IFR_EINVAL;
    if (!p || !dev_p || !q || !kc || !vc || !xb) return c->fail(IFR_EINVAL, "attention: null pointer");
    if (kv_dtype != IFR_F16 && kv_dtype != IFR_F32) return c->fail(IFR_EINVAL, "attention: kv dtype F16 or F32");
    if (!p->head_size || p->head_size % 8 || p->head_size > 128)
        return c->fail(IFR_EUNSUPPORTED, "attention: head_size %u (a multiple of 8, at most 128)", p->head_size);
    if (!p->n_heads || !p->kv_mul || p->n_heads % p->kv_mul) return c->fail(IFR_EINVAL, "attention: n_heads %% kv_mul");
    const uint32_t g = p->kv_mul;
    const uint32_t n_kv = p->n_heads / g;
    if (p->kv_dim != n_kv * p->head_size) return c->fail(IFR_EINVAL, "attention: kv_dim != n_kv_heads * head_size");
    if (p->pos >= p->seq_len) return c->fail(IFR_EINVAL, "attention: pos %u >= seq_len %u", p->pos, p->seq_len);
    if (p->pos >= (1u << 30)) return c->fail(IFR_EUNSUPPORTED, "attention: pos %u too large", p->pos);
    if ((uintptr_t)q % 16 || (uintptr_t)kc % 16 || (uintptr_t)vc % 16)
        return c->fail(IFR_EINVAL, "attention: q and caches must be 16-byte aligned");
    const uint32_t T = p->pos + 1;
    const uint32_t S = attn_splits_for(T, p->head_size);
    const size_t part_o = (size_t)p->n_heads * S * p->head_size, part_ml = (size_t)p->n_heads * S * 2;
    ifr_status st = c->ensure_scratch((part_o + part_ml) * sizeof(float));
    if (st) return st;
    AttnArgs a{};
    a.q = q;
    a.k_cache = kc;
    a.v_cache = vc;
    a.out = xb;
    a.part_o = (float *)c->scratch;
    a.part_ml = (float *)c->scratch + part_o;
    a.pos = &dev_p->pos;
    a.kv_dim = p->kv_dim;
    a.n_splits = S;
    a.seq_cap = T;
    a.spec_rows = T;
    a.n_out = p->n_heads * p->head_size;
    a.head_size = p->head_size;
    a.kv_mul = g;
    return launch_attn(c, kv_dtype, a, n_kv);
}

IFR_API ifr_status ifr_argmax(ifr_ctx *c, const float *v, uint32_t n, uint32_t *dev_index) {
    if (!c) return IFR_EINVAL;
    if (!v || !dev_index) return c->fail(IFR_EINVAL, "argmax: null pointer");
    if (!n) return c->fail(IFR_EINVAL, "argmax: empty input");
    ifr_status st = c->ensure_scratch(MAX_PARTS * sizeof(uint64_t));
    if (st) return st;
    ArgmaxArgs a{};
    a.v = v;
    a.n = n;
    a.part_keys = (uint64_t *)c->scratch;
    const uint32_t parts = std::min((n + 255) / 256, MAX_PARTS);
    if ((st = c->launch("argmax_part_k", dim3(parts), dim3(256), 0, a))) return st;
    ArgmaxArgs b{};
    b.n_parts = parts;
    b.part_keys = (uint64_t *)c->scratch;
    b.out_index = dev_index;
    return c->launch("argmax_final_k", dim3(1), dim3(1024), 0, b);
}

IFR_API ifr_status ifr_sample(ifr_ctx *c, const float *logits, float *probs, uint32_t n, float temperature, float topp,
                              const float *dev_coin, uint32_t *dev_index) {
    if (!c) return IFR_EINVAL;
    if (!logits || !dev_index) return c->fail(IFR_EINVAL, "sample: null pointer");
    if (!n) return c->fail(IFR_EINVAL, "sample: empty input");
    if (!std::isfinite(temperature) || std::isnan(topp))
        return c->fail(IFR_EINVAL, "sample: temperature must be finite and topp a number");
    if (temperature == 0.0f) return ifr_argmax(c, logits, n, dev_index); // sampler.rs:33-35
    if (!probs || !dev_coin) return c->fail(IFR_EINVAL, "sample: null pointer");
    if (n > SAMPLE_MAX_N) return c->fail(IFR_EUNSUPPORTED, "sample: n %u above %u", n, SAMPLE_MAX_N);
    if (((uintptr_t)logits | (uintptr_t)probs) & 15) return c->fail(IFR_EINVAL, "sample: logits/probs not 16-byte aligned");
    ifr_status st = c->ensure_scratch(MAX_PARTS * sizeof(uint64_t) + SAMPLE_WORK_BYTES);
    if (st) return st;
    SampleArgs a{};
    a.logits = logits;
    a.probs = probs;
    a.n = n;
    a.temperature = temperature;
    a.topp = topp;
    a.part_keys = (uint64_t *)c->scratch;
    a.keys_of_y = 1;
    if ((st = launch_keys_of_y(c, logits, n, temperature, (uint64_t *)c->scratch, a.n_parts))) return st;
    a.coin = dev_coin;
    a.work = (uint8_t *)c->scratch + MAX_PARTS * sizeof(uint64_t);
    a.out_index = dev_index;
    return launch_sample(c, a);
}

IFR_API ifr_status ifr_quantize(ifr_ctx *c, void *out, const float *x, int32_t dtype, uint64_t n) {
    if (!c) return IFR_EINVAL;
    const int qk = qk_of(dtype);
    if (!qk) return c->fail(IFR_EINVAL, "quantize: unknown dtype %d", dtype);
    if (n % (uint64_t)qk) return c->fail(IFR_EINVAL, "quantize: n not a multiple of %d", qk);
    if (!n) return IFR_OK;
    if (!out || !x) return c->fail(IFR_EINVAL, "quantize: null pointer");
    QuantArgs a{(uint8_t *)out, x, n / (uint64_t)qk, dtype, 0};
    const uint64_t g = (a.n_blocks + 63) / 64;
    if (g > 0x7FFFFFFFull) return c->fail(IFR_EINVAL, "quantize: too many blocks for one launch");
    return c->launch("quantize_k", dim3((uint32_t)g), dim3(64), 0, a);
}

IFR_API ifr_status ifr_fill_normal(ifr_ctx *c, float *out, uint64_t n, uint64_t seed, uint64_t stream, float mean,
                                   float std) {
    if (!c) return IFR_EINVAL;
    if (!n) return IFR_OK;
    if (!out) return c->fail(IFR_EINVAL, "fill_normal: null pointer");
    FillArgs a{};
    a.out = out;
    a.n = n;
    // key = mix of (seed, stream): distinct streams never share pairs
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull + 0x2545F4914F6CDD1Dull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    a.key = z ^ (z >> 31);
    a.mean = mean;
    a.std = std;
    const uint64_t pairs = (n + 1) / 2;
    const uint32_t g = (uint32_t)std::min<uint64_t>((pairs + 255) / 256, 65536);
    return c->launch("fill_normal_k", dim3(g), dim3(256), 0, a);
}

// ----------------------------------------------------------------- model --

IFR_API ifr_status ifr_llama2_weights_create(ifr_ctx *c, const ifr_llama2_config *cfg, ifr_llama2_weights **out) {
    if (!c || !out) return IFR_EINVAL;
    *out = nullptr;
    ifr_status st = validate_cfg(c, cfg);
    if (st) return st;
    static std::atomic<uint64_t> next_id{0};
    auto *w = new ifr_llama2_weights();
    w->ctx = c;
    w->cfg = *cfg;
    w->id = ++next_id;
    w->layers.resize(cfg->n_layers);
    *out = w;
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_weights_set(ifr_llama2_weights *w, const char *name, int32_t dtype, const void *data,
                                          uint32_t rows, uint32_t cols) {
    if (!w || !name) return IFR_EINVAL;
    ifr_ctx *c = w->ctx;
    const ifr_llama2_config &cfg = w->cfg;
    w->gen++; // a graph captured with the table before this call is stale
    if (!data) return c->fail(IFR_EINVAL, "%s: null data", name);
    if (!qk_of(dtype)) return c->fail(IFR_EINVAL, "%s: unknown dtype %d", name, dtype);
    const uint32_t kv_dim = cfg.hidden / cfg.n_heads * cfg.n_kv_heads;
    Tens t{dtype, (const uint8_t *)data, rows, cols};
    auto want = [&](uint32_t r, uint32_t cc, bool vec) -> ifr_status {
        if (rows != r || cols != cc) return c->fail(IFR_EINVAL, "%s: shape %ux%u, expected %ux%u", name, rows, cols, r, cc);
        if (vec && dtype != IFR_F32) return c->fail(IFR_EUNSUPPORTED, "%s: norm weights must be F32", name);
        if (cc % (uint32_t)qk_of(dtype)) return c->fail(IFR_EINVAL, "%s: cols not a multiple of the block", name);
        if (!vec && !gemv_fmt_name(dtype) && strcmp(name, "token_embd.weight"))
            return c->fail(IFR_EUNSUPPORTED, "%s: dtype %d has no GEMV kernel", name, dtype);
        return IFR_OK;
    };
    ifr_status st;
    if (!strcmp(name, "token_embd.weight")) {
        if ((st = want(cfg.vocab, cfg.hidden, false))) return st;
        w->token_embd = t;
        return IFR_OK;
    }
    if (!strcmp(name, "output.weight")) {
        if ((st = want(cfg.vocab, cfg.hidden, false))) return st;
        w->output = t;
        return IFR_OK;
    }
    if (!strcmp(name, "output_norm.weight")) {
        if ((st = want(1, cfg.hidden, true))) return st;
        w->output_norm = t;
        return IFR_OK;
    }
    unsigned layer = 0;
    char field[64] = {0}, kind[8] = {0};
    if (sscanf(name, "blk.%u.%63[a-z_].%7[a-z]", &layer, field, kind) != 3 || layer >= cfg.n_layers)
        return c->fail(IFR_EINVAL, "unknown tensor name %s", name);
    LayerW &L = w->layers[layer];
    const std::string f = field;
    if (!strcmp(kind, "bias")) { // Qwen2's QKV biases: F32 vectors
        if (f == "attn_q") { if ((st = want(1, cfg.hidden, true))) return st; L.q_bias = t; }
        else if (f == "attn_k") { if ((st = want(1, kv_dim, true))) return st; L.k_bias = t; }
        else if (f == "attn_v") { if ((st = want(1, kv_dim, true))) return st; L.v_bias = t; }
        else return c->fail(IFR_EINVAL, "unknown tensor name %s", name);
        return IFR_OK;
    }
    if (strcmp(kind, "weight")) return c->fail(IFR_EINVAL, "unknown tensor name %s", name);
    if (f == "attn_norm") { if ((st = want(1, cfg.hidden, true))) return st; L.attn_norm = t; }
    else if (f == "ffn_norm") { if ((st = want(1, cfg.hidden, true))) return st; L.ffn_norm = t; }
    else if (f == "attn_q") { if ((st = want(cfg.hidden, cfg.hidden, false))) return st; L.attn_q = t; }
    else if (f == "attn_k") { if ((st = want(kv_dim, cfg.hidden, false))) return st; L.attn_k = t; }
    else if (f == "attn_v") { if ((st = want(kv_dim, cfg.hidden, false))) return st; L.attn_v = t; }
    else if (f == "attn_output") { if ((st = want(cfg.hidden, cfg.hidden, false))) return st; L.attn_output = t; }
    else if (f == "ffn_gate") { if ((st = want(cfg.ffn, cfg.hidden, false))) return st; L.ffn_gate = t; }
    else if (f == "ffn_up") { if ((st = want(cfg.ffn, cfg.hidden, false))) return st; L.ffn_up = t; }
    else if (f == "ffn_down") { if ((st = want(cfg.hidden, cfg.ffn, false))) return st; L.ffn_down = t; }
    else return c->fail(IFR_EINVAL, "unknown tensor name %s", name);
    return IFR_OK;
}

IFR_API void ifr_llama2_weights_destroy(ifr_llama2_weights *w) {
    if (!w) return;
    if (!w->owned.empty()) {
        hipStreamSynchronize(w->ctx->stream);
        for (void *p : w->owned) hipFree(p);
    }
    delete w;
}

static ifr_status gguf_u32(const ifr_gguf *g, const std::string &key, uint32_t &v) {
    if (ifr_gguf_get_scalar(g, key.c_str(), IFR_GGUF_U32, &v))
        return ifr_free_error() = "gguf: " + key + " missing or not a U32", IFR_EINVAL;
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_config_from_gguf(const ifr_gguf *g, ifr_llama2_config *cfg) {
    if (!g || !cfg) return ifr_free_error() = "null argument", IFR_EINVAL;
    // the architecture picks the key prefix and the RoPE pairing, as
    // ChatLlm::from_gguf (inferi-chat/src/llm.rs:71-92) picks LlamaModelType
    // (models/llama2/mod.rs:18-30)
    const char *arch = nullptr;
    uint64_t alen = 0;
    bool qwen2 = false;
    if (!ifr_gguf_get_string(g, "general.architecture", &arch, &alen)) {
        std::string a(arch, alen);
        for (char &ch : a) ch = (char)tolower((unsigned char)ch);
        qwen2 = a.find("qwen2") != std::string::npos;
    }
    ifr_llama2_config c{};
    const std::string m = qwen2 ? "qwen2" : "llama";
    ifr_status st;
    if ((st = gguf_u32(g, m + ".embedding_length", c.hidden)) || (st = gguf_u32(g, m + ".feed_forward_length", c.ffn)) ||
        (st = gguf_u32(g, m + ".block_count", c.n_layers)) || (st = gguf_u32(g, m + ".attention.head_count", c.n_heads)) ||
        (st = gguf_u32(g, m + ".attention.head_count_kv", c.n_kv_heads)) ||
        (st = gguf_u32(g, m + ".context_length", c.max_pos)))
        return st;
    uint64_t vocab = 0;
    int32_t et;
    if (ifr_gguf_get_array(g, "tokenizer.ggml.tokens", &et, &vocab, nullptr))
        return ifr_free_error() = "gguf: tokenizer.ggml.tokens missing or not an array", IFR_EINVAL;
    if (vocab == 0 || vocab > 0xFFFFFFFFull) return ifr_free_error() = "gguf: vocabulary size out of range", IFR_EINVAL;
    c.vocab = (uint32_t)vocab;
    c.rope_theta = 10000.0f;
    c.rms_eps = 1.0e-6f;
    // optional keys: absent -> default; present with another type -> error (as_f32 panics)
    for (auto [key, dst] : {std::pair<std::string, float *>{m + ".rope.freq_base", &c.rope_theta},
                            {m + ".attention.layer_norm_rms_epsilon", &c.rms_eps}}) {
        if (ifr_gguf_metadata_type(g, key.c_str(), nullptr, nullptr) < 0) continue;
        if (ifr_gguf_get_scalar(g, key.c_str(), IFR_GGUF_F32, dst))
            return ifr_free_error() = "gguf: " + key + " is not an F32", IFR_EINVAL;
    }
    c.kv_dtype = IFR_F32;
    c.rope_variant = qwen2 ? IFR_ROPE_NEOX : IFR_ROPE_ORIGINAL;
    *cfg = c;
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_weights_from_gguf(ifr_ctx *c, const ifr_gguf *g, const ifr_llama2_config *cfg,
                                                ifr_llama2_weights **out) {
    if (!c || !g || !cfg || !out) return IFR_EINVAL;
    *out = nullptr;
    ifr_llama2_weights *w = nullptr;
    ifr_status st = ifr_llama2_weights_create(c, cfg, &w);
    if (st) return st;
    std::vector<std::string> names = {"token_embd.weight", "output_norm.weight"};
    if (ifr_gguf_tensor_info(g, "output.weight", nullptr, nullptr, nullptr, nullptr, nullptr) == IFR_OK)
        names.push_back("output.weight");
    for (uint32_t l = 0; l < cfg->n_layers; l++) {
        for (const char *f : {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up",
                              "ffn_down"})
            names.push_back("blk." + std::to_string(l) + "." + f + ".weight");
        for (const char *f : {"attn_q", "attn_k", "attn_v"}) { // Qwen2's biases, when the file has them
            const std::string b = "blk." + std::to_string(l) + "." + f + ".bias";
            if (ifr_gguf_tensor_info(g, b.c_str(), nullptr, nullptr, nullptr, nullptr, nullptr) == IFR_OK)
                names.push_back(b);
        }
    }
    for (const std::string &name : names) {
        int32_t dtype;
        uint64_t dims[4];
        uint32_t rank;
        const void *data;
        uint64_t bytes;
        if (ifr_gguf_tensor_info(g, name.c_str(), &dtype, dims, &rank, &data, &bytes)) {
            ifr_llama2_weights_destroy(w);
            return c->fail(IFR_EINVAL, "gguf: %s", ifr_free_error().c_str());
        }
        if (!data || rank < 1 || rank > 2 || dims[2] != 1 || dims[3] != 1 || dims[0] > 0xFFFFFFFFull ||
            dims[1] > 0xFFFFFFFFull) {
            ifr_llama2_weights_destroy(w);
            return c->fail(IFR_EINVAL, "gguf: %s has rank %u or a type without data", name.c_str(), rank);
        }
        // rank 1: a vector of dims[0] (rows 1); rank 2: [rows, cols] (gguf.rs:591-593)
        const uint32_t rows = rank == 1 ? 1u : (uint32_t)dims[0], cols = rank == 1 ? (uint32_t)dims[0] : (uint32_t)dims[1];
        void *dev = nullptr;
        if ((st = ifr_alloc(c, std::max<size_t>(bytes, 16), &dev))) {
            ifr_llama2_weights_destroy(w);
            return st;
        }
        w->owned.push_back(dev);
        if ((st = c->hip(hipMemcpy(dev, data, bytes, hipMemcpyHostToDevice), "hipMemcpy(gguf tensor)")) ||
            (st = ifr_llama2_weights_set(w, name.c_str(), dtype, dev, rows, cols))) {
            ifr_llama2_weights_destroy(w);
            return st;
        }
    }
    *out = w;
    return IFR_OK;
}

static void state_free(ifr_llama2_state *s) {
    if (!s) return;
    hipStreamSynchronize(s->ctx->stream);
    if (s->graph) hipGraphExecDestroy(s->graph);
    for (auto &r : s->retired) {
        hipGraphExecDestroy(r.first);
        hipEventDestroy(r.second);
    }
    for (void *p : s->allocs) hipFree(p);
    delete s;
}

IFR_API ifr_status ifr_llama2_state_create(ifr_ctx *c, const ifr_llama2_config *cfg, ifr_llama2_state **out) {
    if (!c || !out) return IFR_EINVAL;
    *out = nullptr;
    ifr_status st = validate_cfg(c, cfg);
    if (st) return st;
    auto *s = new ifr_llama2_state();
    s->ctx = c;
    s->cfg = *cfg;
    s->head_size = cfg->hidden / cfg->n_heads;
    s->kv_dim = s->head_size * cfg->n_kv_heads;
    s->kv_mul = cfg->n_heads / cfg->n_kv_heads;
    s->n_splits = attn_splits_for(cfg->max_pos, s->head_size);
    auto alloc = [&](size_t bytes, void **p) -> ifr_status {
        ifr_status e = c->hip(hipMalloc(p, std::max<size_t>(bytes, 16)), "hipMalloc(state)");
        if (e) return e;
        s->allocs.push_back(*p);
        return c->hip(hipMemset(*p, 0, std::max<size_t>(bytes, 16)), "hipMemset(state)");
    };
    const size_t H = cfg->hidden, F = cfg->ffn, KV = s->kv_dim;
    const size_t esz = cfg->kv_dtype == IFR_F16 ? 2 : 4;
    s->layer_kv_bytes = ((size_t)cfg->max_pos * KV * esz + 255) & ~(size_t)255;
#define A(ptr, bytes) if ((st = alloc((bytes), (void **)&(ptr)))) { state_free(s); return st; }
    A(s->x, H * 4) A(s->xb, H * 4) A(s->xb2, H * 4) A(s->q, H * 4) A(s->att, H * 4)
    A(s->ktmp, KV * 4) A(s->vtmp, KV * 4) A(s->hb, F * 4) A(s->hb2, F * 4)
    A(s->logits, (size_t)cfg->vocab * 4) A(s->probs, (size_t)cfg->vocab * 4) A(s->smp_work, SAMPLE_WORK_BYTES)
    A(s->tokens, ((size_t)cfg->max_pos + 1) * 4)
    A(s->ctl, sizeof(StepCtl)) A(s->rms_cfg, sizeof(ifr_rms_norm_config)) A(s->rope_cfg, sizeof(ifr_rope_config))
    A(s->attn_params, sizeof(ifr_attn_params))
    s->part_keys_cap = std::max(MAX_PARTS, (uint32_t)((cfg->vocab + GEMV_ONE_WAVES * 2 - 1) / (GEMV_ONE_WAVES * 2)));
    A(s->part_keys, (size_t)s->part_keys_cap * 8)
    A(s->part_o, (size_t)cfg->n_heads * s->n_splits * s->head_size * 4)
    A(s->part_ml, (size_t)cfg->n_heads * s->n_splits * 2 * 4)
    A(s->rope_tab, (size_t)s->head_size / 2 * 4)
    A(s->xq_a, xq_bytes(H)) A(s->xq_f, xq_bytes(H)) A(s->xq_att, xq_bytes(H)) A(s->xq_h, xq_bytes(F))
    A(s->xq_u, xq_bytes(std::max(H, F))) A(s->ss_a, H / 16 * 4) A(s->ss_f, H / 16 * 4)
    A(s->kcache, s->layer_kv_bytes * cfg->n_layers)
    A(s->vcache, s->layer_kv_bytes * cfg->n_layers)
#undef A
    ifr_rms_norm_config rc{cfg->rms_eps};
    if ((st = c->hip(hipMemcpy(s->rms_cfg, &rc, sizeof rc, hipMemcpyHostToDevice), "hipMemcpy"))) { state_free(s); return st; }
    {   // theta of pair i: base^(-(2i)/hs), f32 exponent, f64 power rounded once
        std::vector<float> tab(s->head_size / 2);
        for (uint32_t i = 0; i < s->head_size / 2; i++)
            tab[i] = (float)std::pow((double)cfg->rope_theta, (double)(-(float)(2 * i) / (float)s->head_size));
        if ((st = c->hip(hipMemcpy(s->rope_tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice), "hipMemcpy"))) {
            state_free(s);
            return st;
        }
    }
    *out = s;
    return ifr_llama2_state_reset(s, nullptr, 0, 0);
}

IFR_API void ifr_llama2_state_destroy(ifr_llama2_state *s) { state_free(s); }

IFR_API ifr_status ifr_llama2_state_reset(ifr_llama2_state *s, const uint32_t *prompt, uint32_t n, uint32_t pos) {
    if (!s) return IFR_EINVAL;
    ifr_ctx *c = s->ctx;
    const ifr_llama2_config &cfg = s->cfg;
    if (n && !prompt) return c->fail(IFR_EINVAL, "null prompt");
    if (n > cfg.max_pos) return c->fail(IFR_EINVAL, "prompt longer than max_pos");
    if (pos >= cfg.max_pos) return c->fail(IFR_EINVAL, "pos %u >= max_pos %u", pos, cfg.max_pos);
    for (uint32_t i = 0; i < n; i++)
        if (prompt[i] >= cfg.vocab) return c->fail(IFR_EINVAL, "prompt token %u out of range", prompt[i]);
    ifr_status st;
    if ((st = c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize"))) return st;
    if (n && (st = c->hip(hipMemcpy(s->tokens, prompt, n * 4, hipMemcpyHostToDevice), "hipMemcpy(tokens)"))) return st;
    StepCtl ctl{pos, n, cfg.max_pos, 0};
    s->host_pos = pos;
    ifr_rope_config rope{s->head_size, s->kv_dim, pos, cfg.rope_theta};
    ifr_attn_params ap{cfg.max_pos, s->kv_dim, s->kv_mul, cfg.n_heads, s->head_size, pos};
    if ((st = c->hip(hipMemcpy(s->ctl, &ctl, sizeof ctl, hipMemcpyHostToDevice), "hipMemcpy(ctl)"))) return st;
    if ((st = c->hip(hipMemcpy(s->rope_cfg, &rope, sizeof rope, hipMemcpyHostToDevice), "hipMemcpy(rope)"))) return st;
    return c->hip(hipMemcpy(s->attn_params, &ap, sizeof ap, hipMemcpyHostToDevice), "hipMemcpy(attn)");
}

static ifr_status check_weights(ifr_ctx *c, const ifr_llama2_state *s, const ifr_llama2_weights *w) {
    if (!w) return c->fail(IFR_EINVAL, "null weights");
    const ifr_llama2_config &a = s->cfg, &b = w->cfg;
    if (a.n_layers != b.n_layers || a.hidden != b.hidden || a.ffn != b.ffn || a.n_heads != b.n_heads ||
        a.n_kv_heads != b.n_kv_heads || a.vocab != b.vocab)
        return c->fail(IFR_EINVAL, "state and weights were made for different configs");
    if (!w->token_embd.data || !w->output_norm.data) return c->fail(IFR_EINVAL, "token_embd/output_norm not set");
    for (uint32_t l = 0; l < b.n_layers; l++) {
        const LayerW &L = w->layers[l];
        const Tens *all[] = {&L.attn_norm, &L.attn_q, &L.attn_k, &L.attn_v, &L.attn_output,
                             &L.ffn_norm, &L.ffn_gate, &L.ffn_up, &L.ffn_down};
        for (const Tens *t : all)
            if (!t->data) return c->fail(IFR_EINVAL, "layer %u has an unset tensor", l);
    }
    const Tens &out = w->output.data ? w->output : w->token_embd;
    if (!gemv_fmt_name(out.dtype)) return c->fail(IFR_EUNSUPPORTED, "output head dtype %d has no GEMV kernel", out.dtype);
    return IFR_OK;
}

// ---------------------------------------------------------------- prefill --

// Y[m][n] (+)= sum_k Xh[m][k] * deq(W)[n][k] on the matrix cores, the weight
// tiles dequantized to f16 inside the kernels (device/pf_gemm.h: 256 x 256
// tiles; device/prefill.h gemm_f16_body: 128 x 128 tiles, the same results
// bit for bit).
static uint32_t pf_row_bytes(const Tens &w) {
    return (w.cols / (uint32_t)qk_of(w.dtype)) * (uint32_t)bytes_of(w.dtype);
}

enum PfEpi { PF_EPI_STORE = 0, PF_EPI_ADD = 1, PF_EPI_SWIGLU = 2 };
// Products with at least this many 256 x 256 tiles take that form (every
// product of a 4096-token pass at the 8B shape: 256 to 1792 tiles); smaller
// ones run 128 x 128 tiles, four times the workgroups.
constexpr uint32_t PF_BIG_TILES_MIN = 128;

// One product of a pass: nm (1 to 3) matrices of one type stacked by rows
// into Y[M][ldy] f32 (stored or added), or (SwiGLU) gate m[0] and up m[1]
// into h[M][ldy] = f16(up * silu(gate)).  X rows (pitch ldx halves) must be
// 16-byte aligned.  rope (may be null): the stacked Q | K | V store product
// may fuse pf_rope_kv_k's work into its epilogue (warp-specialized form
// only); *fused says whether it did.
static ifr_status launch_pf_gemm(ifr_ctx *c, const void *xh, uint32_t ldx, const Tens *const *m, int nm, void *y,
                                 uint32_t ldy, uint32_t M, PfEpi epi, const PfArgs *rope = nullptr,
                                 bool *fused = nullptr) {
    if (fused) *fused = false;
    PfGemmArgs g{};
    g.x = xh;
    g.w0 = m[0]->data;
    g.w1 = nm > 1 ? m[1]->data : m[0]->data;
    g.w2 = nm > 2 ? m[2]->data : g.w1;
    g.y = y;
    g.M = M;
    g.K = m[0]->cols;
    g.ldx = ldx;
    g.ldy = ldy;
    g.row_bytes = pf_row_bytes(*m[0]);
    if (epi == PF_EPI_SWIGLU) {
        g.n1 = g.n2 = m[0]->rows;
        g.N = 2 * m[0]->rows;
    } else {
        g.n1 = m[0]->rows;
        g.n2 = g.n1 + (nm > 1 ? m[1]->rows : 0);
        g.N = g.n2 + (nm > 2 ? m[2]->rows : 0);
    }
    g.tiles_n = (g.N + PF_BIG_TILE - 1) / PF_BIG_TILE;
    g.tiles_m = (M + PF_BIG_TILE - 1) / PF_BIG_TILE;
    static const char *epi_name[3] = {"store", "add", "swiglu"};
    // the large form addresses X rows with 32-bit byte offsets
    const bool big_ok = (uint64_t)M * ldx * 2 < (1ull << 32);
    const bool big = big_ok && (c->pf_tile == 256 || (c->pf_tile == 0 && g.tiles_n * g.tiles_m >= PF_BIG_TILES_MIN));
    if (big && c->pf_ws && m[0]->dtype == IFR_Q4_K) {
        // a last round of at most 128 tiles (half the CUs) runs as twice as
        // many 256 x 128 halves, one round over every CU
        const uint32_t tiles = g.tiles_n * g.tiles_m, tail = tiles % PF_WS_ROUND;
        g.tiles_full = tail != 0 && tail <= PF_WS_ROUND / 2 ? tiles - tail : tiles;
        if (rope && epi == PF_EPI_STORE && nm == 3) {
            g.rope = 1;
            g.rope_cs = rope->rope_cs;
            g.q_bias = rope->q_bias;
            g.k_bias = rope->k_bias;
            g.v_bias = rope->v_bias;
            g.k_cache = rope->k_cache;
            g.v_cache = rope->v_cache;
            g.head_size = rope->head_size;
            g.p0 = rope->p0;
            g.kv_f16 = rope->kv_f16;
            if (fused) *fused = true;
        }
        return c->launch(std::string("pf_gemm_q4_k_ws_") + epi_name[epi], dim3(tiles + (tiles - g.tiles_full)),
                         dim3(PF_WS_THREADS), 0, g);
    }
    if (big)
        return c->launch(std::string("pf_gemm_") + gemv_fmt_name(m[0]->dtype) + "_" + epi_name[epi],
                         dim3(g.tiles_n * g.tiles_m), dim3(PF_BIG_THREADS), 0, g);
    const dim3 grid((g.N + PF_GEMM_TILE - 1) / PF_GEMM_TILE, (M + PF_GEMM_TILE - 1) / PF_GEMM_TILE);
    return c->launch(std::string("gemm_") + gemv_fmt_name(m[0]->dtype) + "_f16_" + epi_name[epi], grid, dim3(256), 0, g);
}

// A matrix the prefill GEMM takes: a quantized GGUF type, K a whole number
// of its 64-element steps, rows aligned for the tile loads (16 bytes for
// Q4_K/Q5_K, 4 for the others).
static ifr_status check_pf_matrix(ifr_ctx *c, int32_t dtype, uint32_t cols, const void *w) {
    if (!gemv_fmt_name(dtype)) return c->fail(IFR_EUNSUPPORTED, "prefill GEMM: dtype %d has no tile loader", dtype);
    if (cols % 64 || cols % (uint32_t)qk_of(dtype)) return c->fail(IFR_EUNSUPPORTED, "prefill GEMM: cols %u not a multiple of 64 and of the block", cols);
    const uintptr_t need = gemv_align(dtype);
    if ((uintptr_t)w % need) return c->fail(IFR_EINVAL, "prefill GEMM: weights not %u-byte aligned", (unsigned)need);
    return IFR_OK;
}

IFR_API ifr_status ifr_gemm_quant(ifr_ctx *c, float *y, const void *w, int32_t dtype, uint32_t rows, uint32_t cols,
                                  const void *x_f16, uint32_t m, int32_t accumulate) {
    if (!c) return IFR_EINVAL;
    if (!y || !w || !x_f16) return c->fail(IFR_EINVAL, "gemm_quant: null pointer");
    if (!rows || !m || !cols) return c->fail(IFR_EINVAL, "gemm_quant: rows, m and cols must be > 0");
    ifr_status st = check_pf_matrix(c, dtype, cols, w);
    if (st) return st;
    if ((uintptr_t)x_f16 % 16) return c->fail(IFR_EINVAL, "gemm_quant: x must be 16-byte aligned");
    Tens t;
    t.dtype = dtype;
    t.data = (const uint8_t *)w;
    t.rows = rows;
    t.cols = cols;
    const Tens *mats[1] = {&t};
    return launch_pf_gemm(c, x_f16, cols, mats, 1, y, rows, m, accumulate ? PF_EPI_ADD : PF_EPI_STORE);
}

// The layer matrices in the prefill products' order.
static void pf_mats(const LayerW &L, const Tens *m[7]) {
    m[0] = &L.attn_q;
    m[1] = &L.attn_k;
    m[2] = &L.attn_v;
    m[3] = &L.attn_output;
    m[4] = &L.ffn_gate;
    m[5] = &L.ffn_up;
    m[6] = &L.ffn_down;
}

static ifr_status pf_ensure_scratch(ifr_llama2_state *s) {
    if (s->pf_x) return IFR_OK;
    ifr_ctx *c = s->ctx;
    const ifr_llama2_config &cfg = s->cfg;
    // a pass covers up to C tokens (no more than the cache holds): larger
    // passes give the GEMMs and the causal attention more workgroups (512
    // tokens per pass measured 2.7x slower on a 4095-token prompt)
    const uint32_t C = std::min(c->pf_chunk ? c->pf_chunk : PF_CHUNK, (cfg.max_pos + 63) / 64 * 64);
    const uint32_t H = cfg.hidden, F = cfg.ffn, qd = cfg.n_heads * s->head_size;
    s->pf_chunk = C;
    s->pf_ldh = std::max(H, qd);
    auto A = [&](size_t bytes, void **p) -> ifr_status {
        ifr_status e = c->hip(hipMalloc(p, bytes), "hipMalloc(prefill)");
        if (!e) s->allocs.push_back(*p);
        return e;
    };
    ifr_status st;
    if ((st = A((size_t)C * H * 4, (void **)&s->pf_x))) return st;
    if ((st = A((size_t)C * s->pf_ldh * 2, (void **)&s->pf_xh))) return st;
    if ((st = A((size_t)C * (qd + 2 * s->kv_dim) * 4, (void **)&s->pf_qkv))) return st;
    if ((st = A((size_t)C * s->head_size * 4, (void **)&s->pf_rope_cs))) return st;
    return A((size_t)C * F * 2, (void **)&s->pf_h);
}

IFR_API ifr_status ifr_llama2_prefill(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, uint32_t n) {
    if (!c || !s) return IFR_EINVAL;
    ifr_status st = check_weights(c, s, w);
    if (st) return st;
    const ifr_llama2_config &cfg = s->cfg;
    bool mixed_ffn = false; // a layer whose gate and up types differ
    for (const LayerW &L : w->layers) {
        const Tens *mats[7];
        pf_mats(L, mats);
        for (const Tens *t : mats)
            if ((st = check_pf_matrix(c, t->dtype, t->cols, t->data))) return st;
        mixed_ffn |= L.ffn_gate.dtype != L.ffn_up.dtype;
    }
    if (!n) return IFR_OK;
    if ((st = pf_ensure_scratch(s))) return st;
    // the position lives on the device: read it once
    StepCtl ctl;
    if ((st = c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize"))) return st;
    if ((st = c->hip(hipMemcpy(&ctl, s->ctl, sizeof ctl, hipMemcpyDeviceToHost), "hipMemcpy(ctl)"))) return st;
    const uint32_t pos0 = ctl.pos;
    if ((uint64_t)pos0 + n > cfg.max_pos) return c->fail(IFR_EINVAL, "prefill: %u tokens from position %u exceed max_pos", n, pos0);
    if (pos0 + n > ctl.n_forced) return c->fail(IFR_EINVAL, "prefill: positions up to %u hold no prompt token", pos0 + n);
    if (mixed_ffn && !s->pf_gu) {
        // separate gate and up products into f32, then the SiLU pass
        const size_t bytes = (size_t)s->pf_chunk * 2 * cfg.ffn * 4;
        if ((st = c->hip(hipMalloc((void **)&s->pf_gu, bytes), "hipMalloc(prefill gate/up)"))) return st;
        s->allocs.push_back(s->pf_gu);
    }

    const uint32_t H = cfg.hidden, F = cfg.ffn, hs = s->head_size, kvd = s->kv_dim, qd = cfg.n_heads * hs;
    const uint32_t G = s->kv_mul, ldq = qd + 2 * kvd, ldh = s->pf_ldh;
    char attn_name[64];
    snprintf(attn_name, sizeof attn_name, "pf_attn_%s_h%u", cfg.kv_dtype == IFR_F16 ? "f16" : "f32", attn_hsp(hs));
    const uint32_t attn_qt = 128 / G; // device/prefill.h: PFA_ROWS / kv_mul queries per workgroup
    for (uint32_t c0 = 0; c0 < n; c0 += s->pf_chunk) {
        const uint32_t M = std::min(s->pf_chunk, n - c0), p0 = pos0 + c0;
        PfArgs a{};
        a.x = s->pf_x;
        a.xh = s->pf_xh;
        a.ldh = ldh;
        a.hidden = H;
        a.eps = cfg.rms_eps;
        a.M = M;
        a.p0 = p0;
        a.tokens = s->tokens;
        a.table = w->token_embd.data;
        a.row_bytes = H / (uint32_t)qk_of(w->token_embd.dtype) * (uint32_t)bytes_of(w->token_embd.dtype);
        a.fmt = w->token_embd.dtype;
        a.qkv = s->pf_qkv;
        a.ld_qkv = ldq;
        a.q_dim = qd;
        a.kv_dim = kvd;
        a.head_size = hs;
        a.rope_tab = s->rope_tab;
        a.kv_f16 = cfg.kv_dtype == IFR_F16;
        a.ffn = F;
        a.gu = s->pf_gu;
        a.h = s->pf_h;
        a.neox = cfg.rope_variant == IFR_ROPE_NEOX;
        a.kv_mul = G;
        a.rope_cs = s->pf_rope_cs;
        if ((st = c->launch("pf_embed_k", dim3(M), dim3(256), 0, a))) return st;
        if ((st = c->launch("pf_rope_tab_k", dim3(M), dim3(64), 0, a))) return st;
        // the Q/K/V product may take over pf_rope_kv_k: pairs (2i, 2i + 1),
        // and the epilogue's 32-bit offsets cover the cache and qkv rows
        const bool fuse_ok = c->pf_rope_fuse && !a.neox && s->layer_kv_bytes < (1ull << 32) &&
                             (uint64_t)M * ldq * 4 < (1ull << 32);
        for (uint32_t l = 0; l < cfg.n_layers; l++) {
            const LayerW &L = w->layers[l];
            const Tens *mats[7];
            pf_mats(L, mats);
            a.k_cache = s->kcache + (size_t)l * s->layer_kv_bytes;
            a.v_cache = s->vcache + (size_t)l * s->layer_kv_bytes;
            a.gamma = (const float *)L.attn_norm.data;
            a.q_bias = (const float *)L.q_bias.data;
            a.k_bias = (const float *)L.k_bias.data;
            a.v_bias = (const float *)L.v_bias.data;
            if ((st = c->launch("pf_rmsnorm_f16_k", dim3(M), dim3(256), 0, a))) return st;
            // Q, K and V into adjacent columns of qkv: each run of matrices of
            // one type as one stacked product
            bool fused = false;
            for (int i = 0, col = 0; i < 3;) {
                int j = i + 1;
                while (j < 3 && mats[j]->dtype == mats[i]->dtype) j++;
                if ((st = launch_pf_gemm(c, s->pf_xh, ldh, mats + i, j - i, s->pf_qkv + col, ldq, M, PF_EPI_STORE,
                                         fuse_ok ? &a : nullptr, &fused)))
                    return st;
                for (int k = i; k < j; k++) col += (int)mats[k]->rows;
                i = j;
            }
            if (!fused && (st = c->launch("pf_rope_kv_k", dim3(M), dim3(256), 0, a))) return st;
            // the last layer's attention and FFN feed only its residual
            // stream, which nothing reads (the pass's product is the KV rows;
            // the next decode step starts from the embedding): not run
            if (l + 1 == cfg.n_layers) break;
            if ((st = c->launch(attn_name, dim3(cfg.n_kv_heads, (M + attn_qt - 1) / attn_qt), dim3(256), 0, a))) return st;
            if ((st = launch_pf_gemm(c, s->pf_xh, ldh, mats + 3, 1, s->pf_x, H, M, PF_EPI_ADD))) return st;
            a.gamma = (const float *)L.ffn_norm.data;
            if ((st = c->launch("pf_rmsnorm_f16_k", dim3(M), dim3(256), 0, a))) return st;
            if (L.ffn_gate.dtype == L.ffn_up.dtype) {
                // h = up * silu(gate) in the product's epilogue
                if ((st = launch_pf_gemm(c, s->pf_xh, ldh, mats + 4, 2, s->pf_h, F, M, PF_EPI_SWIGLU))) return st;
            } else {
                if ((st = launch_pf_gemm(c, s->pf_xh, ldh, mats + 4, 1, s->pf_gu, 2 * F, M, PF_EPI_STORE))) return st;
                if ((st = launch_pf_gemm(c, s->pf_xh, ldh, mats + 5, 1, s->pf_gu + F, 2 * F, M, PF_EPI_STORE))) return st;
                if ((st = c->launch("pf_silu_k", dim3((F + 255) / 256, M), dim3(256), 0, a))) return st;
            }
            if ((st = launch_pf_gemm(c, s->pf_h, F, mats + 6, 1, s->pf_x, H, M, PF_EPI_ADD))) return st;
        }
    }
    // advance the device position (and the unfused path's op parameters)
    const uint32_t pos = pos0 + n;
    if ((st = c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize"))) return st;
    ctl.pos = pos;
    s->host_pos = pos;
    ifr_rope_config rope{hs, kvd, pos, cfg.rope_theta};
    ifr_attn_params ap{cfg.max_pos, kvd, G, cfg.n_heads, hs, pos};
    if ((st = c->hip(hipMemcpy(s->ctl, &ctl, sizeof ctl, hipMemcpyHostToDevice), "hipMemcpy(ctl)"))) return st;
    if ((st = c->hip(hipMemcpy(s->rope_cfg, &rope, sizeof rope, hipMemcpyHostToDevice), "hipMemcpy(rope)"))) return st;
    return c->hip(hipMemcpy(s->attn_params, &ap, sizeof ap, hipMemcpyHostToDevice), "hipMemcpy(attn)");
}

static void host_advance(ifr_llama2_state *s, uint32_t steps) {
    s->host_pos = (uint32_t)std::min<uint64_t>((uint64_t)s->host_pos + steps, s->cfg.max_pos - 1);
}

IFR_API ifr_status ifr_llama2_launch(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, int32_t fused) {
    if (!c || !s) return IFR_EINVAL;
    ifr_status st = check_weights(c, s, w);
    if (st) return st;
    s->step_spec = attn_spec_for(s->host_pos, s->cfg.max_pos);
    if ((st = enqueue_step(c, s, w, fused))) return st;
    host_advance(s, 1);
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_generate(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, uint32_t n_steps,
                                       int32_t use_graph) {
    if (!c || !s) return IFR_EINVAL;
    ifr_status st = check_weights(c, s, w);
    if (st) return st;
    if (!use_graph) {
        for (uint32_t i = 0; i < n_steps; i++) {
            s->step_spec = attn_spec_for(s->host_pos, s->cfg.max_pos);
            if ((st = enqueue_step(c, s, w, 1))) return st;
            host_advance(s, 1);
        }
        return IFR_OK;
    }
    // one captured step per position bucket: replayed for the steps of the
    // bucket, captured again (after the stream drains) when the position
    // leaves it, or when the weights, options or sampler changed
    for (size_t i = 0; i < s->retired.size();) {
        if (hipEventQuery(s->retired[i].second) == hipSuccess) {
            hipGraphExecDestroy(s->retired[i].first);
            hipEventDestroy(s->retired[i].second);
            s->retired[i] = s->retired.back();
            s->retired.pop_back();
        } else {
            i++;
        }
    }
    uint32_t done = 0;
    while (done < n_steps) {
        const uint32_t spec = attn_spec_for(s->host_pos, s->cfg.max_pos);
        if (!s->graph || s->graph_wid != w->id || s->graph_wgen != w->gen || s->graph_fused != 1 ||
            s->graph_opt != c->opt_gen || s->graph_sampler != s->sampler_gen || s->graph_spec != spec) {
            if (s->graph) {
                hipEvent_t ev = nullptr;
                if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess &&
                    hipEventRecord(ev, c->stream) == hipSuccess) {
                    s->retired.emplace_back(s->graph, ev);
                } else {
                    if (ev) hipEventDestroy(ev);
                    hipStreamSynchronize(c->stream);
                    hipGraphExecDestroy(s->graph);
                }
                s->graph = nullptr;
            }
            s->step_spec = spec;
            if ((st = c->hip(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture")))
                return st;
            ifr_status est = enqueue_step(c, s, w, 1);
            hipGraph_t g = nullptr;
            st = c->hip(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture");
            if (est) {
                if (g) hipGraphDestroy(g);
                return est;
            }
            if (st) return st;
            st = c->hip(hipGraphInstantiate(&s->graph, g, nullptr, nullptr, 0), "hipGraphInstantiate");
            hipGraphDestroy(g);
            if (st) return st;
            s->graph_wid = w->id;
            s->graph_wgen = w->gen;
            s->graph_fused = 1;
            s->graph_opt = c->opt_gen;
            s->graph_sampler = s->sampler_gen;
            s->graph_spec = spec;
        }
        // steps left in this bucket (the last position, max_pos - 1, repeats)
        const uint32_t left = s->host_pos + 1 >= s->cfg.max_pos ? n_steps - done
                            : std::min(n_steps - done, spec - s->host_pos);
        for (uint32_t i = 0; i < left; i++)
            if ((st = c->hip(hipGraphLaunch(s->graph, c->stream), "hipGraphLaunch"))) return st;
        host_advance(s, left);
        done += left;
    }
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_time_stage(ifr_ctx *c, ifr_llama2_state *s, const ifr_llama2_weights *w, const char *stage,
                                         uint32_t iters, float *us_per_launch) {
    if (!c || !s || !stage || !us_per_launch) return IFR_EINVAL;
    if (!iters) return c->fail(IFR_EINVAL, "time_stage: zero iterations");
    ifr_status st = check_weights(c, s, w);
    if (st) return st;
    const std::string n = stage;
    const uint32_t mask = n == "qkv" ? ST_QKV : n == "attention" ? ST_ATTN : n == "attn_output" ? ST_O
                        : n == "ffn_gate_up" ? ST_GATEUP : n == "ffn_down" ? ST_DOWN : 0u;
    if (!mask) return c->fail(IFR_EINVAL, "time_stage: unknown stage '%s'", stage);
    const uint32_t L = s->cfg.n_layers;
    s->step_spec = attn_spec_for(s->host_pos, s->cfg.max_pos);
    auto pass = [&]() -> ifr_status {
        for (uint32_t l = 0; l < L; l++) {
            uint32_t n_ss = s->cfg.hidden / 16; // the partial sums a previous step's down GEMV left in ss_a
            ifr_status e = enqueue_layer(c, s, w, 1, l, mask, n_ss);
            if (e) return e;
        }
        return IFR_OK;
    };
    if ((st = pass())) return st; // warm-up
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((st = c->hip(hipEventCreate(&e0), "hipEventCreate"))) return st;
    if ((st = c->hip(hipEventCreate(&e1), "hipEventCreate"))) {
        hipEventDestroy(e0);
        return st;
    }
    st = c->hip(hipEventRecord(e0, c->stream), "hipEventRecord");
    for (uint32_t i = 0; i < iters && !st; i++) st = pass();
    if (!st) st = c->hip(hipEventRecord(e1, c->stream), "hipEventRecord");
    if (!st) st = c->hip(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.0f;
    if (!st) st = c->hip(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (!st) *us_per_launch = ms * 1000.0f / (float)((uint64_t)iters * L);
    return st;
}

IFR_API ifr_status ifr_llama2_set_sampler(ifr_llama2_state *s, float temperature, float topp, uint64_t seed) {
    if (!s) return IFR_EINVAL;
    if (!std::isfinite(temperature) || std::isnan(topp))
        return s->ctx->fail(IFR_EINVAL, "sampler: temperature must be finite and topp a number");
    if (temperature != 0.0f && s->cfg.vocab > SAMPLE_MAX_N)
        return s->ctx->fail(IFR_EUNSUPPORTED, "sampler: vocab %u above %u", s->cfg.vocab, SAMPLE_MAX_N);
    s->temperature = temperature;
    s->topp = topp;
    s->seed = seed;
    s->sampler_gen++;
    return IFR_OK;
}

IFR_API ifr_status ifr_llama2_read_tokens(ifr_llama2_state *s, uint32_t *host, uint32_t start, uint32_t n) {
    if (!s || (!host && n)) return IFR_EINVAL;
    if ((uint64_t)start + n > (uint64_t)s->cfg.max_pos + 1) return s->ctx->fail(IFR_EINVAL, "token range out of bounds");
    return ifr_download(s->ctx, host, s->tokens + start, (size_t)n * 4);
}

IFR_API ifr_status ifr_llama2_state_buffer(ifr_llama2_state *s, const char *name, int32_t layer, void **p, size_t *bytes) {
    if (!s || !name || !p) return IFR_EINVAL;
    const ifr_llama2_config &cfg = s->cfg;
    size_t b = 0;
    std::string n = name;
    if (n == "x") { *p = s->x; b = cfg.hidden * 4; }
    else if (n == "q") { *p = s->q; b = cfg.hidden * 4; }
    else if (n == "att") { *p = s->att; b = cfg.hidden * 4; }
    else if (n == "logits") { *p = s->logits; b = (size_t)cfg.vocab * 4; }
    else if (n == "probs") { *p = s->probs; b = (size_t)cfg.vocab * 4; }
    else if (n == "pos") { *p = &s->ctl->pos; b = 4; }
    else if (n == "part_ml") { *p = s->part_ml; b = (size_t)cfg.n_kv_heads * s->n_splits * s->kv_mul * 2 * 4; }
    else if (n == "part_o") { *p = s->part_o; b = (size_t)cfg.n_kv_heads * s->n_splits * s->kv_mul * s->head_size * 4; }
    else if (n == "tokens") { *p = s->tokens; b = ((size_t)cfg.max_pos + 1) * 4; }
    else if (n == "key_cache" || n == "value_cache") {
        if (layer < 0 || (uint32_t)layer >= cfg.n_layers) return s->ctx->fail(IFR_EINVAL, "layer out of range");
        *p = (n == "key_cache" ? s->kcache : s->vcache) + (size_t)layer * s->layer_kv_bytes;
        b = (size_t)cfg.max_pos * s->kv_dim * (cfg.kv_dtype == IFR_F16 ? 2 : 4);
    } else return s->ctx->fail(IFR_EINVAL, "unknown state buffer %s", name);
    if (bytes) *bytes = b;
    return IFR_OK;
}

} // extern "C"

// gfx950 kernels of inferi_hip, compiled into one code object
// (hipcc --genco --offload-arch=gfx950) that the host library loads with
// hipModuleLoad and launches with hipModuleLaunchKernel.  Every kernel takes
// one argument struct (csrc/kargs.h) by value.
#include "device/attention.h"
#include "device/elementwise.h"
#include "device/gemv.h"
#include "device/prefill.h"
#include "device/sample.h"

using namespace ifr;

// gemv_<fmt>_<mode>: integer path (x quantized by its producer, v_dot4),
// up to 16 waves per workgroup; gemv_<fmt>_<mode>_f32: exact fp32 path.
// Four waves per SIMD (at most 128 VGPRs) keeps enough loads in flight.
#define GEMV_KERNEL(NAME, FMT, MODE)                                                                   \
    extern "C" __global__ void __launch_bounds__(GEMV_INT_MAX_WAVES * 64)                            \
        __attribute__((amdgpu_waves_per_eu(GEMV_INT_WPE, 8))) NAME(GemvArgs a) {                     \
        gemv_int_body<FMT, MODE, GEMV_INT_PIPE, GEMV_INT_NI>(a);                                     \
    }                                                                                                \
    extern "C" __global__ void __launch_bounds__(GemvGeom<MODE>::W * 64)                             \
        __attribute__((amdgpu_waves_per_eu(4, 8))) NAME##_f32(GemvArgs a) {                          \
        gemv_f32_body<FMT, MODE>(a);                                                                 \
    }

#ifndef GEMV_INT_PIPE
#define GEMV_INT_PIPE false
#endif
#ifndef GEMV_INT_NI
#define GEMV_INT_NI 1
#endif
#ifndef GEMV_INT_WPE
#define GEMV_INT_WPE 4
#endif

// one-item form of the local modes (plain, qkv)
#define GEMV_ONE_KERNEL(NAME, FMT, MODE)                                                               \
    extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) NAME##_one(GemvArgs a) {         \
        gemv_one_body<FMT, MODE>(a);                                                                 \
    }

// one-item form of the grouped modes: R rows per wave, RW row waves, KS K-slices
#define GEMV_GRP_KERNEL(NAME, FMT, MODE, R, RW, KS)                                                     \
    extern "C" __global__ void __launch_bounds__(RW * KS * 64) NAME##_r##R##w##RW##k##KS(GemvArgs a) { \
        gemv_grp_body<FMT, MODE, R, RW, KS>(a);                                                         \
    }
// gate/up with h in f32, and the down GEMV that quantizes its f32 input itself
extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) gemv_q4_k_gateup_one(GemvArgs a) {
    gemv_one_body<Q4_K, GEMV_GATEUP>(a);
}
// one-item forms with four rows per wave (option gemv_grp bits 7 and 8)
extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) gemv_q4_k_gateup_one4(GemvArgs a) {
    gemv_one_body<Q4_K, GEMV_GATEUP, 4>(a);
}
extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) gemv_q4_k_qkv_one4(GemvArgs a) {
    gemv_one_body<Q4_K, GEMV_QKV, 4>(a);
}
extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) gemv_q4_k_plain_one4(GemvArgs a) {
    gemv_one_body<Q4_K, GEMV_PLAIN, 4>(a);
}
extern "C" __global__ void __launch_bounds__(GEMV_INT_MAX_WAVES * 64)
    __attribute__((amdgpu_waves_per_eu(GEMV_INT_WPE, 8))) gemv_q4_k_resid_xf(GemvArgs a) {
    gemv_int_body<Q4_K, GEMV_RESID, GEMV_INT_PIPE, GEMV_INT_NI, true>(a);
}
// the output head in workgroups of at most 4 waves with up to 256 VGPRs (the
// Q6_K integer step spills at 128)
extern "C" __global__ void __launch_bounds__(4 * 64) __attribute__((amdgpu_waves_per_eu(2, 8)))
gemv_q6_k_head_w2(GemvArgs a) {
    gemv_int_body<Q6_K, GEMV_HEAD, GEMV_INT_PIPE, GEMV_INT_NI>(a);
}
GEMV_GRP_KERNEL(gemv_q4_k_resid, Q4_K, GEMV_RESID, 2, 8, 1)
GEMV_GRP_KERNEL(gemv_q4_k_resid, Q4_K, GEMV_RESID, 4, 4, 4)
GEMV_GRP_KERNEL(gemv_q4_k_gateup, Q4_K, GEMV_GATEUP, 4, 8, 1)
GEMV_GRP_KERNEL(gemv_q4_k_gateup, Q4_K, GEMV_GATEUP, 2, 16, 1)

// the plain one-item form on an f32 x it quantizes itself (ifr_matmul_quant)
#define GEMV_ONE_XF_KERNEL(NAME, FMT)                                                                 \
    extern "C" __global__ void __launch_bounds__(GEMV_ONE_WAVES * 64) NAME##_one_xf(GemvArgs a) {      \
        gemv_one_body<FMT, GEMV_PLAIN, 2, true>(a);                                                   \
    }

// the looping plain form on an f32 x it quantizes itself (ifr_matmul_quant, K past one step)
#define GEMV_XF_KERNEL(NAME, FMT)                                                                      \
    extern "C" __global__ void __launch_bounds__(GEMV_INT_MAX_WAVES * 64)                            \
        __attribute__((amdgpu_waves_per_eu(GEMV_INT_WPE, 8))) NAME##_xf(GemvArgs a) {                  \
        gemv_int_body<FMT, GEMV_PLAIN, GEMV_INT_PIPE, GEMV_INT_NI, true>(a);                         \
    }

#define GEMV_ALL_MODES(FMTNAME, FMT)                  \
    GEMV_ONE_KERNEL(gemv_##FMTNAME##_plain, FMT, GEMV_PLAIN) \
    GEMV_ONE_XF_KERNEL(gemv_##FMTNAME##_plain, FMT)          \
    GEMV_XF_KERNEL(gemv_##FMTNAME##_plain, FMT)              \
    GEMV_ONE_KERNEL(gemv_##FMTNAME##_qkv, FMT, GEMV_QKV)     \
    GEMV_ONE_KERNEL(gemv_##FMTNAME##_head, FMT, GEMV_HEAD)   \
    GEMV_KERNEL(gemv_##FMTNAME##_plain, FMT, GEMV_PLAIN)   \
    GEMV_KERNEL(gemv_##FMTNAME##_resid, FMT, GEMV_RESID)   \
    GEMV_KERNEL(gemv_##FMTNAME##_qkv, FMT, GEMV_QKV)       \
    GEMV_KERNEL(gemv_##FMTNAME##_gateup, FMT, GEMV_GATEUP) \
    GEMV_KERNEL(gemv_##FMTNAME##_head, FMT, GEMV_HEAD)

GEMV_ALL_MODES(q4_k, Q4_K)
GEMV_ALL_MODES(q5_k, Q5_K)
GEMV_ALL_MODES(q6_k, Q6_K)
GEMV_ALL_MODES(q8_0, Q8_0)
GEMV_ALL_MODES(q4_0, Q4_0)
GEMV_ALL_MODES(q4_1, Q4_1)
GEMV_ALL_MODES(q5_0, Q5_0)
GEMV_ALL_MODES(q5_1, Q5_1)
GEMV_ALL_MODES(q8_k, Q8_K)
GEMV_ALL_MODES(f16, F16)
GEMV_ALL_MODES(f32, F32)

// decode attention: head sizes padded to 64 or 128, 1..8 query heads per workgroup
#define ATTN_KERNEL(HSP, GT)                                                                        \
    extern "C" __global__ void __launch_bounds__(256) attn_f16_h##HSP##_g##GT(AttnArgs a) {         \
        attn_split_body<HSP, GT, true>(a);                                                          \
    }                                                                                               \
    extern "C" __global__ void __launch_bounds__(256) attn_f32_h##HSP##_g##GT(AttnArgs a) {         \
        attn_split_body<HSP, GT, false>(a);                                                         \
    }
#define ATTN_KERNELS(HSP) \
    ATTN_KERNEL(HSP, 1) ATTN_KERNEL(HSP, 2) ATTN_KERNEL(HSP, 3) ATTN_KERNEL(HSP, 4) \
    ATTN_KERNEL(HSP, 5) ATTN_KERNEL(HSP, 6) ATTN_KERNEL(HSP, 7) ATTN_KERNEL(HSP, 8)
ATTN_KERNELS(64)
ATTN_KERNELS(128)
extern "C" __global__ void __launch_bounds__(64) attn_merge(AttnArgs a) { attn_merge_body(a); }

extern "C" __global__ void __launch_bounds__(1024) rms_norm_k(EltArgs a) { rms_norm_body(a); }
extern "C" __global__ void __launch_bounds__(256) rope_k(EltArgs a) { rope_body(a); }
extern "C" __global__ void __launch_bounds__(256) silu_k(EltArgs a) { silu_body(a); }
extern "C" __global__ void __launch_bounds__(256) add_k(EltArgs a) { add_body(a); }
extern "C" __global__ void __launch_bounds__(256) argmax_part_k(ArgmaxArgs a) { argmax_part_body(a); }
extern "C" __global__ void __launch_bounds__(1024) argmax_final_k(ArgmaxArgs a) { argmax_final_body(a); }
extern "C" __global__ void __launch_bounds__(256) sample_exp_k(SampleArgs a) { sample_exp_body(a); }
extern "C" __global__ void __launch_bounds__(256) sample_prob_k(SampleArgs a) { sample_prob_body(a); }
extern "C" __global__ void __launch_bounds__(256) sample_group_k(SampleArgs a) { sample_group_body(a); }
extern "C" __global__ void __launch_bounds__(1024) sample_select_k(SampleArgs a) { sample_select_body(a); }
extern "C" __global__ void __launch_bounds__(256) embed_k(EmbedArgs a) { embed_body(a); }
extern "C" __global__ void __launch_bounds__(256) quant_act_k(QActArgs a) { quant_act_body(a); }
extern "C" __global__ void __launch_bounds__(256) kv_store_k(KvStoreArgs a) { kv_store_body(a); }
extern "C" __global__ void __launch_bounds__(256) dequant_k(DequantArgs a) { dequant_body(a); }
extern "C" __global__ void __launch_bounds__(64) quantize_k(QuantArgs a) { quantize_body(a); }
extern "C" __global__ void __launch_bounds__(256) fill_normal_k(FillArgs a) { fill_normal_body(a); }

// prompt (prefill) path: the GEMM in 256 x 256 tiles (eight waves, two per
// SIMD) and in 128 x 128 tiles, each with the store, accumulate and SwiGLU
// epilogues
#define PF_GEMM_KERNELS(FMTNAME, FMT)                                                                             \
    extern "C" __global__ void __launch_bounds__(PG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))           \
    pf_gemm_##FMTNAME##_store(PfGemmArgs a) {                                                                     \
        pf_gemm_body<FMT, PG_STORE>(a);                                                                           \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(PG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))           \
    pf_gemm_##FMTNAME##_add(PfGemmArgs a) {                                                                       \
        pf_gemm_body<FMT, PG_ADD>(a);                                                                             \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(PG_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))           \
    pf_gemm_##FMTNAME##_swiglu(PfGemmArgs a) {                                                                    \
        pf_gemm_body<FMT, PG_SWIGLU>(a);                                                                          \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) gemm_##FMTNAME##_f16_store(PfGemmArgs a) {                  \
        gemm_f16_body<FMT, PG_STORE>(a);                                                                          \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) gemm_##FMTNAME##_f16_add(PfGemmArgs a) {                    \
        gemm_f16_body<FMT, PG_ADD>(a);                                                                            \
    }                                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) gemm_##FMTNAME##_f16_swiglu(PfGemmArgs a) {                 \
        gemm_f16_body<FMT, PG_SWIGLU>(a);                                                                         \
    }
PF_GEMM_KERNELS(q4_k, Q4_K)
PF_GEMM_KERNELS(q5_k, Q5_K)
PF_GEMM_KERNELS(q6_k, Q6_K)
PF_GEMM_KERNELS(q8_k, Q8_K)
PF_GEMM_KERNELS(q8_0, Q8_0)
PF_GEMM_KERNELS(q4_0, Q4_0)
PF_GEMM_KERNELS(q4_1, Q4_1)
PF_GEMM_KERNELS(q5_0, Q5_0)
PF_GEMM_KERNELS(q5_1, Q5_1)
PF_GEMM_KERNELS(f16, F16)
PF_GEMM_KERNELS(f32, F32)
// the warp-specialized Q4_K product (option pf_ws): 12 waves, three per SIMD
extern "C" __global__ void __launch_bounds__(PGW_THREADS) pf_gemm_q4_k_ws_store(PfGemmArgs a) {
    pf_gemm_ws_body<PG_STORE>(a);
}
extern "C" __global__ void __launch_bounds__(PGW_THREADS) pf_gemm_q4_k_ws_add(PfGemmArgs a) {
    pf_gemm_ws_body<PG_ADD>(a);
}
extern "C" __global__ void __launch_bounds__(PGW_THREADS) pf_gemm_q4_k_ws_swiglu(PfGemmArgs a) {
    pf_gemm_ws_body<PG_SWIGLU>(a);
}
extern "C" __global__ void __launch_bounds__(256) pf_embed_k(PfArgs a) { pf_embed_body(a); }
extern "C" __global__ void __launch_bounds__(256) pf_rmsnorm_f16_k(PfArgs a) { pf_rmsnorm_f16_body(a); }
extern "C" __global__ void __launch_bounds__(64) pf_rope_tab_k(PfArgs a) { pf_rope_tab_body(a); }
extern "C" __global__ void __launch_bounds__(256) pf_rope_kv_k(PfArgs a) { pf_rope_kv_body(a); }
extern "C" __global__ void __launch_bounds__(256) pf_silu_k(PfArgs a) { pf_silu_body(a); }

#define PF_ATTN_KERNEL(HSP)                                                                     \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PF_ATTN_WPE, 8)))  \
    pf_attn_f16_h##HSP(PfArgs a) {                                                                   \
        pf_attn_body<HSP, true>(a);                                                              \
    }                                                                                            \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PF_ATTN_WPE, 8)))  \
    pf_attn_f32_h##HSP(PfArgs a) {                                                                   \
        pf_attn_body<HSP, false>(a);                                                             \
    }
#ifndef PF_ATTN_WPE
#define PF_ATTN_WPE 2
#endif
PF_ATTN_KERNEL(64)
PF_ATTN_KERNEL(128)

// All device code of the library, compiled into one gfx950 code object
// (hipcc --genco) that the host library embeds and loads with
// hipModuleLoadData.  Kernel names are extern "C" so the host can look them
// up with hipModuleGetFunction:
//   cq_gemv_<fmt>_x<f16|f32>_y<f32|f16>   decode GEMV (m-tiles of 16)
//   cq_gemv1_<fmt>_y<f32|f16>[_epi|_gated] decode GEMV, one fp16 activation row
//   cq_gemv2_<fmt>_y<f32|f16>[_epi]       decode GEMV, one fp16 row, streaming (K-quants)
//   cq_gemvd_<fmt>_n<1|2|4>_y<f32|f16>   decode GEMV, 2..16 fp16 rows, direct activations (K-quants)
//   cq_gemm_<fmt>_x<f16|f32>_y<f32|f16>   prefill dequant-GEMM (K-quants)
//   cq_gemm2_<fmt>_n<1|2>_m<8|16>_y<f32|f16>  prefill dequant-GEMM, large tiles, fp16 x
//   cq_xsums_f16                          activation sub-block sums for its min term
//   cq_splitk_reduce_y<f32|f16>           sum of its split-K partials
//   cq_dequant_<fmt>                      bit-exact dequantisation
#include "cq_gemv.h"
#include "cq_gemv1.h"
#include "cq_gemv2.h"
#include "cq_gemvd.h"
#include "cq_gemm.h"
#include "cq_gemm2.h"
#include "cq_dequant.h"

#define GEMV_KERNEL(NAME, FMT, XT, YT)                                               \
  extern "C" __global__ void __launch_bounds__(512) NAME(const GemvArgs a) { \
    gemv_body<FMT, XT, YT>(a);                                                       \
  }

#define GEMV_FMT(fname, FMT)                          \
  GEMV_KERNEL(cq_gemv_##fname##_xf16_yf32, FMT, 0, 0) \
  GEMV_KERNEL(cq_gemv_##fname##_xf16_yf16, FMT, 0, 1) \
  GEMV_KERNEL(cq_gemv_##fname##_xf32_yf32, FMT, 1, 0) \
  GEMV_KERNEL(cq_gemv_##fname##_xf32_yf16, FMT, 1, 1)

GEMV_FMT(q4_0, CQ_Q4_0)
GEMV_FMT(q4_1, CQ_Q4_1)
GEMV_FMT(q5_0, CQ_Q5_0)
GEMV_FMT(q5_1, CQ_Q5_1)
GEMV_FMT(q8_0, CQ_Q8_0)
GEMV_FMT(q4_k, CQ_Q4_K)
GEMV_FMT(q5_k, CQ_Q5_K)
GEMV_FMT(q6_k, CQ_Q6_K)

#define DEQUANT_KERNEL(fname, FMT)                                                  \
  extern "C" __global__ void __launch_bounds__(256) cq_dequant_##fname(const DequantArgs a) { \
    const long long c = (long long)blockIdx.x * blockDim.x + threadIdx.x;          \
    if (c < a.chunks) dequant_chunk<FMT>(a.w, a.out, c);                            \
  }

DEQUANT_KERNEL(q4_0, CQ_Q4_0)
DEQUANT_KERNEL(q4_1, CQ_Q4_1)
DEQUANT_KERNEL(q5_0, CQ_Q5_0)
DEQUANT_KERNEL(q5_1, CQ_Q5_1)
DEQUANT_KERNEL(q8_0, CQ_Q8_0)
DEQUANT_KERNEL(q4_k, CQ_Q4_K)
DEQUANT_KERNEL(q5_k, CQ_Q5_K)
DEQUANT_KERNEL(q6_k, CQ_Q6_K)

#define GEMM_KERNEL(NAME, FMT, XT, YT)                                               \
  extern "C" __global__ void __launch_bounds__(512) NAME(const GemmArgs a) {         \
    gemm_body<FMT, XT, YT>(a);                                                       \
  }
#define GEMM_FMT(fname, FMT)                          \
  GEMM_KERNEL(cq_gemm_##fname##_xf16_yf32, FMT, 0, 0) \
  GEMM_KERNEL(cq_gemm_##fname##_xf16_yf16, FMT, 0, 1) \
  GEMM_KERNEL(cq_gemm_##fname##_xf32_yf32, FMT, 1, 0) \
  GEMM_KERNEL(cq_gemm_##fname##_xf32_yf16, FMT, 1, 1)

GEMM_FMT(q4_k, CQ_Q4_K)
GEMM_FMT(q5_k, CQ_Q5_K)
GEMM_FMT(q6_k, CQ_Q6_K)

// MT = 8 tiles use 64-72 KB of LDS, so two 4-wave workgroups fill a compute
// unit when each wave fits 256 registers (two waves per SIMD).  (One 8-wave
// workgroup sharing the activation tile measured the same.)
#define GEMM2_KERNEL_NW(NAME, FMT, YT, NT, MT, NW)                                                        \
  extern "C" __global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(MT == 8 ? 2 : 1))) \
  NAME(const LtArgs a) {                                                                                    \
    gemm2_body<FMT, YT, NT, MT, NW>(a);                                                                     \
  }
#define GEMM2_KERNEL(NAME, FMT, YT, NT, MT) GEMM2_KERNEL_NW(NAME, FMT, YT, NT, MT, 4)
GEMM2_KERNEL(cq_gemm2_q4_k_n1_m8_yf32, CQ_Q4_K, 0, 1, 8)
GEMM2_KERNEL(cq_gemm2_q4_k_n1_m8_yf16, CQ_Q4_K, 1, 1, 8)
GEMM2_KERNEL(cq_gemm2_q4_k_n1_m16_yf32, CQ_Q4_K, 0, 1, 16)
GEMM2_KERNEL(cq_gemm2_q4_k_n1_m16_yf16, CQ_Q4_K, 1, 1, 16)
GEMM2_KERNEL(cq_gemm2_q4_k_n2_m8_yf32, CQ_Q4_K, 0, 2, 8)
GEMM2_KERNEL(cq_gemm2_q4_k_n2_m8_yf16, CQ_Q4_K, 1, 2, 8)
GEMM2_KERNEL(cq_gemm2_q4_k_n2_m16_yf32, CQ_Q4_K, 0, 2, 16)
GEMM2_KERNEL(cq_gemm2_q4_k_n2_m16_yf16, CQ_Q4_K, 1, 2, 16)
GEMM2_KERNEL(cq_gemm2_q5_k_n1_m8_yf32, CQ_Q5_K, 0, 1, 8)
GEMM2_KERNEL(cq_gemm2_q5_k_n1_m8_yf16, CQ_Q5_K, 1, 1, 8)
GEMM2_KERNEL(cq_gemm2_q5_k_n1_m16_yf32, CQ_Q5_K, 0, 1, 16)
GEMM2_KERNEL(cq_gemm2_q5_k_n1_m16_yf16, CQ_Q5_K, 1, 1, 16)
GEMM2_KERNEL(cq_gemm2_q5_k_n2_m8_yf32, CQ_Q5_K, 0, 2, 8)
GEMM2_KERNEL(cq_gemm2_q5_k_n2_m8_yf16, CQ_Q5_K, 1, 2, 8)
GEMM2_KERNEL(cq_gemm2_q5_k_n2_m16_yf32, CQ_Q5_K, 0, 2, 16)
GEMM2_KERNEL(cq_gemm2_q5_k_n2_m16_yf16, CQ_Q5_K, 1, 2, 16)
GEMM2_KERNEL(cq_gemm2_q6_k_n1_m8_yf32, CQ_Q6_K, 0, 1, 8)
GEMM2_KERNEL(cq_gemm2_q6_k_n1_m8_yf16, CQ_Q6_K, 1, 1, 8)
GEMM2_KERNEL(cq_gemm2_q6_k_n1_m16_yf32, CQ_Q6_K, 0, 1, 16)
GEMM2_KERNEL(cq_gemm2_q6_k_n1_m16_yf16, CQ_Q6_K, 1, 1, 16)
GEMM2_KERNEL(cq_gemm2_q6_k_n2_m8_yf32, CQ_Q6_K, 0, 2, 8)
GEMM2_KERNEL(cq_gemm2_q6_k_n2_m8_yf16, CQ_Q6_K, 1, 2, 8)
GEMM2_KERNEL(cq_gemm2_q6_k_n2_m16_yf32, CQ_Q6_K, 0, 2, 16)
GEMM2_KERNEL(cq_gemm2_q6_k_n2_m16_yf16, CQ_Q6_K, 1, 2, 16)
extern "C" __global__ void __launch_bounds__(256) cq_splitk_reduce_yf32(const float* part, void* y, int splits,
                                                                       long long mn, int n, CqEpi epi) {
  splitk_reduce_body<0>(part, y, splits, mn, n, epi);
}
extern "C" __global__ void __launch_bounds__(256) cq_splitk_reduce_yf16(const float* part, void* y, int splits,
                                                                       long long mn, int n, CqEpi epi) {
  splitk_reduce_body<1>(part, y, splits, mn, n, epi);
}
extern "C" __global__ void __launch_bounds__(256) cq_xsums_f16(const _Float16* x, _Float16* xs, int M, int K) {
  xsums_body(x, xs, M, K);
}

#define GEMV1_KERNEL(NAME, FMT, YT, EPI)                                                \
  extern "C" __global__ void __launch_bounds__((64 * gv1_kernel_waves<FMT, EPI>())) NAME(const Gv1Args a) { \
    gemv1_body<FMT, YT, EPI>(a);                                                        \
  }
#define GEMV1_FMT(fname, FMT)                          \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf32, FMT, 0, 0)     \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf16, FMT, 1, 0)     \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf32_epi, FMT, 0, 1) \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf16_epi, FMT, 1, 1) \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf32_gated, FMT, 0, 2) \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf16_gated, FMT, 1, 2)
GEMV1_FMT(q4_k, CQ_Q4_K)
GEMV1_FMT(q5_k, CQ_Q5_K)
GEMV1_FMT(q6_k, CQ_Q6_K)
GEMV1_FMT(q4_0, CQ_Q4_0)
GEMV1_FMT(q4_1, CQ_Q4_1)
GEMV1_FMT(q5_0, CQ_Q5_0)
GEMV1_FMT(q5_1, CQ_Q5_1)
GEMV1_FMT(q8_0, CQ_Q8_0)
// The int8 activation path for Q4_K, Q4_0 and Q8_0, whose default is the
// register path: cheaper to set up, chosen by the host when every wave has
// at most one task (small weights: 4096 x 4096 Q4_0 5.6 against 6.7 us;
// Q5_K and Q6_K measured slower on it).
#define GEMV1_I8_WAVES(FMT) (FMT == CQ_Q4_K ? 8 : 4)
#define GEMV1_I8_KERNEL(NAME, FMT, YT, EPI)                                                          \
  extern "C" __global__ void __launch_bounds__(64 * GEMV1_I8_WAVES(FMT)) NAME(const Gv1Args a) { \
    gemv1_body<FMT, YT, EPI, GEMV1_I8_WAVES(FMT), 0>(a);                                       \
  }
#define GEMV1_I8_FMT(fname, FMT)                                 \
  GEMV1_I8_KERNEL(cq_gemv1_##fname##_yf32_i8, FMT, 0, 0)         \
  GEMV1_I8_KERNEL(cq_gemv1_##fname##_yf16_i8, FMT, 1, 0)         \
  GEMV1_I8_KERNEL(cq_gemv1_##fname##_yf32_epi_i8, FMT, 0, 1)     \
  GEMV1_I8_KERNEL(cq_gemv1_##fname##_yf16_epi_i8, FMT, 1, 1)
GEMV1_I8_FMT(q4_k, CQ_Q4_K)
GEMV1_I8_FMT(q4_0, CQ_Q4_0)
GEMV1_I8_FMT(q8_0, CQ_Q8_0)
// Rows of 65 to 128 units: each row's halves on a wave pair (gemv1k_body).
#define GEMV1K_KERNEL(NAME, FMT, YT, EPI)                                                   \
  extern "C" __global__ void __launch_bounds__(64 * GV1K_WAVES) NAME(const Gv1Args a) { \
    gemv1k_body<FMT, YT, EPI>(a);                                                       \
  }
#define GEMV1K_FMT(fname, FMT)                               \
  GEMV1K_KERNEL(cq_gemv1k_##fname##_yf32, FMT, 0, 0)         \
  GEMV1K_KERNEL(cq_gemv1k_##fname##_yf16, FMT, 1, 0)         \
  GEMV1K_KERNEL(cq_gemv1k_##fname##_yf32_epi, FMT, 0, 1)     \
  GEMV1K_KERNEL(cq_gemv1k_##fname##_yf16_epi, FMT, 1, 1)
GEMV1K_FMT(q4_k, CQ_Q4_K)
GEMV1K_FMT(q5_k, CQ_Q5_K)
GEMV1K_FMT(q6_k, CQ_Q6_K)
GEMV1K_FMT(q4_0, CQ_Q4_0)

#ifndef CQ_GV2_DEPTH
#define CQ_GV2_DEPTH 3
#endif
#define GV2_WAVES 8
#define GEMV2_KERNEL(NAME, FMT, YT, EPI)                                                        \
  extern "C" __global__ void __launch_bounds__(64 * GV2_WAVES) NAME(const Gv2Args a) {          \
    gemv2_body<FMT, YT, GV2_WAVES, CQ_GV2_DEPTH, EPI>(a);                                       \
  }
#define GEMV2_FMT(fname, FMT)                          \
  GEMV2_KERNEL(cq_gemv2_##fname##_yf32, FMT, 0, 0)     \
  GEMV2_KERNEL(cq_gemv2_##fname##_yf16, FMT, 1, 0)     \
  GEMV2_KERNEL(cq_gemv2_##fname##_yf32_epi, FMT, 0, 1) \
  GEMV2_KERNEL(cq_gemv2_##fname##_yf16_epi, FMT, 1, 1)
GEMV2_FMT(q4_k, CQ_Q4_K)
GEMV2_FMT(q5_k, CQ_Q5_K)
GEMV2_FMT(q6_k, CQ_Q6_K)

#ifndef CQ_GVD_DEPTH
#define CQ_GVD_DEPTH 2
#endif
#define GEMVD_KERNEL(NAME, FMT, YT, NT)                                                  \
  extern "C" __global__ void __launch_bounds__(64 * GVD_MAX_WAVES) NAME(const GvdArgs a) { \
    gemvd_body<FMT, YT, NT, CQ_GVD_DEPTH>(a);                                            \
  }
#define GEMVD_FMT(fname, FMT)                          \
  GEMVD_KERNEL(cq_gemvd_##fname##_n1_yf32, FMT, 0, 1) \
  GEMVD_KERNEL(cq_gemvd_##fname##_n1_yf16, FMT, 1, 1) \
  GEMVD_KERNEL(cq_gemvd_##fname##_n2_yf32, FMT, 0, 2) \
  GEMVD_KERNEL(cq_gemvd_##fname##_n2_yf16, FMT, 1, 2) \
  GEMVD_KERNEL(cq_gemvd_##fname##_n4_yf32, FMT, 0, 4) \
  GEMVD_KERNEL(cq_gemvd_##fname##_n4_yf16, FMT, 1, 4)
GEMVD_FMT(q4_k, CQ_Q4_K)
GEMVD_FMT(q5_k, CQ_Q5_K)
GEMVD_FMT(q6_k, CQ_Q6_K)

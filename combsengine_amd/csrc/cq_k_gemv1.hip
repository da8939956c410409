// Kernels of the library, compiled with hipcc --genco into one gfx950 code
// object of four (cq_k_*.hip); the host library embeds all four and looks
// each kernel up by its extern "C" name with hipModuleGetFunction.
// This object: the single-row decode GEMVs cq_gemv1_* (fp16-register and
// int8 paths, gated gate/up) and cq_gemv1k_* (rows of 65-128 units).
#include "cq_gemv1.h"
#include "cq_gemvr.h"

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
// Several weights of one format and K against one activation row (the
// projections that share an input, e.g. q / k / v), fp16-register path.
#define GEMV1_MULTI_FMT(fname, FMT)                     \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf32_multi, FMT, 0, 3) \
  GEMV1_KERNEL(cq_gemv1_##fname##_yf16_multi, FMT, 1, 3)
GEMV1_MULTI_FMT(q4_k, CQ_Q4_K)
GEMV1_MULTI_FMT(q5_k, CQ_Q5_K)
GEMV1_MULTI_FMT(q6_k, CQ_Q6_K)
GEMV1_MULTI_FMT(q4_0, CQ_Q4_0)
GEMV1_MULTI_FMT(q8_0, CQ_Q8_0)
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


// Single-row decode with rows split across a wave's lanes (cq_gemvr.h):
// [y dtype] x [activation pieces per thread 1, 2, 4, 8]; four rows of loads
// in flight per wave (eight measured slower at every shape tried).
#define GEMVR_KERNEL(NAME, YT, XR)                                                               \
  extern "C" __global__ void __launch_bounds__(64 * GVR_MAXW) NAME(const GvrArgs a) {            \
    gvr_q4k_body<YT, XR, 4>(a);                                                                  \
  }
#define GEMVR_Y(YN, YT)                              \
  GEMVR_KERNEL(cq_gemvr_q4_k_##YN##_x1, YT, 1)       \
  GEMVR_KERNEL(cq_gemvr_q4_k_##YN##_x2, YT, 2)       \
  GEMVR_KERNEL(cq_gemvr_q4_k_##YN##_x4, YT, 4)       \
  GEMVR_KERNEL(cq_gemvr_q4_k_##YN##_x8, YT, 8)
GEMVR_Y(yf32, 0)
GEMVR_Y(yf16, 1)

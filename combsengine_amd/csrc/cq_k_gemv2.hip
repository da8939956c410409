// Kernels of the library, compiled with hipcc --genco into one gfx950 code
// object of four (cq_k_*.hip); the host library embeds all four and looks
// each kernel up by its extern "C" name with hipModuleGetFunction.
// This object: the streaming quarter-superblock single-row GEMV cq_gemv2_*
// (K-quants) and the batched decode GEMV with activations loaded once per
// workgroup cq_gemvq_* (K-quants, K <= 4096).
#include "cq_gemv2.h"
#include "cq_gemvq.h"

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


// Batched decode, K <= 4096: activations loaded once per workgroup, weight
// columns streamed per wave (cq_gemvq.h).
#define GEMVQ_KERNEL(NAME, FMT, YT, MODE, MSUM, EPI) \
  extern "C" __global__ void __launch_bounds__(64 * GVQ_MAX_WAVES) NAME(const GvqArgs a) { gemvq_body<FMT, YT, MODE, MSUM, EPI>(a); }
// one weight (plain, and with the bias / gated epilogue), several weights
// (segments), the gated gate / up pair
#define GEMVQ_FMT(fname, FMT)                                              \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf32, FMT, 0, 0, false, false)           \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf16, FMT, 1, 0, false, false)           \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf32_epi, FMT, 0, 0, false, true)        \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf16_epi, FMT, 1, 0, false, true)        \
  GEMVQ_KERNEL(cq_gemvq_##fname##_multi_yf32, FMT, 0, 1, false, false)     \
  GEMVQ_KERNEL(cq_gemvq_##fname##_multi_yf16, FMT, 1, 1, false, false)     \
  GEMVQ_KERNEL(cq_gemvq_##fname##_gated_yf32, FMT, 0, 2, false, false)     \
  GEMVQ_KERNEL(cq_gemvq_##fname##_gated_yf16, FMT, 1, 2, false, false)
// Q4_K / Q5_K: the same with the min term against the column's sub-block sums
#define GEMVQ_FMT_MS(fname, FMT)                                           \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf32_ms, FMT, 0, 0, true, false)         \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf16_ms, FMT, 1, 0, true, false)         \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf32_ms_epi, FMT, 0, 0, true, true)      \
  GEMVQ_KERNEL(cq_gemvq_##fname##_yf16_ms_epi, FMT, 1, 0, true, true)      \
  GEMVQ_KERNEL(cq_gemvq_##fname##_multi_yf32_ms, FMT, 0, 1, true, false)   \
  GEMVQ_KERNEL(cq_gemvq_##fname##_multi_yf16_ms, FMT, 1, 1, true, false)   \
  GEMVQ_KERNEL(cq_gemvq_##fname##_gated_yf32_ms, FMT, 0, 2, true, false)   \
  GEMVQ_KERNEL(cq_gemvq_##fname##_gated_yf16_ms, FMT, 1, 2, true, false)
GEMVQ_FMT(q4_k, CQ_Q4_K)
GEMVQ_FMT(q5_k, CQ_Q5_K)
GEMVQ_FMT(q6_k, CQ_Q6_K)
GEMVQ_FMT(q4_0, CQ_Q4_0)
GEMVQ_FMT(q5_0, CQ_Q5_0)
GEMVQ_FMT(q8_0, CQ_Q8_0)
GEMVQ_FMT(q4_1, CQ_Q4_1)
GEMVQ_FMT(q5_1, CQ_Q5_1)
GEMVQ_FMT_MS(q4_k, CQ_Q4_K)
GEMVQ_FMT_MS(q5_k, CQ_Q5_K)

// Kernels of the library, compiled with hipcc --genco into one gfx950 code
// object of four (cq_k_*.hip); the host library embeds all four and looks
// each kernel up by its extern "C" name with hipModuleGetFunction.
// This object: the 16-row MFMA decode GEMV (cq_gemv_*), the batched
// direct-activation decode GEMV (cq_gemvd_*) and the bit-exact dequant
// kernels (cq_dequant_*).
#include "cq_gemv.h"
#include "cq_gemvd.h"
#include "cq_gemvs.h"
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


// Batched decode with the activations shared through LDS and the K range
// split over workgroups (cq_gemvs.h).
#define GEMVS_KERNEL(NAME, FMT, YT) \
  extern "C" __global__ void __launch_bounds__(64 * GVS_WAVES) NAME(const GvsArgs a) { gemvs_body<FMT, YT>(a); }
GEMVS_KERNEL(cq_gemvs_q4_k_yf32, CQ_Q4_K, 0)
GEMVS_KERNEL(cq_gemvs_q4_k_yf16, CQ_Q4_K, 1)
GEMVS_KERNEL(cq_gemvs_q5_k_yf32, CQ_Q5_K, 0)
GEMVS_KERNEL(cq_gemvs_q5_k_yf16, CQ_Q5_K, 1)
GEMVS_KERNEL(cq_gemvs_q6_k_yf32, CQ_Q6_K, 0)
GEMVS_KERNEL(cq_gemvs_q6_k_yf16, CQ_Q6_K, 1)

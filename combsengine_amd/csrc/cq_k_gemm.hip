// Kernels of the library, compiled with hipcc --genco into one gfx950 code
// object of four (cq_k_*.hip); the host library embeds all four and looks
// each kernel up by its extern "C" name with hipModuleGetFunction.
// This object: the prefill dequant-GEMMs (cq_gemm_*, cq_gemm2_*, cq_gemml_*), the
// activation sub-block sums of their min term (cq_xsums_f16) and the split-K
// reduction (cq_splitk_reduce_*).
#include "cq_gemm.h"
#include "cq_gemm2.h"
#include "cq_gemml.h"

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
  extern "C" __global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) \
  NAME(const LtArgs a) {                                                                                    \
    gemm2_body<FMT, YT, NT, MT, NW>(a);                                                                     \
  }
#define GEMM2_KERNEL(NAME, FMT, YT, NT, MT) GEMM2_KERNEL_NW(NAME, FMT, YT, NT, MT, (MT == 16 ? 8 : 4))
// MT = 4 (64 activation rows, one weight tile per wave): 110 registers and
// 36 KB of LDS, so four 4-wave workgroups share a compute unit (four waves
// per SIMD) to hide the weight and activation latency of short prefills.
#define GEMM2_KERNEL_M4(NAME, FMT, YT)                                                             \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) \
  NAME(const LtArgs a) {                                                                       \
    gemm2_body<FMT, YT, 1, 4, 4>(a);                                                           \
  }
GEMM2_KERNEL_M4(cq_gemm2_q4_k_n1_m4_yf32, CQ_Q4_K, 0)
GEMM2_KERNEL_M4(cq_gemm2_q4_k_n1_m4_yf16, CQ_Q4_K, 1)
GEMM2_KERNEL_M4(cq_gemm2_q5_k_n1_m4_yf32, CQ_Q5_K, 0)
GEMM2_KERNEL_M4(cq_gemm2_q5_k_n1_m4_yf16, CQ_Q5_K, 1)
GEMM2_KERNEL_M4(cq_gemm2_q6_k_n1_m4_yf32, CQ_Q6_K, 0)
GEMM2_KERNEL_M4(cq_gemm2_q6_k_n1_m4_yf16, CQ_Q6_K, 1)
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

// fp32 activations as two fp16 row blocks: xh[i] = hi = fp16(x[i]) and
// xh[mk + i] = lo = fp16(x[i] - hi) (the hi + lo pair the fp32-x kernels
// also use); four values per thread.
extern "C" __global__ void __launch_bounds__(256) cq_split_f32(const float* x, _Float16* xh, long long mk) {
  const long long i0 = 4 * ((long long)blockIdx.x * blockDim.x + threadIdx.x);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const long long i = i0 + e;
    if (i < mk) {
      const float v = x[i];
      const _Float16 hi = (_Float16)v;
      xh[i] = hi;
      xh[mk + i] = (_Float16)(v - (float)hi);
    }
  }
}

// Prefill dequant-GEMM for the 32-value block formats (cq_gemml.h):
// [format] x [NT 1, 2] x [y dtype]; two workgroups per compute unit.
#define GEMML_KERNEL(NAME, FMT, YT, NT)                                                                     \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) NAME(const LgArgs a) { \
    gemml_body<FMT, YT, NT, 4>(a);                                                                         \
  }
#define GEMML_FMT(fname, FMT)                          \
  GEMML_KERNEL(cq_gemml_##fname##_n1_yf32, FMT, 0, 1)  \
  GEMML_KERNEL(cq_gemml_##fname##_n1_yf16, FMT, 1, 1)  \
  GEMML_KERNEL(cq_gemml_##fname##_n2_yf32, FMT, 0, 2)  \
  GEMML_KERNEL(cq_gemml_##fname##_n2_yf16, FMT, 1, 2)
// 64 activation rows (MT = 4), one weight tile per wave: four workgroups per
// compute unit for short prefills
#define GEMML_KERNEL_M4(NAME, FMT, YT)                                                             \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) \
  NAME(const LgArgs a) {                                                                       \
    gemml_body<FMT, YT, 1, 4, 4>(a);                                                           \
  }
#define GEMML_FMT_M4(fname, FMT)                          \
  GEMML_KERNEL_M4(cq_gemml_##fname##_n1_m4_yf32, FMT, 0) \
  GEMML_KERNEL_M4(cq_gemml_##fname##_n1_m4_yf16, FMT, 1)
GEMML_FMT_M4(q4_0, CQ_Q4_0)
GEMML_FMT_M4(q5_0, CQ_Q5_0)
GEMML_FMT_M4(q8_0, CQ_Q8_0)
GEMML_FMT_M4(q4_1, CQ_Q4_1)
GEMML_FMT_M4(q5_1, CQ_Q5_1)
GEMML_FMT(q4_0, CQ_Q4_0)
GEMML_FMT(q5_0, CQ_Q5_0)
GEMML_FMT(q8_0, CQ_Q8_0)
GEMML_FMT(q4_1, CQ_Q4_1)
GEMML_FMT(q5_1, CQ_Q5_1)

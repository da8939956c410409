// Device helpers shared by the gfx950 GGUF dequant-matmul kernels.
//
// GGUF blocks are stored unchanged in HBM (18/22/34/144/176/210-byte blocks),
// so most fields are only 2-byte aligned.  All weight loads go through
// __builtin_memcpy, which the gfx950 backend lowers to single unaligned
// global_load_dword{,x2,x4} instructions (unaligned access mode is on for
// amdhsa), never to byte loads.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "cq_epi.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// GGML type ids, as in the GGUF file format.
enum : int {
  CQ_Q4_0 = 2, CQ_Q4_1 = 3, CQ_Q5_0 = 6, CQ_Q5_1 = 7, CQ_Q8_0 = 8, CQ_Q4_K = 12, CQ_Q5_K = 13, CQ_Q6_K = 14
};

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  uint16_t v;
  __builtin_memcpy(&v, p, 2);
  return v;
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
__device__ __forceinline__ u2v ld_u64(const uint8_t* p) {
  u2v v;
  __builtin_memcpy(&v, p, 8);
  return v;
}
__device__ __forceinline__ u4v ld_u128(const uint8_t* p) {
  u4v v;
  __builtin_memcpy(&v, p, 16);
  return v;
}

// IEEE binary16 bits -> f32 (exact conversion).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// (mask & a) | (~mask & b)  (v_bfi_b32)
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (mask & a) | (~mask & b); }
// rotate right (v_alignbit_b32)
__device__ __forceinline__ uint32_t rotr(uint32_t v, uint32_t s) { return __builtin_amdgcn_alignbit(v, v, s); }

// A lane's float from another lane of its 16-lane row, by a DPP modifier on
// a VALU move (no LDS round trip, unlike __shfl_xor's ds_bpermute, whose
// latency a reduction chain pays once per step).  CTRL: 0xB1 lane ^ 1,
// 0x4E lane ^ 2 (quad permutes), 0x141 the mirror within each 8 lanes, 0x140
// the mirror within the 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over each aligned group of G lanes (G a power of two, 1..64, uniform);
// every lane of a group gets the same value: within 16 lanes by DPP (pairs,
// then quads, then the mirrors, which pair each lane with one of the other
// half's, all of whose lanes hold that half's sum), across rows by shuffles.
__device__ __forceinline__ float lane_group_sum(float v, int G) {
  if (G >= 2) v += dpp_f32<0xB1>(v);
  if (G >= 4) v += dpp_f32<0x4E>(v);
  if (G >= 8) v += dpp_f32<0x141>(v);
  if (G >= 16) v += dpp_f32<0x140>(v);
  if (G >= 32) v += __shfl_xor(v, 16, 64);
  if (G >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 hsplat(float v) {
  _Float16 h = (_Float16)v;
  return h2{h, h};
}
// Single-rounding packed fp16 a*b+c (v_pk_fma_f16).  The unpack tricks below
// rely on it: (1024+q)*s - 1024*s is an exact small integer in fp16.
__device__ __forceinline__ uint32_t pk_fma(uint32_t v, h2 s, h2 c) {
  return as_u32(__builtin_elementwise_fma(as_h2(v), s, c));
}
__device__ __forceinline__ h8 mk_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4v v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}

// D[16x16] += A[16x32] * B[32x16], fp16 in, fp32 accumulate.
// Lane l supplies A row (l&15), B column (l&15), both at k-group (l>>4);
// it receives D rows 4*(l>>4)+r, column (l&15), r = 0..3.
__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// One lane's view of the activations staged in LDS as fp16: row m = (lane & 15)
// of the current activation tile, for the K chunk starting at c0.  Lanes whose
// row is beyond M read nothing and contribute zeros.
// XT = 0: fp16 x as is.  XT = 1: fp32 x was split at staging time into
// hi = fp16(x) and lo = fp16(x - hi), so the MFMA sees ~22 significant bits.
template <int XT>
struct XRow {
  const _Float16* hi;
  const _Float16* lo;
  // Lanes whose activation row is beyond M read row 0 instead: MFMA output
  // row i depends only on A row i, and rows >= M are never stored, so no
  // lane needs a branch or a zero fill.
  __device__ XRow(const _Float16* hi_base, const _Float16* lo_base, int row, int stride, int c0, bool on)
      : hi(hi_base + (on ? row : 0) * stride - c0), lo(lo_base + (on ? row : 0) * stride - c0) {}
};

template <int XT>
struct A8 {
  h8 hi;
  h8 lo;
};

// 8 consecutive activations starting at element k.
template <int XT>
__device__ __forceinline__ A8<XT> load_a8(const XRow<XT>& xr, int k) {
  A8<XT> a;
  a.hi = *(const h8*)(xr.hi + k);
  a.lo = XT ? *(const h8*)(xr.lo + k) : a.hi;
  return a;
}

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// 4 activations at k0 followed by 4 at k1.
template <int XT>
__device__ __forceinline__ A8<XT> load_a4x2(const XRow<XT>& xr, int k0, int k1) {
  A8<XT> a;
  const h4 p = *(const h4*)(xr.hi + k0), q = *(const h4*)(xr.hi + k1);
  a.hi = __builtin_shufflevector(p, q, 0, 1, 2, 3, 4, 5, 6, 7);
  if (XT) {
    const h4 pl = *(const h4*)(xr.lo + k0), ql = *(const h4*)(xr.lo + k1);
    a.lo = __builtin_shufflevector(pl, ql, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    a.lo = a.hi;
  }
  return a;
}

template <int XT>
__device__ __forceinline__ f4 mfma_x(const A8<XT>& a, h8 b, f4 c) {
  c = mfma(a.hi, b, c);
  if (XT) c = mfma(a.lo, b, c);
  return c;
}

// get_scale_min_k4 for sub-block j (0..7) from the 12 packed scale bytes held
// in three little-endian words s0 (bytes 0-3), s1 (4-7), s2 (8-11).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t& sc, uint32_t& mn) {
  const int sh = 8 * (j & 3);
  const uint32_t b0 = (s0 >> sh) & 0xFF, b1 = (s1 >> sh) & 0xFF, b2 = (s2 >> sh) & 0xFF;
  if (j < 4) {
    sc = b0 & 63;
    mn = b1 & 63;
  } else {
    sc = (b2 & 0x0F) | ((b0 >> 6) << 4);
    mn = (b2 >> 4) | ((b1 >> 6) << 4);
  }
}

// ---------------------------------------------------------------------------
// Output epilogue (CqEpi): v = acc (+ bias[n]); with aux, v = act(v) * aux[i].
// SiLU is v * sigmoid(v) (burn's silu); the tanh GELU is
// 0.5 v (1 + tanh(u)), u = sqrt(2/pi) (v + 0.044715 v^3), evaluated through
// the identity 0.5 (1 + tanh(u)) = sigmoid(2u); the exact GELU is
// 0.5 v (1 + erf(v / sqrt(2))).
__device__ __forceinline__ float cq_sigmoid(float z) { return 1.0f / (1.0f + __expf(-z)); }
__device__ __forceinline__ float cq_act(float v, int act) {
  if (act == CQ_EPI_ACT_SILU) return v * cq_sigmoid(v);
  if (act == CQ_EPI_ACT_GELU_TANH) {
    const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return v * cq_sigmoid(2.0f * u);
  }
  return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
}
// A projection's output in y's dtype: the reference's fp16 model casts each
// op's fp32 result to fp16 before the bias add or the gated product
// (qlinear.rs:84-98, 126-143; llama.rs:301-303), so with fp16 y the
// epilogues round the accumulator first.
template <int YT>
__device__ __forceinline__ float cq_round_y(float v) {
  return YT ? (float)(_Float16)v : v;
}
// idx: flat index of the output element [m][n]; n: its column.
template <int YT>
__device__ __forceinline__ float cq_epilogue(const CqEpi& e, float v, size_t idx, int n) {
  if (!e.bias && !e.aux) return v;
  v = cq_round_y<YT>(v);
  if (e.bias) v += e.bias_f16 ? (float)((const _Float16*)e.bias)[n] : ((const float*)e.bias)[n];
  if (e.aux) {
    const float u = e.aux_f16 ? (float)((const _Float16*)e.aux)[idx] : ((const float*)e.aux)[idx];
    v = cq_act(v, e.act) * u;
  }
  return v;
}
// Epilogue from values loaded beforehand (b = bias[n], u = aux[idx]; unused
// parts are ignored).  Streaming kernels load them ahead of their weight
// stream: a load at store time would make the in-order load counter wait for
// every weight load still in flight.
template <int YT>
__device__ __forceinline__ float cq_epi_apply(const CqEpi& e, float v, float b, float u) {
  if (!e.bias && !e.aux) return v;
  v = cq_round_y<YT>(v);
  if (e.bias) v += b;
  if (e.aux) v = cq_act(v, e.act) * u;
  return v;
}
// The epilogue with the activation fixed at compile time (ACT < 0: bias
// only): kernels that store many outputs per thread pick the activation
// once, instead of carrying every activation's code at every store.
template <int ACT>
__device__ __forceinline__ float cq_act_t(float v) {
  if constexpr (ACT == CQ_EPI_ACT_SILU) return v * cq_sigmoid(v);
  else if constexpr (ACT == CQ_EPI_ACT_GELU_TANH) return v * cq_sigmoid(2.0f * 0.7978845608028654f * (v + 0.044715f * v * v * v));
  else return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
}
template <int YT, int ACT>
__device__ __forceinline__ float cq_epi_apply_t(const CqEpi& e, float v, float b, float u) {
  v = cq_round_y<YT>(v);
  if (e.bias) v += b;
  if constexpr (ACT >= 0) v = cq_act_t<ACT>(v) * u;
  return v;
}
// The one-launch gated product act(g) * u of two fp32 projections, each
// first rounded to y's dtype.
template <int YT>
__device__ __forceinline__ float cq_gated(float g, float u, int act) {
  return cq_act(cq_round_y<YT>(g), act) * cq_round_y<YT>(u);
}
__device__ __forceinline__ float cq_epi_bias(const CqEpi& e, int n) {
  if (!e.bias) return 0.0f;
  return e.bias_f16 ? (float)((const _Float16*)e.bias)[n] : ((const float*)e.bias)[n];
}
__device__ __forceinline__ float cq_epi_aux(const CqEpi& e, size_t idx) {
  if (!e.aux) return 0.0f;
  return e.aux_f16 ? (float)((const _Float16*)e.aux)[idx] : ((const float*)e.aux)[idx];
}
template <int YT>
__device__ __forceinline__ void cq_store_raw(void* y, float v, size_t idx) {
  if (YT) ((_Float16*)y)[idx] = (_Float16)v;
  else ((float*)y)[idx] = v;
}
// Stores one output element through the epilogue.
template <int YT>
__device__ __forceinline__ void cq_store(void* y, const CqEpi& e, float v, size_t idx, int n) {
  v = cq_epilogue<YT>(e, v, idx, n);
  if (YT) ((_Float16*)y)[idx] = (_Float16)v;
  else ((float*)y)[idx] = v;
}
// Stores a thread's NT x MT MFMA output tiles (row m0 + 16 tm + 4 g + r,
// column n0 + 16 t + j; value scale[t] * acc[t][tm][r]) through the bias /
// gated epilogue, for kernels with many outputs per thread.  The activation
// is chosen once, and every bias and aux value is loaded before the first
// store: loads and stores share the in-order vmcnt counter, so loads
// interleaved with stores (or behind a per-value dtype branch, whose join
// waits) turn the store tail into a chain of memory round trips.  aux must
// have y's dtype (the gated product's aux is y itself); returns false,
// storing nothing, when it does not.
template <int YT, int NT, int MT>
__device__ __forceinline__ bool cq_store_tiles_epi(const CqEpi& e, void* y, int M, int N, int m0, int n0, int g,
                                                   int j, const f4 (&acc)[NT][MT], const float (&scale)[NT]) {
  if (e.aux && e.aux_f16 != YT) return false;
  auto run = [&](auto actc) {
    constexpr int ACT = decltype(actc)::value;
    float bv[NT], uv[NT][MT][4];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int nc = min(n0 + 16 * t + j, N - 1);
      bv[t] = cq_epi_bias(e, nc);
#pragma unroll
      for (int tm = 0; tm < MT; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const size_t idx = (size_t)min(m0 + 16 * tm + 4 * g + r, M - 1) * N + nc;
          uv[t][tm][r] = ACT < 0 ? 0.0f : YT ? (float)((const _Float16*)e.aux)[idx] : ((const float*)e.aux)[idx];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the stores
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int tm = 0; tm < MT; tm++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + 16 * tm + 4 * g + r, n = n0 + 16 * t + j;
          if (m < M && n < N)
            cq_store_raw<YT>(y, cq_epi_apply_t<YT, ACT>(e, scale[t] * acc[t][tm][r], bv[t], uv[t][tm][r]),
                             (size_t)m * N + n);
        }
  };
  if (!e.aux) run(std::integral_constant<int, -1>{});
  else if (e.act == CQ_EPI_ACT_SILU) run(std::integral_constant<int, CQ_EPI_ACT_SILU>{});
  else if (e.act == CQ_EPI_ACT_GELU_TANH) run(std::integral_constant<int, CQ_EPI_ACT_GELU_TANH>{});
  else run(std::integral_constant<int, CQ_EPI_ACT_GELU>{});
  return true;
}

// Device helpers shared by the gfx950 GGUF dequant-matmul kernels.
//
// GGUF blocks are stored unchanged in HBM (18/22/34/144/176/210-byte blocks),
// so most fields are only 2-byte aligned.  All weight loads go through
// __builtin_memcpy, which the gfx950 backend lowers to single unaligned
// global_load_dword{,x2,x4} instructions (unaligned access mode is on for
// amdhsa), never to byte loads.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

// GGML type ids, as in the GGUF file format.
enum : int { CQ_Q4_0 = 2, CQ_Q5_0 = 6, CQ_Q8_0 = 8, CQ_Q4_K = 12, CQ_Q5_K = 13, CQ_Q6_K = 14 };

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

// One lane's slice of the activation matrix: row m of x (fp16 or fp32).
// Lanes whose row is beyond M contribute zeros and touch no memory.
// XT = 0: fp16 x used as is.  XT = 1: fp32 x split into hi + lo fp16 parts
// (hi = fp16(x), lo = fp16(x - hi)), so the MFMA sees ~22 significant bits.
template <int XT>
struct XRow {
  const uint8_t* base;
  bool on;
  __device__ XRow(const void* x, int m, int M, int K) {
    on = m < M;
    base = (const uint8_t*)x + (size_t)(on ? m : 0) * K * (XT ? 4 : 2);
  }
};

template <int XT>
struct A8 {
  h8 hi;
  h8 lo;
};

template <int XT>
__device__ __forceinline__ void cvt_split(const float* f, A8<XT>& a) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    _Float16 h = (_Float16)f[i];
    a.hi[i] = h;
    if (XT) a.lo[i] = (_Float16)(f[i] - (float)h);
  }
}

// 8 consecutive activations starting at element k.
template <int XT>
__device__ __forceinline__ A8<XT> load_a8(const XRow<XT>& xr, int k) {
  A8<XT> a;
  if (!XT) {
    u4v v = xr.on ? ld_u128(xr.base + (size_t)k * 2) : u4v{0, 0, 0, 0};
    a.hi = __builtin_bit_cast(h8, v);
    a.lo = a.hi;
  } else {
    float f[8];
    if (xr.on) {
      u4v v0 = ld_u128(xr.base + (size_t)k * 4), v1 = ld_u128(xr.base + (size_t)k * 4 + 16);
      __builtin_memcpy(f, &v0, 16);
      __builtin_memcpy(f + 4, &v1, 16);
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) f[i] = 0.0f;
    }
    cvt_split<XT>(f, a);
  }
  return a;
}

// 4 activations at k0 followed by 4 at k1.
template <int XT>
__device__ __forceinline__ A8<XT> load_a4x2(const XRow<XT>& xr, int k0, int k1) {
  A8<XT> a;
  if (!XT) {
    u2v p = xr.on ? ld_u64(xr.base + (size_t)k0 * 2) : u2v{0, 0};
    u2v q = xr.on ? ld_u64(xr.base + (size_t)k1 * 2) : u2v{0, 0};
    u4v v = {p.x, p.y, q.x, q.y};
    a.hi = __builtin_bit_cast(h8, v);
    a.lo = a.hi;
  } else {
    float f[8];
    if (xr.on) {
      u4v v0 = ld_u128(xr.base + (size_t)k0 * 4), v1 = ld_u128(xr.base + (size_t)k1 * 4);
      __builtin_memcpy(f, &v0, 16);
      __builtin_memcpy(f + 4, &v1, 16);
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) f[i] = 0.0f;
    }
    cvt_split<XT>(f, a);
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

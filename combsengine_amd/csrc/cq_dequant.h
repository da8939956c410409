// Bit-exact GPU dequantisers (the validation path).  GPU twins of the
// reference's scalar dequantizers, gguf.rs:755-999, and of its dequant-only
// CubeCL kernels (qmatmul.rs:70-84, 361-382, 427-436, 850-875, 1032-1059,
// 1155-1179).  Every f32 product and difference is rounded separately, in the
// reference's order; contraction into FMA is switched off here.
#pragma once
#include "cq_common.h"

struct DequantArgs {
  const uint8_t* w;
  float* out;
  long long chunks;  // 32-value chunks
};

// One thread per 32-value chunk: a legacy block, or sub-block c%8 of
// K-quant superblock c/8.
template <int FMT>
__device__ __forceinline__ void dequant_chunk(const uint8_t* __restrict__ w, float* __restrict__ out, long long c) {
#pragma clang fp contract(off)
  float v[32];
  if constexpr (FMT == CQ_Q4_0) {  // gguf.rs:755-774
    const uint8_t* b = w + c * 18;
    const float d = f16_bits_to_f32(ld_u16(b));
    for (int j = 0; j < 16; j++) {
      const uint32_t byte = b[2 + j];
      v[j] = (float)((int)(byte & 0x0F) - 8) * d;
      v[j + 16] = (float)((int)(byte >> 4) - 8) * d;
    }
  } else if constexpr (FMT == CQ_Q5_0) {  // gguf.rs:825-847
    const uint8_t* b = w + c * 22;
    const float d = f16_bits_to_f32(ld_u16(b));
    const uint32_t qh = ld_u32(b + 2);
    for (int j = 0; j < 16; j++) {
      const uint32_t byte = b[6 + j];
      const int lo = (int)((byte & 0x0F) | (((qh >> j) & 1u) << 4)) - 16;
      const int hi = (int)((byte >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16;
      v[j] = (float)lo * d;
      v[j + 16] = (float)hi * d;
    }
  } else if constexpr (FMT == CQ_Q4_1) {  // gguf.rs:798-820: q * d + m
    const uint8_t* b = w + c * 20;
    const float d = f16_bits_to_f32(ld_u16(b)), m = f16_bits_to_f32(ld_u16(b + 2));
    for (int j = 0; j < 16; j++) {
      const uint32_t byte = b[4 + j];
      v[j] = (float)(byte & 0x0F) * d + m;
      v[j + 16] = (float)(byte >> 4) * d + m;
    }
  } else if constexpr (FMT == CQ_Q5_1) {  // gguf.rs:851-874: 5-bit q * d + m
    const uint8_t* b = w + c * 24;
    const float d = f16_bits_to_f32(ld_u16(b)), m = f16_bits_to_f32(ld_u16(b + 2));
    const uint32_t qh = ld_u32(b + 4);
    for (int j = 0; j < 16; j++) {
      const uint32_t byte = b[8 + j];
      const uint32_t lo = (byte & 0x0F) | (((qh >> j) & 1u) << 4);
      const uint32_t hi = (byte >> 4) | (((qh >> (j + 16)) & 1u) << 4);
      v[j] = (float)lo * d + m;
      v[j + 16] = (float)hi * d + m;
    }
  } else if constexpr (FMT == CQ_Q8_0) {  // gguf.rs:779-794
    const uint8_t* b = w + c * 34;
    const float d = f16_bits_to_f32(ld_u16(b));
    for (int j = 0; j < 32; j++) v[j] = (float)(int8_t)b[2 + j] * d;
  } else if constexpr (FMT == CQ_Q4_K || FMT == CQ_Q5_K) {  // gguf.rs:894-961
    const int bb = FMT == CQ_Q4_K ? 144 : 176;
    const uint8_t* sb = w + (c >> 3) * bb;
    const int q = (int)(c & 7), j = q >> 1, t = q & 1;
    const float d = f16_bits_to_f32(ld_u16(sb)), dmin = f16_bits_to_f32(ld_u16(sb + 2));
    uint32_t sc, mn;
    scale_min_k4(2 * j + t, ld_u32(sb + 4), ld_u32(sb + 8), ld_u32(sb + 12), sc, mn);
    const float d1 = d * (float)sc, fmin = dmin * (float)mn;
    const uint8_t* qs = sb + (FMT == CQ_Q4_K ? 16 : 48) + 32 * j;
    for (int l = 0; l < 32; l++) {
      uint32_t n = t ? (qs[l] >> 4) : (qs[l] & 0x0F);
      if (FMT == CQ_Q5_K) n |= ((sb[16 + l] >> (2 * j + t)) & 1u) << 4;
      v[l] = d1 * (float)n - fmin;
    }
  } else {  // Q6_K, gguf.rs:968-999: chunk = (half, quadrant)
    const uint8_t* sb = w + (c >> 3) * 210;
    const int q = (int)(c & 7), hh = q >> 2, t = q & 3;
    const float d = f16_bits_to_f32(ld_u16(sb + 208));
    for (int l = 0; l < 32; l++) {
      const uint32_t qlb = sb[64 * hh + 32 * (t & 1) + l];
      const uint32_t nib = t >= 2 ? (qlb >> 4) : (qlb & 0x0F);
      const uint32_t hb = (sb[128 + 32 * hh + l] >> (2 * t)) & 3u;
      const int qv = (int)(nib | (hb << 4)) - 32;
      const int scv = (int)(int8_t)sb[192 + 8 * hh + l / 16 + 2 * t];
      v[l] = d * (float)scv * (float)qv;
    }
  }
  float4* o = (float4*)(out + c * 32);
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

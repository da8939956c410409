// Host GGUF quantisers behind cq_quantize() (include/combs_qlinear.h).
//
// asqrzk/CombsEngine only reads GGUF files; it ships no quantiser (its
// scalar dequantisers are engine/core/combs-formats/src/gguf.rs:755-999).
// Inputs for the benchmarks and tests are therefore produced with a
// restatement of the published ggml reference quantisers
// (ggml-quants.c quantize_row_{q4_0,q5_0,q8_0,q4_K,q5_K,q6_K}_ref and their
// helpers make_qx_quants / make_qkx2_quants, llama.cpp, MIT licence; the
// library itself is not part of the reference tree or this image).  The
// packed byte layouts they emit are the ones the dequantisers read.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

#include "../../include/combs_qlinear.h"

namespace {

// IEEE f32 -> binary16, round to nearest even (what ggml's
// GGML_FP32_TO_FP16 and half::f16::from_f32 do).
uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7FFFFFFFu;
  if (absx >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0));
  if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520: inf
  if (absx < 0x38800000u) {  // below the smallest normal half: subnormal or zero
    if (absx < 0x33000000u) return (uint16_t)sign;  // < 2^-25 rounds to 0
    const int e = (int)(absx >> 23);
    uint32_t man = (absx & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - e;  // man >> shift gives units of 2^-24
    uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = ((absx >> 13) - (112u << 10));
  const uint32_t rem = absx & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void put_f16(uint8_t* p, float v) {
  const uint16_t h = f32_to_f16(v);
  p[0] = (uint8_t)(h & 0xFF);
  p[1] = (uint8_t)(h >> 8);
}

// Round to nearest, ties to even (ggml nearest_int's magic-number trick is
// exactly this for |v| < 2^22).
inline int nearest_int(float v) { return (int)std::nearbyint(v); }

const float kGroupMaxEps = 1e-15f;

// ---- 32-value formats ------------------------------------------------------

void quant_q8_0(const float* x, uint8_t* y) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
  const float d = amax / 127.0f;
  const float id = d ? 1.0f / d : 0.0f;
  put_f16(y, d);
  for (int j = 0; j < 32; j++) y[2 + j] = (uint8_t)(int8_t)std::round(x[j] * id);
}

void quant_q4_0(const float* x, uint8_t* y) {
  float amax = 0.0f, mx = 0.0f;
  for (int j = 0; j < 32; j++)
    if (amax < std::fabs(x[j])) {
      amax = std::fabs(x[j]);
      mx = x[j];
    }
  const float d = mx / -8.0f;
  const float id = d ? 1.0f / d : 0.0f;
  put_f16(y, d);
  for (int j = 0; j < 16; j++) {
    const int a = std::min(15, (int)(int8_t)(x[j] * id + 8.5f));
    const int b = std::min(15, (int)(int8_t)(x[16 + j] * id + 8.5f));
    y[2 + j] = (uint8_t)(a | (b << 4));
  }
}

void quant_q5_0(const float* x, uint8_t* y) {
  float amax = 0.0f, mx = 0.0f;
  for (int j = 0; j < 32; j++)
    if (amax < std::fabs(x[j])) {
      amax = std::fabs(x[j]);
      mx = x[j];
    }
  const float d = mx / -16.0f;
  const float id = d ? 1.0f / d : 0.0f;
  put_f16(y, d);
  uint32_t qh = 0;
  for (int j = 0; j < 16; j++) {
    const int a = std::min(31, (int)(int8_t)(x[j] * id + 16.5f));
    const int b = std::min(31, (int)(int8_t)(x[16 + j] * id + 16.5f));
    y[6 + j] = (uint8_t)((a & 0x0F) | ((b & 0x0F) << 4));
    qh |= ((uint32_t)(a & 0x10) >> 4) << j;
    qh |= ((uint32_t)(b & 0x10) >> 4) << (j + 16);
  }
  memcpy(y + 2, &qh, 4);
}

// Asymmetric 32-value blocks (ggml quantize_row_q4_1_ref / q5_1_ref):
// d = (max - min) / (2^bits - 1), m = min, q = round((x - min) / d).
void quant_q4_1(const float* x, uint8_t* y) {
  float mn = x[0], mx = x[0];
  for (int j = 1; j < 32; j++) {
    mn = std::min(mn, x[j]);
    mx = std::max(mx, x[j]);
  }
  const float d = (mx - mn) / 15.0f;
  const float id = d ? 1.0f / d : 0.0f;
  put_f16(y, d);
  put_f16(y + 2, mn);
  for (int j = 0; j < 16; j++) {
    const int a = std::min(15, (int)(int8_t)((x[j] - mn) * id + 0.5f));
    const int b = std::min(15, (int)(int8_t)((x[16 + j] - mn) * id + 0.5f));
    y[4 + j] = (uint8_t)(a | (b << 4));
  }
}

void quant_q5_1(const float* x, uint8_t* y) {
  float mn = x[0], mx = x[0];
  for (int j = 1; j < 32; j++) {
    mn = std::min(mn, x[j]);
    mx = std::max(mx, x[j]);
  }
  const float d = (mx - mn) / 31.0f;
  const float id = d ? 1.0f / d : 0.0f;
  put_f16(y, d);
  put_f16(y + 2, mn);
  uint32_t qh = 0;
  for (int j = 0; j < 16; j++) {
    const uint32_t a = (uint8_t)((x[j] - mn) * id + 0.5f);
    const uint32_t b = (uint8_t)((x[16 + j] - mn) * id + 0.5f);
    y[8 + j] = (uint8_t)((a & 0x0F) | ((b & 0x0F) << 4));
    qh |= ((a & 0x10) >> 4) << j;
    qh |= ((b & 0x10) >> 4) << (j + 16);
  }
  memcpy(y + 4, &qh, 4);
}

// ---- K-quant helpers -------------------------------------------------------

// Weighted asymmetric fit of n values to [0, nmax] (ggml make_qkx2_quants).
float make_qkx2_quants(int n, int nmax, const float* x, const float* w, uint8_t* L, float* the_min, uint8_t* Laux,
                       float rmin, float rdelta, int nstep) {
  float mn = x[0], mx = x[0], sum_w = w[0], sum_x = sum_w * x[0];
  for (int i = 1; i < n; i++) {
    mn = std::min(mn, x[i]);
    mx = std::max(mx, x[i]);
    sum_w += w[i];
    sum_x += w[i] * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    for (int i = 0; i < n; i++) L[i] = 0;
    *the_min = -mn;
    return 0.0f;
  }
  float iscale = nmax / (mx - mn);
  float scale = 1.0f / iscale;
  float best_error = 0;
  for (int i = 0; i < n; i++) {
    const int l = std::max(0, std::min(nmax, nearest_int(iscale * (x[i] - mn))));
    L[i] = (uint8_t)l;
    const float diff = scale * l + mn - x[i];
    best_error += w[i] * diff * diff;
  }
  if (nstep < 1) {
    *the_min = -mn;
    return scale;
  }
  for (int is = 0; is <= nstep; is++) {
    iscale = (rmin + rdelta * is + nmax) / (mx - mn);
    float sum_l = 0, sum_l2 = 0, sum_xl = 0;
    for (int i = 0; i < n; i++) {
      const int l = std::max(0, std::min(nmax, nearest_int(iscale * (x[i] - mn))));
      Laux[i] = (uint8_t)l;
      sum_l += w[i] * l;
      sum_l2 += w[i] * l * l;
      sum_xl += w[i] * l * x[i];
    }
    const float D = sum_w * sum_l2 - sum_l * sum_l;
    if (D > 0) {
      float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
      float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
      if (this_min > 0) {
        this_min = 0;
        this_scale = sum_xl / sum_l2;
      }
      float cur_error = 0;
      for (int i = 0; i < n; i++) {
        const float diff = this_scale * Laux[i] + this_min - x[i];
        cur_error += w[i] * diff * diff;
      }
      if (cur_error < best_error) {
        for (int i = 0; i < n; i++) L[i] = Laux[i];
        best_error = cur_error;
        scale = this_scale;
        mn = this_min;
      }
    }
  }
  *the_min = -mn;
  return scale;
}

// Symmetric fit to [-nmax, nmax-1] with x^2 weights (ggml make_qx_quants,
// rmse_type 1).  L receives l + nmax.
float make_qx_quants(int n, int nmax, const float* x, int8_t* L) {
  float mx = 0, amax = 0;
  for (int i = 0; i < n; i++) {
    const float ax = std::fabs(x[i]);
    if (ax > amax) {
      amax = ax;
      mx = x[i];
    }
  }
  if (amax < kGroupMaxEps) {
    for (int i = 0; i < n; i++) L[i] = 0;
    return 0.0f;
  }
  float iscale = -nmax / mx;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; i++) {
    const int l = std::max(-nmax, std::min(nmax - 1, nearest_int(iscale * x[i])));
    L[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; is++) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / mx;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; i++) {
      const int l = std::max(-nmax, std::min(nmax - 1, nearest_int(iscale * x[i])));
      const float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; i++) {
        const int l = std::max(-nmax, std::min(nmax - 1, nearest_int(iscale * x[i])));
        L[i] = (int8_t)(nmax + l);
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
  }
}

// Shared by Q4_K (nmax 15) and Q5_K (nmax 31): 8 sub-blocks of 32, 6-bit
// scales and mins packed as ggml does; L receives the final quants.
void quant_kq_scales(const float* x, int nmax, float rmin, int nstep, uint8_t* y, uint8_t* L) {
  float mins[8], scales[8], weights[32];
  uint8_t Laux[32];
  float max_scale = 0, max_min = 0;
  for (int j = 0; j < 8; j++) {
    float sum_x2 = 0;
    for (int l = 0; l < 32; l++) sum_x2 += x[32 * j + l] * x[32 * j + l];
    const float av_x = std::sqrt(sum_x2 / 32);
    for (int l = 0; l < 32; l++) weights[l] = av_x + std::fabs(x[32 * j + l]);
    scales[j] = make_qkx2_quants(32, nmax, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, rmin, 0.1f, nstep);
    max_scale = std::max(max_scale, scales[j]);
    max_min = std::max(max_min, mins[j]);
  }
  const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
  const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
  uint8_t* sc = y + 4;
  memset(sc, 0, 12);
  for (int j = 0; j < 8; j++) {
    const uint8_t ls = (uint8_t)std::min(63, nearest_int(inv_scale * scales[j]));
    const uint8_t lm = (uint8_t)std::min(63, nearest_int(inv_min * mins[j]));
    if (j < 4) {
      sc[j] = ls;
      sc[j + 4] = lm;
    } else {
      sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
      sc[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  put_f16(y, max_scale / 63.f);
  put_f16(y + 2, max_min / 63.f);
  const float dd = f16_to_f32((uint16_t)(y[0] | (y[1] << 8)));
  const float dm = f16_to_f32((uint16_t)(y[2] | (y[3] << 8)));
  for (int j = 0; j < 8; j++) {
    uint8_t s, m;
    get_scale_min_k4(j, sc, &s, &m);
    const float d = dd * s;
    if (!d) continue;
    const float dmv = dm * m;
    for (int ii = 0; ii < 32; ii++) {
      const int l = nearest_int((x[32 * j + ii] + dmv) / d);
      L[32 * j + ii] = (uint8_t)std::max(0, std::min(nmax, l));
    }
  }
}

void quant_q4_k(const float* x, uint8_t* y) {
  uint8_t L[256];
  quant_kq_scales(x, 15, -1.0f, 20, y, L);
  uint8_t* q = y + 16;
  for (int j = 0; j < 256; j += 64) {
    for (int l = 0; l < 32; l++) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    q += 32;
  }
}

void quant_q5_k(const float* x, uint8_t* y) {
  uint8_t L[256];
  quant_kq_scales(x, 31, -0.5f, 15, y, L);
  uint8_t* qh = y + 16;
  uint8_t* ql = y + 48;
  memset(qh, 0, 32);
  uint8_t m1 = 1, m2 = 2;
  for (int n = 0; n < 256; n += 64) {
    for (int j = 0; j < 32; j++) {
      int l1 = L[n + j];
      if (l1 > 15) {
        l1 -= 16;
        qh[j] |= m1;
      }
      int l2 = L[n + j + 32];
      if (l2 > 15) {
        l2 -= 16;
        qh[j] |= m2;
      }
      ql[j] = (uint8_t)(l1 | (l2 << 4));
    }
    m1 <<= 2;
    m2 <<= 2;
    ql += 32;
  }
}

void quant_q6_k(const float* x, uint8_t* y) {
  int8_t L[256];
  float scales[16];
  float max_scale = 0, max_abs_scale = 0;
  for (int ib = 0; ib < 16; ib++) {
    const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
    scales[ib] = scale;
    const float abs_scale = std::fabs(scale);
    if (abs_scale > max_abs_scale) {
      max_abs_scale = abs_scale;
      max_scale = scale;
    }
  }
  uint8_t* ql = y;
  uint8_t* qh = y + 128;
  int8_t* sc = (int8_t*)(y + 192);
  if (max_abs_scale < kGroupMaxEps) {
    memset(y, 0, 210);
    return;
  }
  const float iscale = -128.f / max_scale;
  put_f16(y + 208, 1.0f / iscale);
  for (int ib = 0; ib < 16; ib++) sc[ib] = (int8_t)std::min(127, nearest_int(iscale * scales[ib]));
  const float dd = f16_to_f32((uint16_t)(y[208] | (y[209] << 8)));
  for (int j = 0; j < 16; j++) {
    const float d = dd * sc[j];
    if (!d) continue;
    for (int ii = 0; ii < 16; ii++) {
      const int l = std::max(-32, std::min(31, nearest_int(x[16 * j + ii] / d)));
      L[16 * j + ii] = (int8_t)(l + 32);
    }
  }
  for (int j = 0; j < 256; j += 128) {
    for (int l = 0; l < 32; l++) {
      const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
      const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
      ql[l] = (uint8_t)(q1 | (q3 << 4));
      ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
      qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                        ((L[j + l + 96] >> 4) << 6));
    }
    ql += 64;
    qh += 32;
  }
}

}  // namespace

extern "C" cq_status cq_quantize(int format, const float* src, int64_t rows, int64_t k, void* dst, size_t dst_bytes,
                                 int threads) {
  size_t need = 0;
  cq_status st = cq_tensor_bytes(format, rows, k, &need);
  if (st != CQ_OK) return st;
  if (!src || !dst) return CQ_ERR_NULL;
  if (dst_bytes < need) return CQ_ERR_BAD_SHAPE;
  const int qk = cq_block_values(format), bb = cq_block_bytes(format);
  void (*fn)(const float*, uint8_t*) = nullptr;
  switch (format) {
    case CQ_Q4_0: fn = quant_q4_0; break;
    case CQ_Q5_0: fn = quant_q5_0; break;
    case CQ_Q4_1: fn = quant_q4_1; break;
    case CQ_Q5_1: fn = quant_q5_1; break;
    case CQ_Q8_0: fn = quant_q8_0; break;
    case CQ_Q4_K: fn = quant_q4_k; break;
    case CQ_Q5_K: fn = quant_q5_k; break;
    case CQ_Q6_K: fn = quant_q6_k; break;
    default: return CQ_ERR_BAD_FORMAT;
  }
  const int64_t nblocks = rows * (k / qk);
  uint8_t* out = (uint8_t*)dst;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : omp_get_max_threads())
  for (int64_t b = 0; b < nblocks; b++) fn(src + b * qk, out + b * bb);
  return CQ_OK;
}

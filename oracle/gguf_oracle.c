/*
 * gguf_oracle.c -- CPU restatement of the reference's GGUF dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared
 * against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library (combsengine_amd) never links, loads or
 * falls back to it.
 *
 * Reference: asqrzk/CombsEngine (Rust).  Every function cites the reference
 * file:line it restates.  Paths are relative to the reference repo root:
 *   gguf.rs    = engine/core/combs-formats/src/gguf.rs
 *   qmatmul.rs = engine/core/combs-models/src/qmatmul.rs
 *
 * Build with -ffp-contract=off: Rust never fuses a*b+c into an FMA, so the
 * restated f32 arithmetic must not be contracted either (bit-exact dequant).
 *
 * Pinning (what checks each function beyond re-reading the formula):
 *   orc_f16_to_f32       exhaustive over all 65536 inputs vs numpy float16.
 *   orc_tensor_bytes     reference config sizes (gguf.rs:732-740 table).
 *   orc_dequant Q8_0     reference known answer: d=0.5, q=+-2 -> +-1.0
 *                        (combs-formats/tests/gguf.rs:75-81,113-120).
 *   orc_dequant Q4_0     reference known answers reference_block / all-0x88
 *                        (combs-core/src/quant.rs:81-133) + single-nibble
 *                        position probes.
 *   orc_dequant Q5_0/K-quants   single-field position probes (one field set,
 *                        all others zero, checked against the value index the
 *                        GGUF layout assigns), exhaustive scale_min_k4 against
 *                        an independent bit-field packer, and the closed form
 *                        for constant blocks.
 *   orc_ref_matmul       float64 dot within f32 rounding bounds.
 *   orc_fused_matmul     agrees with orc_ref_matmul(dequant) to the reference
 *                        tolerance 1e-3*max(|e|,1) (qmatmul.rs:1831-1837).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* GGML type ids (the GGUF on-disk enum; gguf.rs GGML_* constants). */
enum {
  ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_Q8_0 = 8,
  ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14
};

/* IEEE binary16 -> binary32, exact (the `half` crate 2.7.1 `to_f32` that the
 * reference calls at gguf.rs:758,782,828,897-898,932-933,971 is exact). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static float rd_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Values per block and bytes per block: gguf.rs:709-748 (tensor_byte_size). */
int orc_block_values(int fmt) {
  switch (fmt) {
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return 0;
  }
}

int orc_block_bytes(int fmt) {
  switch (fmt) {
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    default: return 0;
  }
}

/* gguf.rs:709-748: element count must be a multiple of the block; -1 on error. */
int64_t orc_tensor_bytes(int fmt, int64_t n_elems) {
  int qk = orc_block_values(fmt);
  if (qk == 0 || n_elems < 0 || n_elems % qk != 0) return -1;
  return n_elems / qk * orc_block_bytes(fmt);
}

/* gguf.rs:879-888 (scale_min_k4, ggml get_scale_min_k4). */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* gguf.rs:755-774 */
static void dq_q4_0(const uint8_t *b, float *o) {
  float d = rd_f16(b);
  for (int j = 0; j < 16; j++) {
    uint8_t byte = b[2 + j];
    o[j] = (float)((int)(byte & 0x0F) - 8) * d;
    o[j + 16] = (float)((int)(byte >> 4) - 8) * d;
  }
}

/* gguf.rs:798-820 (Q4_1: value = q*d + m). */
static void dq_q4_1(const uint8_t *b, float *o) {
  float d = rd_f16(b), m = rd_f16(b + 2);
  for (int j = 0; j < 16; j++) {
    uint8_t byte = b[4 + j];
    o[j] = (float)(byte & 0x0F) * d + m;
    o[j + 16] = (float)(byte >> 4) * d + m;
  }
}

/* gguf.rs:825-847 */
static void dq_q5_0(const uint8_t *b, float *o) {
  float d = rd_f16(b);
  uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
  for (int j = 0; j < 16; j++) {
    uint8_t byte = b[6 + j];
    int lo = (int)((byte & 0x0F) | (((qh >> j) & 1u) << 4)) - 16;
    int hi = (int)((byte >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16;
    o[j] = (float)lo * d;
    o[j + 16] = (float)hi * d;
  }
}

/* gguf.rs:851-874 (Q5_1). */
static void dq_q5_1(const uint8_t *b, float *o) {
  float d = rd_f16(b), m = rd_f16(b + 2);
  uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
  for (int j = 0; j < 16; j++) {
    uint8_t byte = b[8 + j];
    uint32_t lo = (byte & 0x0F) | (((qh >> j) & 1u) << 4);
    uint32_t hi = (byte >> 4) | (((qh >> (j + 16)) & 1u) << 4);
    o[j] = (float)lo * d + m;
    o[j + 16] = (float)hi * d + m;
  }
}

/* gguf.rs:779-794 */
static void dq_q8_0(const uint8_t *b, float *o) {
  float d = rd_f16(b);
  for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)b[2 + j] * d;
}

/* gguf.rs:894-925: v = d1*q - fmin with d1 = d*sc, fmin = dmin*m, each rounded. */
static void dq_q4_k(const uint8_t *sb, float *o) {
  float d = rd_f16(sb), dmin = rd_f16(sb + 2);
  const uint8_t *scales = sb + 4, *qs = sb + 16;
  for (int j = 0; j < 4; j++) {
    uint8_t sc1, m1, sc2, m2;
    orc_scale_min_k4(2 * j, scales, &sc1, &m1);
    orc_scale_min_k4(2 * j + 1, scales, &sc2, &m2);
    float d1 = d * (float)sc1, fmin1 = dmin * (float)m1;
    float d2 = d * (float)sc2, fmin2 = dmin * (float)m2;
    for (int l = 0; l < 32; l++) *o++ = d1 * (float)(qs[32 * j + l] & 0x0F) - fmin1;
    for (int l = 0; l < 32; l++) *o++ = d2 * (float)(qs[32 * j + l] >> 4) - fmin2;
  }
}

/* gguf.rs:929-961 */
static void dq_q5_k(const uint8_t *sb, float *o) {
  float d = rd_f16(sb), dmin = rd_f16(sb + 2);
  const uint8_t *scales = sb + 4, *qh = sb + 16, *qs = sb + 48;
  for (int j = 0; j < 4; j++) {
    uint8_t sc1, m1, sc2, m2;
    orc_scale_min_k4(2 * j, scales, &sc1, &m1);
    orc_scale_min_k4(2 * j + 1, scales, &sc2, &m2);
    float d1 = d * (float)sc1, fmin1 = dmin * (float)m1;
    float d2 = d * (float)sc2, fmin2 = dmin * (float)m2;
    for (int l = 0; l < 32; l++) {
      uint32_t lo = qs[32 * j + l] & 0x0F, hi = (qh[l] >> (2 * j)) & 1u;
      *o++ = d1 * (float)(lo | (hi << 4)) - fmin1;
    }
    for (int l = 0; l < 32; l++) {
      uint32_t lo = qs[32 * j + l] >> 4, hi = (qh[l] >> (2 * j + 1)) & 1u;
      *o++ = d2 * (float)(lo | (hi << 4)) - fmin2;
    }
  }
}

/* gguf.rs:968-999: v = (d * sc) * q, left to right. */
static void dq_q6_k(const uint8_t *sb, float *o) {
  float d = rd_f16(sb + 208);
  for (int h = 0; h < 2; h++) {
    const uint8_t *ql = sb + 64 * h, *qh = sb + 128 + 32 * h;
    const int8_t *sc = (const int8_t *)(sb + 192 + 8 * h);
    float *v = o + 128 * h;
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
      int q1 = (int)(int8_t)((ql[l] & 0x0F) | ((qh[l] & 0x03) << 4)) - 32;
      int q2 = (int)(int8_t)((ql[l + 32] & 0x0F) | (((qh[l] & 0x0C) >> 2) << 4)) - 32;
      int q3 = (int)(int8_t)((ql[l] >> 4) | (((qh[l] & 0x30) >> 4) << 4)) - 32;
      int q4 = (int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] & 0xC0) >> 6) << 4)) - 32;
      v[l] = d * (float)sc[is] * (float)q1;
      v[l + 32] = d * (float)sc[is + 2] * (float)q2;
      v[l + 64] = d * (float)sc[is + 4] * (float)q3;
      v[l + 96] = d * (float)sc[is + 6] * (float)q4;
    }
  }
}

/* Dequantise a whole block stream (gguf.rs:755-999 + the size checks each
 * dequantizer does).  Returns 0 on success, -1 on a bad format, -2 when
 * nbytes is not a whole number of blocks or disagrees with n. */
int orc_dequant(int fmt, const uint8_t *data, int64_t nbytes, int64_t n, float *out) {
  int qk = orc_block_values(fmt), bb = orc_block_bytes(fmt);
  if (qk == 0) return -1;
  if (nbytes % bb != 0 || nbytes / bb * qk != n) return -2;
  int64_t nb = nbytes / bb;
  for (int64_t i = 0; i < nb; i++) {
    const uint8_t *b = data + i * bb;
    float *o = out + i * qk;
    switch (fmt) {
      case ORC_Q4_0: dq_q4_0(b, o); break;
      case ORC_Q4_1: dq_q4_1(b, o); break;
      case ORC_Q5_0: dq_q5_0(b, o); break;
      case ORC_Q5_1: dq_q5_1(b, o); break;
      case ORC_Q8_0: dq_q8_0(b, o); break;
      case ORC_Q4_K: dq_q4_k(b, o); break;
      case ORC_Q5_K: dq_q5_k(b, o); break;
      case ORC_Q6_K: dq_q6_k(b, o); break;
    }
  }
  return 0;
}

/* qmatmul.rs:1713-1725 (ref_matmul): out[r,c] = sum_i x[r,i]*w[c,i], f32,
 * ascending i. */
void orc_ref_matmul(const float *x, const float *w, int64_t m, int64_t k, int64_t n, float *out) {
  for (int64_t r = 0; r < m; r++)
    for (int64_t c = 0; c < n; c++) {
      float acc = 0.0f;
      for (int64_t i = 0; i < k; i++) acc += x[r * k + i] * w[c * k + i];
      out[r * n + c] = acc;
    }
}

/* The reference's fused kernels, restated per output element with their own
 * accumulation order:
 *   Q4_0 qmatmul.rs:92-125   block_acc over (lo, hi) pairs, acc += d*block_acc
 *   Q5_0 qmatmul.rs:386-423  same with the 5th bit
 *   Q8_0 qmatmul.rs:440-470  block_acc ascending, acc += d*block_acc
 *   Q4_K qmatmul.rs:881-930  sum-split per sub-block pair
 *   Q5_K qmatmul.rs:1064-1117
 *   Q6_K qmatmul.rs:1184-1229 per 16-value group acc += d*sc*sum
 * Returns 0, or -1 for an unsupported format. */
int orc_fused_matmul(int fmt, const uint8_t *w, const float *x, int64_t m, int64_t n, int64_t k, float *out) {
  int qk = orc_block_values(fmt), bb = orc_block_bytes(fmt);
  if (qk == 0 || fmt == ORC_Q4_1 || fmt == ORC_Q5_1) return -1;
  int64_t bpr = k / qk;
  for (int64_t r = 0; r < m; r++) {
    for (int64_t c = 0; c < n; c++) {
      const float *xr = x + r * k;
      float acc = 0.0f;
      for (int64_t kb = 0; kb < bpr; kb++) {
        const uint8_t *b = w + (c * bpr + kb) * bb;
        const float *xb = xr + kb * qk;
        if (fmt == ORC_Q4_0) {
          float d = rd_f16(b), ba = 0.0f;
          for (int jj = 0; jj < 16; jj++) {
            uint8_t byte = b[2 + jj];
            ba += (float)((int)(byte & 0xF) - 8) * xb[jj];
            ba += (float)((int)(byte >> 4) - 8) * xb[16 + jj];
          }
          acc += d * ba;
        } else if (fmt == ORC_Q5_0) {
          float d = rd_f16(b), ba = 0.0f;
          uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
          for (int jj = 0; jj < 16; jj++) {
            uint8_t byte = b[6 + jj];
            int lo = (int)((byte & 0xF) | (((qh >> jj) & 1u) << 4)) - 16;
            int hi = (int)((byte >> 4) | (((qh >> (jj + 16)) & 1u) << 4)) - 16;
            ba += (float)lo * xb[jj];
            ba += (float)hi * xb[16 + jj];
          }
          acc += d * ba;
        } else if (fmt == ORC_Q8_0) {
          float d = rd_f16(b), ba = 0.0f;
          for (int jj = 0; jj < 32; jj++) ba += (float)(int8_t)b[2 + jj] * xb[jj];
          acc += d * ba;
        } else if (fmt == ORC_Q4_K || fmt == ORC_Q5_K) {
          float d = rd_f16(b), dmin = rd_f16(b + 2);
          const uint8_t *scales = b + 4;
          const uint8_t *qh = b + 16;
          const uint8_t *qs = fmt == ORC_Q4_K ? b + 16 : b + 48;
          for (int j = 0; j < 4; j++) {
            float sl = 0, sh = 0, xl = 0, xh = 0;
            for (int l = 0; l < 32; l++) {
              uint32_t byte = qs[32 * j + l];
              uint32_t lo = byte & 0xF, hi = byte >> 4;
              if (fmt == ORC_Q5_K) {
                lo |= ((qh[l] >> (2 * j)) & 1u) << 4;
                hi |= ((qh[l] >> (2 * j + 1)) & 1u) << 4;
              }
              float x1 = xb[64 * j + l], x2 = xb[64 * j + 32 + l];
              sl += (float)lo * x1;
              sh += (float)hi * x2;
              xl += x1;
              xh += x2;
            }
            uint8_t sc1, m1, sc2, m2;
            orc_scale_min_k4(2 * j, scales, &sc1, &m1);
            orc_scale_min_k4(2 * j + 1, scales, &sc2, &m2);
            acc += d * (float)sc1 * sl - dmin * (float)m1 * xl;
            acc += d * (float)sc2 * sh - dmin * (float)m2 * xh;
          }
        } else { /* Q6_K */
          float dsb = rd_f16(b + 208);
          for (int h = 0; h < 2; h++)
            for (int t = 0; t < 4; t++)
              for (int g = 0; g < 2; g++) {
                float sum = 0.0f;
                for (int l0 = 0; l0 < 16; l0++) {
                  int l = g * 16 + l0;
                  uint32_t qlb = b[64 * h + (t % 2) * 32 + l];
                  uint32_t nib = t >= 2 ? qlb >> 4 : qlb & 0xF;
                  uint32_t hi = (b[128 + 32 * h + l] >> (2 * t)) & 3u;
                  int q = (int)(nib | (hi << 4)) - 32;
                  sum += (float)q * xb[128 * h + 32 * t + l];
                }
                int8_t scale = (int8_t)b[192 + 8 * h + g + 2 * t];
                acc += dsb * (float)scale * sum;
              }
        }
      }
      out[r * n + c] = acc;
    }
  }
  return 0;
}

/* The reference CPU path: dense f32 y = x.W^T over the weight
 * dequantised once at load (llama.rs:81-97 -> matmul.rs:34-49 -> burn-ndarray
 * sgemm).  This is the timed CPU baseline, not a parity oracle: it unrolls the
 * k loop over 8 partial sums for speed.  threads <= 1 runs single-threaded
 * (matrixmultiply 0.3.11 without its threading feature); otherwise OpenMP. */
void orc_dense_gemm(const float *x, const float *w, int64_t m, int64_t n, int64_t k, float *out, int threads) {
#ifdef _OPENMP
  int nt = threads < 1 ? 1 : threads;
#pragma omp parallel for schedule(static) num_threads(nt) collapse(2)
#endif
  for (int64_t r = 0; r < m; r++)
    for (int64_t c = 0; c < n; c++) {
      const float *xr = x + r * k, *wc = w + c * k;
      float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      int64_t i = 0;
      for (; i + 8 <= k; i += 8)
        for (int u = 0; u < 8; u++) p[u] += xr[i + u] * wc[i + u];
      float acc = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      for (; i < k; i++) acc += xr[i] * wc[i];
      out[r * n + c] = acc;
    }
  (void)threads;
}

/* Dequantise-at-load with the same threading control (timed separately). */
int orc_dequant_mt(int fmt, const uint8_t *data, int64_t nbytes, int64_t n, float *out, int threads) {
  int qk = orc_block_values(fmt), bb = orc_block_bytes(fmt);
  if (qk == 0) return -1;
  if (nbytes % bb != 0 || nbytes / bb * qk != n) return -2;
  int64_t nb = nbytes / bb;
  int64_t chunk = 4096;
  int64_t nchunks = (nb + chunk - 1) / chunk;
#ifdef _OPENMP
  int nt = threads < 1 ? 1 : threads;
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
  for (int64_t c = 0; c < nchunks; c++) {
    int64_t b0 = c * chunk, b1 = b0 + chunk < nb ? b0 + chunk : nb;
    orc_dequant(fmt, data + b0 * bb, (b1 - b0) * bb, (b1 - b0) * qk, out + b0 * qk);
  }
  (void)threads;
  return 0;
}

/* ---- Synthetic block streams of the reference's own tests ----------------
 * LCG s = s*1664525 + 1013904223, byte = s>>24 (qmatmul.rs:1698-1710,
 * 1784-1792).  Scales are f16 values passed in by the caller, who computes
 * them with the same f32->f16 rounding the reference uses (half::from_f32,
 * round-to-nearest-even), since that conversion is a library routine the
 * tests pin separately (numpy float16). */
static uint32_t lcg_next(uint32_t *s) {
  *s = *s * 1664525u + 1013904223u;
  return *s >> 24;
}

void orc_lcg_bytes(uint8_t *out, int64_t n, uint32_t seed) {
  uint32_t s = seed;
  for (int64_t i = 0; i < n; i++) out[i] = (uint8_t)lcg_next(&s);
}

/* synth_q4_0 (qmatmul.rs:1698-1710): one running LCG from 0x12345678,
 * f16 scale d_b = f16(0.003*((b%11)+1)) supplied as scale16[b % 11]. */
void orc_synth_q4_0(uint8_t *out, int64_t n_blocks, const uint16_t *scale16_mod11) {
  uint32_t s = 0x12345678u;
  for (int64_t b = 0; b < n_blocks; b++) {
    uint8_t *o = out + b * 18;
    uint16_t h = scale16_mod11[b % 11];
    o[0] = (uint8_t)(h & 0xFF);
    o[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 16; j++) o[2 + j] = (uint8_t)lcg_next(&s);
  }
}

// Decode GEMV over GGUF-packed weights on CDNA4 MFMA:  y[m, n] = sum_k x[m, k] * W[n, k]
// for m <= 16 per launch tile.  Replaces the one-thread-per-output CubeCL
// kernels q{4_0,5_0,8_0,4_k,5_k,6_k}_matmul_kernel
// (engine/core/combs-models/src/qmatmul.rs:92-125, 386-423, 440-470, 881-930,
// 1064-1117, 1184-1229).
//
// Work mapping.  A workgroup owns 16 weight rows and 16 activation rows and
// splits the row's K range across its waves (unit u goes to wave u % nw).
// Inside a wave, lane l owns weight row n0 + (l & 15) and k-group g = l >> 4;
// each unit's packed bytes for that row are read by the 4 lanes of the row
// with 16-byte loads, unpacked in registers to exact small-integer fp16
// values (scale folded in where the product stays exact), and fed to
// v_mfma_f32_16x16x32_f16 against the activations.  Per-block/superblock
// scales (fp16 d, dmin) are applied to the fp32 MFMA result, so no weight is
// ever rounded to fp16.
//
// Unpack trick: a 16-bit word 0x6400 | v is the fp16 number 1024 + v for
// 0 <= v < 1024, so OR-ing nibbles under 0x6400 makes fp16 integers with no
// conversion instruction; one v_pk_fma_f16 then removes the 1024 bias and
// applies an integer scale exactly (single rounding of an exact integer).
#pragma once
#include "cq_common.h"

struct GemvArgs {
  const uint8_t* w;   // packed GGUF blocks, [N rows][row_bytes]
  const void* x;      // [M][K] fp16 or fp32
  void* y;            // [M][N] fp32 or fp16
  long long row_bytes;
  int M, N, K;
  int units;          // work units per row
  int kc;             // K values per LDS chunk of activations (multiple of a unit)
  int lds_stride;     // halves per staged activation row (kc + 8)
  CqEpi epi;
};

// Byte selectors for v_perm_b32(hi, lo, sel): byte i of the result takes
// byte sel_i of {hi:lo}; 0x0c yields 0.
#define SEL_B0_B1 0x0c010c00u   // [lo.b0, 0, lo.b1, 0]
#define SEL_B2_B3 0x0c030c02u   // [lo.b2, 0, lo.b3, 0]
#define SEL_X_B01 0x05010400u   // [lo.b0, hi.b0, lo.b1, hi.b1]
#define SEL_X_B23 0x07030602u   // [lo.b2, hi.b2, lo.b3, hi.b3]
#define SEL_B0_E_B1_E 0x04010400u  // [lo.b0, hi.b0, lo.b1, hi.b0]: hi = C64 puts 0x64 above each byte
#define SEL_B2_E_B3_E 0x04030402u
// fp16 exponent byte of 1024: perm(C64, w, SEL_B*_E_*) turns bytes of w into
// the halves 0x64bb, i.e. fp16 1024 + b, and an AND keeps the wanted bits.
#define C64 0x64646464u

// ---------------------------------------------------------------------------
// Q4_K: 144-byte superblock [d f16][dmin f16][scales 12][qs 128]
// (gguf.rs:894-925).  Lane group g takes qs[32g, 32g+32): its low nibbles are
// sub-block 2g (k = 64g + 0..31), its high nibbles sub-block 2g+1
// (k = 64g + 32..63).  MFMA step s (0..7) covers k = 64g + 8s + 0..7.
// Main MFMA: B = q * sc (<= 15*63, exact).  Min MFMA: B = m (6-bit) so that
// sum_k m(k) x_k = sum_sb m_sb * sum(x in sb).  y += d*Cmain - dmin*Cmin.
struct FragQ4K {
  u4v hdr, q0, q1;
};
__device__ __forceinline__ void load_q4k(FragQ4K& f, const uint8_t* sb, int g) {
  f.hdr = ld_u128(sb);
  f.q0 = ld_u128(sb + 16 + 32 * g);
  f.q1 = ld_u128(sb + 32 + 32 * g);
}
// MFMA B operands of one Q4_K superblock for this lane: b[s] for step s
// (k = 64g + 8s .. +7), the per-lane min operands for the two sub-blocks it
// holds (fp16 pairs), and the superblock scales.
struct DecKQ {
  h8 b[8];
  uint32_t um0, um1;
  float d, dmin;
};
// Per-lane scale constants of a K-quant superblock: the lane's two
// sub-blocks 2g (low nibbles) and 2g+1 (high nibbles, seen as 16*q).
struct KQScale {
  h2 s_lo, c_lo, s_hi, c_hi;
  uint32_t um0, um1;
  float d, dmin;
};
__device__ __forceinline__ KQScale kq_scale(const u4v& hdr, int g) {
  uint32_t sc0, m0, sc1, m1;
  scale_min_k4(2 * g, hdr.y, hdr.z, hdr.w, sc0, m0);
  scale_min_k4(2 * g + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
  KQScale k;
  k.s_lo = hsplat((float)sc0);
  k.c_lo = hsplat(-1024.0f * (float)sc0);
  k.s_hi = hsplat((float)sc1 * 0.0625f);
  k.c_hi = hsplat(-64.0f * (float)sc1);
  k.um0 = as_u32(hsplat((float)m0));
  k.um1 = as_u32(hsplat((float)m1));
  k.d = f16_bits_to_f32(hdr.x);
  k.dmin = f16_bits_to_f32(hdr.x >> 16);
  return k;
}
// B operand of MFMA step s (k = 64g + 8s .. +7) of a Q4_K superblock.
__device__ __forceinline__ h8 q4k_b(const FragQ4K& f, const KQScale& k, int s) {
  const uint32_t w[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  const uint32_t wa = w[2 * (s & 3)], wb = w[2 * (s & 3) + 1];
  const uint32_t pa1 = perm(C64, wa, SEL_B0_E_B1_E), pa2 = perm(C64, wa, SEL_B2_E_B3_E);
  const uint32_t pb1 = perm(C64, wb, SEL_B0_E_B1_E), pb2 = perm(C64, wb, SEL_B2_E_B3_E);
  if (s < 4)
    return mk_h8(pk_fma(pa1 & 0x640F640Fu, k.s_lo, k.c_lo), pk_fma(pa2 & 0x640F640Fu, k.s_lo, k.c_lo),
                 pk_fma(pb1 & 0x640F640Fu, k.s_lo, k.c_lo), pk_fma(pb2 & 0x640F640Fu, k.s_lo, k.c_lo));
  return mk_h8(pk_fma(pa1 & 0x64F064F0u, k.s_hi, k.c_hi), pk_fma(pa2 & 0x64F064F0u, k.s_hi, k.c_hi),
               pk_fma(pb1 & 0x64F064F0u, k.s_hi, k.c_hi), pk_fma(pb2 & 0x64F064F0u, k.s_hi, k.c_hi));
}
__device__ __forceinline__ void kq_finish(const KQScale& k, DecKQ& o) {
  o.um0 = k.um0;
  o.um1 = k.um1;
  o.d = k.d;
  o.dmin = k.dmin;
}
__device__ __forceinline__ void decode_q4k(const FragQ4K& f, int g, DecKQ& o) {
  const KQScale k = kq_scale(f.hdr, g);
#pragma unroll
  for (int s = 0; s < 8; s++) o.b[s] = q4k_b(f, k, s);
  kq_finish(k, o);
}

// GEMV step over a decoded K-quant (Q4_K/Q5_K) superblock.  The min term is
// its own MFMA with B = m(sub-block), so sum_k m(k) x_k = sum_sb m_sb * sum(x in sb).
template <int XT>
__device__ __forceinline__ void gemv_kq(const DecKQ& o, const XRow<XT>& xr, int k0, int g, f4& acc) {
  const h8 bm0 = mk_h8(o.um0, o.um0, o.um0, o.um0), bm1 = mk_h8(o.um1, o.um1, o.um1, o.um1);
  f4 c = {0, 0, 0, 0}, cm = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const A8<XT> a = load_a8<XT>(xr, k0 + 64 * g + 8 * s);
    c = mfma_x<XT>(a, o.b[s], c);
    cm = mfma_x<XT>(a, s < 4 ? bm0 : bm1, cm);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(-o.dmin, cm[r], __builtin_fmaf(o.d, c[r], acc[r]));
}

template <int XT>
__device__ __forceinline__ void compute_q4k(const FragQ4K& f, const XRow<XT>& xr, int k0, int g, f4& acc) {
  DecKQ o;
  decode_q4k(f, g, o);
  gemv_kq<XT>(o, xr, k0, g, acc);
}

// ---------------------------------------------------------------------------
// Q5_K: 176-byte superblock [d][dmin][scales 12][qh 32][qs 128]
// (gguf.rs:929-961).  As Q4_K; the 5th bit of value (pair j, byte l, half t)
// is bit 2j+t of qh[l].  Lane group g is pair j = g.
struct FragQ5K {
  u4v hdr, h0, h1, q0, q1;
};
__device__ __forceinline__ void load_q5k(FragQ5K& f, const uint8_t* sb, int g) {
  f.hdr = ld_u128(sb);
  f.h0 = ld_u128(sb + 16);
  f.h1 = ld_u128(sb + 32);
  f.q0 = ld_u128(sb + 48 + 32 * g);
  f.q1 = ld_u128(sb + 64 + 32 * g);
}
// B operand of MFMA step s of a Q5_K superblock (same k mapping as Q4_K).
__device__ __forceinline__ h8 q5k_b(const FragQ5K& f, const KQScale& k, int g, int s) {
  const uint32_t w[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  const uint32_t hb[8] = {f.h0.x, f.h0.y, f.h0.z, f.h0.w, f.h1.x, f.h1.y, f.h1.z, f.h1.w};
  const int rl = (2 * g - 4) & 31, shh = 2 * g + 1;
  const int i0 = 2 * (s & 3);
  uint32_t u[4];
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const uint32_t wq = w[i0 + e], hq = hb[i0 + e];
    if (s < 4) {
      // rotate bit 2g of each qh byte to bit 4 and insert it above the low nibble
      const uint32_t z = bfi(0x10101010u, rotr(hq, rl), wq);
      u[2 * e] = pk_fma(perm(C64, z, SEL_B0_E_B1_E) & 0x641F641Fu, k.s_lo, k.c_lo);
      u[2 * e + 1] = pk_fma(perm(C64, z, SEL_B2_E_B3_E) & 0x641F641Fu, k.s_lo, k.c_lo);
    } else {
      // high nibble at bits 4-7 of the half, bit 2g+1 of qh at bit 8 under 0x64
      const uint32_t hx = ((hq >> shh) & 0x01010101u) | C64;
      u[2 * e] = pk_fma(perm(hx, wq, SEL_X_B01) & 0x65F065F0u, k.s_hi, k.c_hi);
      u[2 * e + 1] = pk_fma(perm(hx, wq, SEL_X_B23) & 0x65F065F0u, k.s_hi, k.c_hi);
    }
  }
  return mk_h8(u[0], u[1], u[2], u[3]);
}
__device__ __forceinline__ void decode_q5k(const FragQ5K& f, int g, DecKQ& o) {
  const KQScale k = kq_scale(f.hdr, g);
#pragma unroll
  for (int s = 0; s < 8; s++) o.b[s] = q5k_b(f, k, g, s);
  kq_finish(k, o);
}

template <int XT>
__device__ __forceinline__ void compute_q5k(const FragQ5K& f, const XRow<XT>& xr, int k0, int g, f4& acc) {
  DecKQ o;
  decode_q5k(f, g, o);
  gemv_kq<XT>(o, xr, k0, g, acc);
}

// ---------------------------------------------------------------------------
// Q6_K: 210-byte superblock [ql 128][qh 64][scales 16 x i8][d f16]
// (gguf.rs:968-999).  Value (half hh, quadrant t, l) = (ql nibble | 2 qh bits
// << 4) - 32 with scale sc[8hh + l/16 + 2t].  Lane group g = (hh = g>>1,
// s = g&1) owns l in [16s, 16s+16) for all four quadrants of half hh.
// The i8 scale is split sc = 16*sh + sl (sh in [-8,7], sl in [0,15]) so both
// (q-32)*sh and (q-32)*sl are exact in fp16; y += d * (16*Chi + Clo).
struct FragQ6K {
  u4v qa, qb, qh;
  u2v sc;
  uint32_t d;
};
__device__ __forceinline__ void load_q6k(FragQ6K& f, const uint8_t* sb, int g) {
  const int hh = g >> 1, s = g & 1;
  f.qa = ld_u128(sb + 64 * hh + 16 * s);
  f.qb = ld_u128(sb + 64 * hh + 32 + 16 * s);
  f.qh = ld_u128(sb + 128 + 32 * hh + 16 * s);
  f.sc = ld_u64(sb + 192 + 8 * hh);
  f.d = ld_u16(sb + 208);
}
// MFMA B operands of one Q6_K superblock for this lane: for step st = 2t + e
// (k = 128hh + 32t + 16s + 8e .. +7), bh[st] = (q-32)*sh and bl[st] = (q-32)*sl.
struct DecQ6 {
  h8 bh[8], bl[8];
  float d;
};
__device__ __forceinline__ int q6k_koff(int g, int st) {
  return 128 * (g >> 1) + 32 * (st >> 1) + 16 * (g & 1) + 8 * (st & 1);
}
// B operands of MFMA step st = 2t + e of a Q6_K superblock.
__device__ __forceinline__ void q6k_b(const FragQ6K& f, int g, int st, h8& bh, h8& bl) {
  const int s = g & 1, t = st >> 1, e = st & 1;
  const uint32_t qa[4] = {f.qa.x, f.qa.y, f.qa.z, f.qa.w};
  const uint32_t qb[4] = {f.qb.x, f.qb.y, f.qb.z, f.qb.w};
  const uint32_t qh[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
  // scale byte index s + 2t within the 8 scales of this half
  const uint32_t word = (t < 2) ? f.sc.x : f.sc.y;
  const int sc = (int)(int8_t)((word >> (8 * ((s + 2 * t) & 3))) & 0xFF);
  const int shv = sc >> 4, slv = sc & 15;
  h2 sh_s, sh_c, sl_s, sl_c;
  if (t < 2) {  // value = 1024 + q6
    sh_s = hsplat((float)shv); sh_c = hsplat(-1056.0f * (float)shv);
    sl_s = hsplat((float)slv); sl_c = hsplat(-1056.0f * (float)slv);
  } else {      // value = 1024 + 16*q6
    sh_s = hsplat((float)shv * 0.0625f); sh_c = hsplat(-96.0f * (float)shv);
    sl_s = hsplat((float)slv * 0.0625f); sl_c = hsplat(-96.0f * (float)slv);
  }
  const uint32_t* ql = (t & 1) ? qb : qa;
  uint32_t uh[4], ul[4];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t wq = ql[2 * e + i], hq = qh[2 * e + i];
    uint32_t v1, v2;
    if (t < 2) {
      // qh bits 2t,2t+1 -> bits 4,5 of each byte, under the low nibble
      const uint32_t z = bfi(0x30303030u, hq << (4 - 2 * t), wq);
      v1 = perm(C64, z, SEL_B0_E_B1_E) & 0x643F643Fu;
      v2 = perm(C64, z, SEL_B2_E_B3_E) & 0x643F643Fu;
    } else {
      // high nibble at bits 4-7, qh bits 2t,2t+1 at bits 8,9 under 0x64
      const uint32_t hx = ((hq >> (2 * t)) & 0x03030303u) | C64;
      v1 = perm(hx, wq, SEL_X_B01) & 0x67F067F0u;
      v2 = perm(hx, wq, SEL_X_B23) & 0x67F067F0u;
    }
    uh[2 * i] = pk_fma(v1, sh_s, sh_c);
    uh[2 * i + 1] = pk_fma(v2, sh_s, sh_c);
    ul[2 * i] = pk_fma(v1, sl_s, sl_c);
    ul[2 * i + 1] = pk_fma(v2, sl_s, sl_c);
  }
  bh = mk_h8(uh[0], uh[1], uh[2], uh[3]);
  bl = mk_h8(ul[0], ul[1], ul[2], ul[3]);
}
__device__ __forceinline__ void decode_q6k(const FragQ6K& f, int g, DecQ6& o) {
#pragma unroll
  for (int st = 0; st < 8; st++) q6k_b(f, g, st, o.bh[st], o.bl[st]);
  o.d = f16_bits_to_f32(f.d);
}

template <int XT>
__device__ __forceinline__ void compute_q6k(const FragQ6K& f, const XRow<XT>& xr, int k0, int g, f4& acc) {
  DecQ6 o;
  decode_q6k(f, g, o);
  f4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
#pragma unroll
  for (int st = 0; st < 8; st++) {
    const A8<XT> a = load_a8<XT>(xr, k0 + q6k_koff(g, st));
    chi = mfma_x<XT>(a, o.bh[st], chi);
    clo = mfma_x<XT>(a, o.bl[st], clo);
  }
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(o.d, __builtin_fmaf(16.0f, chi[r], clo[r]), acc[r]);
}

// ---------------------------------------------------------------------------
// 32-value legacy blocks.  A unit is LB consecutive blocks of one row; every
// block is one MFMA step with its own fp16 scale, applied to the fp32 result.
#define LB 4

// Q4_0: 18-byte block [d][qs 16] (gguf.rs:755-774).  Lane group g takes
// qs[4g, 4g+4): low nibbles are k = 4g..4g+3, high nibbles k = 16+4g..16+4g+3.
struct FragQ40 {
  uint32_t q[LB], d[LB];
};
__device__ __forceinline__ void load_q40(FragQ40& f, const uint8_t* b, int g, int nb) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int ii = i < nb ? i : 0;
    f.q[i] = ld_u32(b + 18 * ii + 2 + 4 * g);
    f.d[i] = ld_u16(b + 18 * ii);
  }
}
// B operand of block i (values k = 4g..4g+3 from the low nibbles of qs
// bytes 4g..4g+3, then k = 16+4g..16+4g+3 from their high nibbles: the A
// side reads x at the same k, load_a4x2) and the block's fp16 scale.
__device__ __forceinline__ h8 legacy_b(const FragQ40& f, int i, int g) {
  (void)g;
  const h2 one = hsplat(1.0f), c_lo = hsplat(-1032.0f);
  const h2 s16 = hsplat(0.0625f), c_hi = hsplat(-72.0f);
  const uint32_t p1 = perm(C64, f.q[i], SEL_B0_E_B1_E), p2 = perm(C64, f.q[i], SEL_B2_E_B3_E);
  return mk_h8(pk_fma(p1 & 0x640F640Fu, one, c_lo), pk_fma(p2 & 0x640F640Fu, one, c_lo),
               pk_fma(p1 & 0x64F064F0u, s16, c_hi), pk_fma(p2 & 0x64F064F0u, s16, c_hi));
}
__device__ __forceinline__ uint32_t legacy_d(const FragQ40& f, int i) { return f.d[i]; }
template <int XT>
__device__ __forceinline__ void compute_q40(const FragQ40& f, const XRow<XT>& xr, int k0, int g, int nb, f4& acc) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    if (i >= nb) break;
    const h8 b = legacy_b(f, i, g);
    const int kb = k0 + 32 * i;
    const A8<XT> a = load_a4x2<XT>(xr, kb + 4 * g, kb + 16 + 4 * g);
    const f4 c = mfma_x<XT>(a, b, f4{0, 0, 0, 0});
    const float d = f16_bits_to_f32(f.d[i]);
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(d, c[r], acc[r]);
  }
}

// Q5_0: 22-byte block [d][qh u32][qs 16] (gguf.rs:825-847).  Same k mapping
// as Q4_0; value j's 5th bit is qh bit j (low nibbles) or j+16 (high).
struct FragQ50 {
  uint32_t q[LB], h[LB], d[LB];
};
__device__ __forceinline__ void load_q50(FragQ50& f, const uint8_t* b, int g, int nb) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int ii = i < nb ? i : 0;
    f.d[i] = ld_u16(b + 22 * ii);
    f.h[i] = ld_u32(b + 22 * ii + 2);
    f.q[i] = ld_u32(b + 22 * ii + 6 + 4 * g);
  }
}
// bits 0..3 of v -> bit 0 of bytes 0..3 (no carries: all partial products
// land on distinct bit positions).
__device__ __forceinline__ uint32_t spread4(uint32_t v) {
  return ((v & 0xFu) * 0x00204081u) & 0x01010101u;
}
__device__ __forceinline__ h8 legacy_b(const FragQ50& f, int i, int g) {
  const h2 one = hsplat(1.0f), c_lo = hsplat(-1040.0f);
  const h2 s16 = hsplat(0.0625f), c_hi = hsplat(-80.0f);
  const uint32_t q = f.q[i];
  const uint32_t hl = spread4(f.h[i] >> (4 * g));
  const uint32_t hh = spread4(f.h[i] >> (16 + 4 * g));
  const uint32_t z = bfi(0x10101010u, hl << 4, q);
  const uint32_t hx = hh | C64;
  return mk_h8(pk_fma(perm(C64, z, SEL_B0_E_B1_E) & 0x641F641Fu, one, c_lo),
               pk_fma(perm(C64, z, SEL_B2_E_B3_E) & 0x641F641Fu, one, c_lo),
               pk_fma(perm(hx, q, SEL_X_B01) & 0x65F065F0u, s16, c_hi),
               pk_fma(perm(hx, q, SEL_X_B23) & 0x65F065F0u, s16, c_hi));
}
__device__ __forceinline__ uint32_t legacy_d(const FragQ50& f, int i) { return f.d[i]; }
template <int XT>
__device__ __forceinline__ void compute_q50(const FragQ50& f, const XRow<XT>& xr, int k0, int g, int nb, f4& acc) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    if (i >= nb) break;
    const h8 b = legacy_b(f, i, g);
    const int kb = k0 + 32 * i;
    const A8<XT> a = load_a4x2<XT>(xr, kb + 4 * g, kb + 16 + 4 * g);
    const f4 c = mfma_x<XT>(a, b, f4{0, 0, 0, 0});
    const float d = f16_bits_to_f32(f.d[i]);
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(d, c[r], acc[r]);
  }
}

// Q4_1 / Q5_1: the asymmetric twins of Q4_0 / Q5_0, value = q * d + m with
// an fp16 min m per block (gguf.rs:798-820, 851-874): 20-byte block
// [d][m][qs 16], 24-byte block [d][m][qh u32][qs 16].  B = q (0..15 / 0..31,
// exact in fp16); the m term is m * sum(x of the block), the sum taken by one
// more MFMA against B = 1.  The reference serves these formats through its
// dense path only (dequantise, then f32 matmul).
struct FragQ41 {
  uint32_t q[LB], dm[LB];
};
__device__ __forceinline__ void load_q41(FragQ41& f, const uint8_t* b, int g, int nb) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int ii = i < nb ? i : 0;
    f.dm[i] = ld_u32(b + 20 * ii);
    f.q[i] = ld_u32(b + 20 * ii + 4 + 4 * g);
  }
}
struct FragQ51 {
  uint32_t q[LB], h[LB], dm[LB];
};
__device__ __forceinline__ void load_q51(FragQ51& f, const uint8_t* b, int g, int nb) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int ii = i < nb ? i : 0;
    f.dm[i] = ld_u32(b + 24 * ii);
    f.h[i] = ld_u32(b + 24 * ii + 4);
    f.q[i] = ld_u32(b + 24 * ii + 8 + 4 * g);
  }
}
// acc += d * (x . q) + m * sum(x) for one block.
template <int XT>
__device__ __forceinline__ void affine_block(const A8<XT>& a, const h8& b, uint32_t dm, f4& acc) {
  const uint32_t one = 0x3C003C00u;  // fp16 1.0 pair
  const h8 ones = mk_h8(one, one, one, one);
  const f4 c = mfma_x<XT>(a, b, f4{0, 0, 0, 0});
  const f4 s = mfma_x<XT>(a, ones, f4{0, 0, 0, 0});
  const float d = f16_bits_to_f32(dm & 0xFFFFu), m = f16_bits_to_f32(dm >> 16);
#pragma unroll
  for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(d, c[r], __builtin_fmaf(m, s[r], acc[r]));
}
// B = q (no offset) for the affine formats; d and m in one word.
__device__ __forceinline__ h8 legacy_b(const FragQ41& f, int i, int g) {
  (void)g;
  const h2 one = hsplat(1.0f), c_lo = hsplat(-1024.0f);
  const h2 s16 = hsplat(0.0625f), c_hi = hsplat(-64.0f);
  const uint32_t p1 = perm(C64, f.q[i], SEL_B0_E_B1_E), p2 = perm(C64, f.q[i], SEL_B2_E_B3_E);
  return mk_h8(pk_fma(p1 & 0x640F640Fu, one, c_lo), pk_fma(p2 & 0x640F640Fu, one, c_lo),
               pk_fma(p1 & 0x64F064F0u, s16, c_hi), pk_fma(p2 & 0x64F064F0u, s16, c_hi));
}
__device__ __forceinline__ uint32_t legacy_d(const FragQ41& f, int i) { return f.dm[i]; }
__device__ __forceinline__ h8 legacy_b(const FragQ51& f, int i, int g) {
  const h2 one = hsplat(1.0f), c_lo = hsplat(-1024.0f);
  const h2 s16 = hsplat(0.0625f), c_hi = hsplat(-64.0f);
  const uint32_t q = f.q[i];
  const uint32_t hl = spread4(f.h[i] >> (4 * g));
  const uint32_t hh = spread4(f.h[i] >> (16 + 4 * g));
  const uint32_t z = bfi(0x10101010u, hl << 4, q);
  const uint32_t hx = hh | C64;
  return mk_h8(pk_fma(perm(C64, z, SEL_B0_E_B1_E) & 0x641F641Fu, one, c_lo),
               pk_fma(perm(C64, z, SEL_B2_E_B3_E) & 0x641F641Fu, one, c_lo),
               pk_fma(perm(hx, q, SEL_X_B01) & 0x65F065F0u, s16, c_hi),
               pk_fma(perm(hx, q, SEL_X_B23) & 0x65F065F0u, s16, c_hi));
}
__device__ __forceinline__ uint32_t legacy_d(const FragQ51& f, int i) { return f.dm[i]; }
template <int XT>
__device__ __forceinline__ void compute_q41(const FragQ41& f, const XRow<XT>& xr, int k0, int g, int nb, f4& acc) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    if (i >= nb) break;
    const int kb = k0 + 32 * i;
    affine_block<XT>(load_a4x2<XT>(xr, kb + 4 * g, kb + 16 + 4 * g), legacy_b(f, i, g), f.dm[i], acc);
  }
}
template <int XT>
__device__ __forceinline__ void compute_q51(const FragQ51& f, const XRow<XT>& xr, int k0, int g, int nb, f4& acc) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    if (i >= nb) break;
    const int kb = k0 + 32 * i;
    affine_block<XT>(load_a4x2<XT>(xr, kb + 4 * g, kb + 16 + 4 * g), legacy_b(f, i, g), f.dm[i], acc);
  }
}

// Q8_0: 34-byte block [d][qs 32 x i8] (gguf.rs:779-794).  Lane group g takes
// qs[8g, 8g+8) = k 8g..8g+7.  i8 s -> fp16 via (s ^ 0x80) = s + 128 placed
// under a 0x64 high byte: 1024 + s + 128, minus 1152.
struct FragQ80 {
  u2v q[LB];
  uint32_t d[LB];
};
__device__ __forceinline__ void load_q80(FragQ80& f, const uint8_t* b, int g, int nb) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int ii = i < nb ? i : 0;
    f.d[i] = ld_u16(b + 34 * ii);
    f.q[i] = ld_u64(b + 34 * ii + 2 + 8 * g);
  }
}
__device__ __forceinline__ h8 legacy_b(const FragQ80& f, int i, int g) {
  (void)g;
  const h2 one = hsplat(1.0f), cb = hsplat(-1152.0f);
  const uint32_t x0 = f.q[i].x ^ 0x80808080u, x1 = f.q[i].y ^ 0x80808080u;
  return mk_h8(pk_fma(perm(0x64646464u, x0, 0x04010400u), one, cb), pk_fma(perm(0x64646464u, x0, 0x04030402u), one, cb),
               pk_fma(perm(0x64646464u, x1, 0x04010400u), one, cb), pk_fma(perm(0x64646464u, x1, 0x04030402u), one, cb));
}
__device__ __forceinline__ uint32_t legacy_d(const FragQ80& f, int i) { return f.d[i]; }
template <int XT>
__device__ __forceinline__ void compute_q80(const FragQ80& f, const XRow<XT>& xr, int k0, int g, int nb, f4& acc) {
#pragma unroll
  for (int i = 0; i < LB; i++) {
    if (i >= nb) break;
    const h8 b = legacy_b(f, i, g);
    const A8<XT> a = load_a8<XT>(xr, k0 + 32 * i + 8 * g);
    const f4 c = mfma_x<XT>(a, b, f4{0, 0, 0, 0});
    const float d = f16_bits_to_f32(f.d[i]);
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(d, c[r], acc[r]);
  }
}

// ---------------------------------------------------------------------------
template <int FMT> struct FmtTraits;
template <> struct FmtTraits<CQ_Q4_K> { static constexpr int vals = 256, bytes = 144; typedef FragQ4K Frag; };
template <> struct FmtTraits<CQ_Q5_K> { static constexpr int vals = 256, bytes = 176; typedef FragQ5K Frag; };
template <> struct FmtTraits<CQ_Q6_K> { static constexpr int vals = 256, bytes = 210; typedef FragQ6K Frag; };
template <> struct FmtTraits<CQ_Q4_0> { static constexpr int vals = 32 * LB, bytes = 18 * LB; typedef FragQ40 Frag; };
template <> struct FmtTraits<CQ_Q5_0> { static constexpr int vals = 32 * LB, bytes = 22 * LB; typedef FragQ50 Frag; };
template <> struct FmtTraits<CQ_Q4_1> { static constexpr int vals = 32 * LB, bytes = 20 * LB; typedef FragQ41 Frag; };
template <> struct FmtTraits<CQ_Q5_1> { static constexpr int vals = 32 * LB, bytes = 24 * LB; typedef FragQ51 Frag; };
template <> struct FmtTraits<CQ_Q8_0> { static constexpr int vals = 32 * LB, bytes = 34 * LB; typedef FragQ80 Frag; };

template <int FMT>
__device__ __forceinline__ void load_unit(typename FmtTraits<FMT>::Frag& f, const uint8_t* p, int g, int nb) {
  if constexpr (FMT == CQ_Q4_K) load_q4k(f, p, g);
  else if constexpr (FMT == CQ_Q5_K) load_q5k(f, p, g);
  else if constexpr (FMT == CQ_Q6_K) load_q6k(f, p, g);
  else if constexpr (FMT == CQ_Q4_0) load_q40(f, p, g, nb);
  else if constexpr (FMT == CQ_Q5_0) load_q50(f, p, g, nb);
  else if constexpr (FMT == CQ_Q4_1) load_q41(f, p, g, nb);
  else if constexpr (FMT == CQ_Q5_1) load_q51(f, p, g, nb);
  else load_q80(f, p, g, nb);
}

template <int FMT, int XT>
__device__ __forceinline__ void compute_unit(const typename FmtTraits<FMT>::Frag& f, const XRow<XT>& xr, int k0,
                                             int g, int nb, f4& acc) {
  if constexpr (FMT == CQ_Q4_K) compute_q4k<XT>(f, xr, k0, g, acc);
  else if constexpr (FMT == CQ_Q5_K) compute_q5k<XT>(f, xr, k0, g, acc);
  else if constexpr (FMT == CQ_Q6_K) compute_q6k<XT>(f, xr, k0, g, acc);
  else if constexpr (FMT == CQ_Q4_0) compute_q40<XT>(f, xr, k0, g, nb, acc);
  else if constexpr (FMT == CQ_Q5_0) compute_q50<XT>(f, xr, k0, g, nb, acc);
  else if constexpr (FMT == CQ_Q4_1) compute_q41<XT>(f, xr, k0, g, nb, acc);
  else if constexpr (FMT == CQ_Q5_1) compute_q51<XT>(f, xr, k0, g, nb, acc);
  else compute_q80<XT>(f, xr, k0, g, nb, acc);
}

#define CQ_MAX_WAVES 8
#define CQ_DEPTH 4  // units of weight loads a wave keeps in flight

// Activation staging, split in two so the weight loads can be issued in
// between: issue() loads up to XS_REG 8-value vectors per thread into
// registers, commit() converts and stores them to LDS (waiting only for those
// loads, which were issued first), and stage_rest() covers any remainder with
// a plain loop.
#define XS_REG 4

// i / vec for 0 <= i < 16 * vec <= 2^20: the quotient through a float
// reciprocal is exact here ((i + 0.5) / vec is at least 0.5 / vec away from
// an integer, far above the float rounding error), and costs 3 VALU ops
// instead of an integer division sequence.
__device__ __forceinline__ int div_small(int i, float rcp) { return (int)(((float)i + 0.5f) * rcp); }

template <int XT>
struct XStage {
  u4v v[XS_REG][XT ? 2 : 1];
};

template <int XT>
__device__ __forceinline__ void stage_issue(const GemvArgs& a, XStage<XT>& st, int m0, int mt, int c0, int len) {
  const int vec = len >> 3, total = mt * vec;
  const float rcp = 1.0f / (float)vec;
#pragma unroll
  for (int q = 0; q < XS_REG; q++) {
    int i = threadIdx.x + q * blockDim.x;
    i = i < total ? i : total - 1;  // clamp: valid address, store skipped
    const int r = div_small(i, rcp), v = i - r * vec;
    // byte offsets of x fit 31 bits (checked on the host)
    const uint32_t src = (uint32_t)((m0 + r) * a.K + c0 + 8 * v) * (XT ? 4u : 2u);
    if (!XT) {
      st.v[q][0] = ld_u128((const uint8_t*)a.x + src);
    } else {
      st.v[q][0] = ld_u128((const uint8_t*)a.x + src);
      st.v[q][XT] = ld_u128((const uint8_t*)a.x + src + 16);
    }
  }
}

template <int XT>
__device__ __forceinline__ void stage_store(const GemvArgs& a, _Float16* hi, _Float16* lo, int i, int vec,
                                            float rcp, const u4v* src) {
  const int r = div_small(i, rcp), v = i - r * vec;
  _Float16* dh = hi + r * a.lds_stride + 8 * v;
  if (!XT) {
    *(u4v*)dh = src[0];
  } else {
    float f[8];
    __builtin_memcpy(f, &src[0], 16);
    __builtin_memcpy(f + 4, &src[XT], 16);
    h8 vh, vl;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      vh[q] = (_Float16)f[q];
      vl[q] = (_Float16)(f[q] - (float)vh[q]);
    }
    *(h8*)dh = vh;
    *(h8*)(lo + r * a.lds_stride + 8 * v) = vl;
  }
}

template <int XT>
__device__ __forceinline__ void stage_commit(const GemvArgs& a, const XStage<XT>& st, _Float16* hi, _Float16* lo,
                                             int m0, int mt, int c0, int len) {
  const int vec = len >> 3, total = mt * vec;
  const float rcp = 1.0f / (float)vec;
#pragma unroll
  for (int q = 0; q < XS_REG; q++) {
    const int i = threadIdx.x + q * blockDim.x;
    if (i < total) stage_store<XT>(a, hi, lo, i, vec, rcp, st.v[q]);
  }
  for (int i = threadIdx.x + XS_REG * blockDim.x; i < total; i += blockDim.x) {
    const int r = div_small(i, rcp);
    const uint32_t src = (uint32_t)((m0 + r) * a.K + c0 + 8 * (i - r * vec)) * (XT ? 4u : 2u);
    u4v t[2];
    t[0] = ld_u128((const uint8_t*)a.x + src);
    if (XT) t[1] = ld_u128((const uint8_t*)a.x + src + 16);
    stage_store<XT>(a, hi, lo, i, vec, rcp, t);
  }
}

// Grid: x = ceil(N/16) row tiles, y = ceil(M/16) activation tiles.
// Block: 64 * nw threads, nw in 1..8.  Dynamic LDS: (XT ? 2 : 1) * mt *
// lds_stride halves, mt = min(16, M).
template <int FMT, int XT, int YT>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
  typedef FmtTraits<FMT> T;
  typedef typename T::Frag Frag;
  __shared__ float red[CQ_MAX_WAVES][4][64];
  extern __shared__ __attribute__((aligned(16))) _Float16 xs[];
  // wave index is uniform across the wave: keep it (and the unit loop) scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int mt = min(16, a.M - m0);
  const int mrows = min(16, a.M);  // rows allocated in LDS
  _Float16* xhi = xs;
  _Float16* xlo = xs + mrows * a.lds_stride;
  const int row = min(n0 + j, a.N - 1);
  const uint8_t* wr = a.w + (size_t)row * a.row_bytes;
  const int blocks = a.K / 32;
  f4 acc = {0, 0, 0, 0};
  for (int c0 = 0; c0 < a.K; c0 += a.kc) {
    const int len = min(a.kc, a.K - c0);
    const int u_end = (c0 + len + T::vals - 1) / T::vals;
    int ub = c0 / T::vals + wave;
    Frag f[CQ_DEPTH];
    // Issue order matters: vmcnt retires loads in order, so the activation
    // loads go first (the LDS store waits only for them), then one group of
    // weight loads; unit d's compute then waits only for its own loads.
    XStage<XT> st;
    stage_issue<XT>(a, st, m0, mt, c0, len);
#pragma unroll
    for (int d = 0; d < CQ_DEPTH; d++) {
      const int u = min(ub + d * nw, u_end - 1);  // past the end: reload a valid unit, skip its compute
      const int nb = (T::vals == 256) ? 0 : min(LB, blocks - u * LB);
      load_unit<FMT>(f[d], wr + (size_t)u * T::bytes, g, nb);
    }
    if (c0 > 0) __syncthreads();  // previous chunk fully consumed
    stage_commit<XT>(a, st, xhi, xlo, m0, mt, c0, len);
    __syncthreads();
    const XRow<XT> xr(xhi, xlo, j, a.lds_stride, c0, j < mt);
    while (true) {
#pragma unroll
      for (int d = 0; d < CQ_DEPTH; d++) {
        const int u = ub + d * nw;
        if (u < u_end) {
          const int nb = (T::vals == 256) ? 0 : min(LB, blocks - u * LB);
          compute_unit<FMT, XT>(f[d], xr, u * T::vals, g, nb, acc);
        }
      }
      ub += CQ_DEPTH * nw;
      if (ub >= u_end) break;
#pragma unroll
      for (int d = 0; d < CQ_DEPTH; d++) {
        const int u = min(ub + d * nw, u_end - 1);
        const int nb = (T::vals == 256) ? 0 : min(LB, blocks - u * LB);
        load_unit<FMT>(f[d], wr + (size_t)u * T::bytes, g, nb);
      }
    }
  }
  if (nw > 1) {
#pragma unroll
    for (int r = 0; r < 4; r++) red[wave][r][lane] = acc[r];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
      const int r = idx >> 6, ln = idx & 63;
      float s = red[0][r][ln];
      for (int w2 = 1; w2 < nw; w2++) s += red[w2][r][ln];
      const int m = m0 + 4 * (ln >> 4) + r, n = n0 + (ln & 15);
      if (m < a.M && n < a.N) cq_store<YT>(a.y, a.epi, s, (size_t)m * a.N + n, n);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = m0 + 4 * g + r, n = n0 + j;
      if (m < a.M && n < a.N) cq_store<YT>(a.y, a.epi, acc[r], (size_t)m * a.N + n, n);
    }
  }
}

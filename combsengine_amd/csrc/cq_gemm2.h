// Prefill dequant-GEMM, large-tile version for fp16 activations and K-quant
// weights:  y[m, n] = sum_k x[m, k] * W[n, k].
//
// The budget that shapes this kernel: on CDNA4 a VALU instruction and an
// MFMA of the same SIMD largely serialise (a 16x16x32 fp16 MFMA is 16
// cycles, a wave64 VALU op about 4), so the VALU work per MFMA, more than
// the MFMA count, sets the speed.  Everything below minimises it:
//
//   - Workgroup tile: 16*MT activation rows x NW waves x NT 16-row weight
//     tiles (MT = 8: 128 rows, 4 waves, two workgroups per compute unit;
//     MT = 16: 256 rows, 8 waves, one; MT = 4: 64 rows, 4 waves, four, for
//     short prefills).  Each wave decodes only its own NT
//     weight tiles, straight from packed bytes in registers into exact fp16
//     MFMA operands (q*sc, as in the decode GEMV), and reuses every decoded
//     operand for MT MFMAs, one per activation tile.  The packed bytes come
//     by buffer loads whose addresses cost no vector instructions in the K
//     loop (row offsets fixed per lane, the step in the scalar offset).
//   - Steps are half superblocks (128 K values), so two activation chunks
//     (up to 256 rows x 128 halves, 64 KB) double-buffer in LDS.  They arrive
//     by global_load_lds (LDS DMA) one step ahead, XOR-swizzled per row so
//     that each 32-lane half of an A-fragment read hits 32 distinct 16-byte
//     bank groups.
//   - MFMA step s uses one nibble half of the packed bytes for all lanes
//     (s < 2: low nibbles / Q6_K quadrants 0-1; s >= 2: high), so no lane
//     takes a different code path and Q4_K's byte unpacks serve both halves.
//   - Accumulator units: acc holds y / d_u for the current superblock u.  At
//     the superblock's first step acc *= d_{u-1} / d_u and its MFMAs then
//     accumulate straight into acc: one VALU per accumulator register per
//     superblock.  The result is d_last * acc.  A superblock with d = 0
//     keeps the previous units and gets zero main operands.
//   - K-quant min term, -dmin * sum_sb m_sb * sum(x in sb): one MFMA of the
//     activation sub-block sums (computed once per launch by cq_xsums_f16,
//     staged in LDS as fp16 hi + lo of sum/64) against the exact 6-bit mins,
//     folded into acc with one FMA per register.
//   - When the tile grid cannot cover the compute units (few weight rows,
//     long K: the o / down projections), K is split over blockIdx.z; each
//     slice writes fp32 partials and cq_splitk_reduce_* sums them into y.
//   - Q6_K's i8 scale is split sc = 16*sh + sl; the operands (q-32)*sh and
//     (q-32)*sl/16 are both exact in fp16 and share the accumulator, whose
//     units are then 16*d.
//
// The reference ran its Q4_K prefill through qmatmul.rs:939-993 (one thread
// per output, x tile in shared memory) and Q5_K/Q6_K untiled
// (qmatmul.rs:1064-1117, 1184-1229).
#pragma once
#include <type_traits>
#include "cq_gemm.h"

typedef __attribute__((address_space(3))) void lt_lds_t;
typedef __attribute__((address_space(1))) void lt_glb_t;

#define LT_KC 128     // K values per step (half a superblock)
#define LT_MAXMT 16   // activation tiles per workgroup, at most
#define LT_RSRC_FLAGS 0x00020000  // buffer resource word 3: raw (stride 0) dword access

struct LtArgs {
  const uint8_t* w;    // packed superblocks, [N rows][row_bytes]
  const _Float16* x;   // [M][K]
  const _Float16* xs;  // [M][K/256][16]: per superblock the 8 sub-block sums/64, fp16 hi then lo
  void* y;             // [M][N] fp32 or fp16
  float* part;         // split K: [splits][M][N] fp32 partial sums (y unused), else null
  long long row_bytes;
  int M, N, K, units;  // units = K / 256
  int usplit;          // superblocks per K slice (blockIdx.z); units when not split
  CqEpi epi;           // applied here, or by the split-K reduction
};


// 16-byte chunk c (0..15) of a staged row holds K values [8c, 8c+8) of the
// step.  MFMA step s, lane group g reads chunk lt_chunk; within each 32-lane
// half of the wave the chunks differ in one bit only (bit 1 for Q4_K/Q5_K,
// bit 2 for Q6_K).  The row swizzle lt_sw XORs that bit with the row's
// parity and the other three bits with the rest of the row index, so that
// both the 16 lanes of one lane group (16 rows, one 256-byte window of bank
// groups) and the 32 lanes of a half wave (two groups, a 512-byte window)
// hit distinct 16-byte bank groups.
template <int FMT>
__device__ __forceinline__ int lt_chunk(int g, int s) {
  if (FMT == CQ_Q6_K) return 8 * (s >> 1) + 4 * (g & 1) + 2 * (g >> 1) + (s & 1);
  return 8 * (g >> 1) + 4 * (s >> 1) + 2 * (g & 1) + (s & 1);
}
template <int FMT>
__device__ __forceinline__ int lt_sw(int r) {
  const int jj = (r & 15) >> 1, p = r & 1;
  if (FMT == CQ_Q6_K) return (p << 2) | (jj & 3) | ((jj & 4) << 1);
  return (p << 1) | (jj & 1) | ((jj & 6) << 1);
}

// Packed bytes of one half superblock (step) for lane (row j, group g).
struct LtQ4K { u4v hdr, q; };
struct LtQ5K { u4v hdr, qh, q; };
struct LtQ6K { u4v ql, qh; u2v sc; uint32_t d; };
template <int FMT> struct LtFrag;
template <> struct LtFrag<CQ_Q4_K> { typedef LtQ4K T; };
template <> struct LtFrag<CQ_Q5_K> { typedef LtQ5K T; };
template <> struct LtFrag<CQ_Q6_K> { typedef LtQ6K T; };

// Fragment loads through a buffer resource: the workgroup's weight rows
// from a uniform base, the lane's row and lane-group offset in a
// loop-invariant voffset, the step's superblock in soffset and the field's
// position as the immediate offset, so no vector arithmetic is spent on
// addresses inside the K loop.
typedef __amdgpu_buffer_rsrc_t lt_rsrc_t;
__device__ __forceinline__ u4v lt_b128(lt_rsrc_t r, uint32_t v, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, v, so, 0);
}
// Per-lane voffsets of one weight row: vr the row, vq the lane group's
// quant bytes, vh its high-bit (Q5_K) or qh (Q6_K) bytes.
struct LtVo { uint32_t vr, vq, vh; };
template <int FMT>
__device__ __forceinline__ LtVo lt_vo(uint32_t row_off, int g) {
  if (FMT == CQ_Q6_K) return {row_off, row_off + 32 * (g & 1) + 16 * (g >> 1), row_off + 16 * (g >> 1)};
  return {row_off, row_off + 32 * (g >> 1) + 16 * (g & 1), row_off + 16 * (g & 1)};
}
// Q4_K (gguf.rs:894-925): qs pair p = 2h + (g>>1) holds sub-blocks 2p (low
// nibbles) and 2p+1 (high); lane group g takes its bytes [16(g&1), +16).
// The second half (H = 1) uses only the header's scale words: its d / dmin
// word is not loaded (a load into a register that is then dead lets the
// compiler reuse that register, which must first wait for the load).
template <int H>
__device__ __forceinline__ void lt_hdr(u4v& hdr, lt_rsrc_t r, const LtVo& v, uint32_t so) {
  if (H == 0) {
    hdr = lt_b128(r, v.vr, so);
  } else {
    const auto w = __builtin_amdgcn_raw_buffer_load_b96(r, v.vr + 4, so, 0);
    hdr = u4v{0u, w[0], w[1], w[2]};
  }
}
template <int H>
__device__ __forceinline__ void lt_load(LtQ4K& f, lt_rsrc_t r, const LtVo& v, uint32_t so) {
  lt_hdr<H>(f.hdr, r, v, so);
  f.q = lt_b128(r, v.vq + 16 + 64 * H, so);
}
// Q5_K (gguf.rs:929-961): as Q4_K, plus qh bytes [16(g&1), +16), whose bit
// b is the 5th bit of sub-block b.
template <int H>
__device__ __forceinline__ void lt_load(LtQ5K& f, lt_rsrc_t r, const LtVo& v, uint32_t so) {
  lt_hdr<H>(f.hdr, r, v, so);
  f.qh = lt_b128(r, v.vh + 16, so);
  f.q = lt_b128(r, v.vq + 48 + 64 * H, so);
}
// Q6_K (gguf.rs:968-999): half h; step s covers quadrant t = 2(s>>1) + (g&1)
// and l = 16(g>>1) + 8(s&1) + 0..7, so ql bytes [64h + 32(g&1) + 16(g>>1), +16)
// serve both nibble halves and qh bytes [32h + 16(g>>1), +16) all steps.
template <int H>
__device__ __forceinline__ void lt_load(LtQ6K& f, lt_rsrc_t r, const LtVo& v, uint32_t so) {
  f.ql = lt_b128(r, v.vq + 64 * H, so);
  f.qh = lt_b128(r, v.vh + 128 + 32 * H, so);
  f.sc = __builtin_amdgcn_raw_buffer_load_b64(r, v.vr + 192 + 8 * H, so, 0);
  f.d = H == 0 ? __builtin_amdgcn_raw_buffer_load_b16(r, v.vr + 208, so, 0) : 0u;  // d: first half only
}

__device__ __forceinline__ uint32_t u4_at(const u4v& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// get_scale_min_k4 for sub-block jb; jb < 4 iff H == 0, the byte lane-dependent.
template <int H>
__device__ __forceinline__ void lt_scale_min(int jb, const u4v& hd, uint32_t& sc, uint32_t& mn) {
  const uint32_t o = 8 * (jb & 3);
  if (H == 0) {
    sc = __builtin_amdgcn_ubfe(hd.y, o, 6);
    mn = __builtin_amdgcn_ubfe(hd.z, o, 6);
  } else {
    sc = __builtin_amdgcn_ubfe(hd.w, o, 4) | (__builtin_amdgcn_ubfe(hd.y, o + 6, 2) << 4);
    mn = __builtin_amdgcn_ubfe(hd.w, o + 4, 4) | (__builtin_amdgcn_ubfe(hd.z, o + 6, 2) << 4);
  }
}

template <int FMT, int YT, int NT, int MT>
struct LtGemm {
  typedef typename LtFrag<FMT>::T Frag;
  static constexpr bool Q6 = FMT == CQ_Q6_K;
  // MT = 16 runs two waves per SIMD with 128 accumulator registers: it
  // trades a little VALU for registers (Q4_K high-nibble operands decoded
  // again at steps 2, 3 instead of kept; the mins built where they are used;
  // a shorter A-fragment ring).
  static constexpr bool LEAN = MT >= 16;

  f4 acc[NT][MT];
  Frag fr[2][NT];            // packed bytes of the step of half H in fr[H]
  float deff[NT];            // units of acc
  float kk[NT];              // -64 * dmin / deff of the current superblock
  bool live[NT];             // d != 0 for the current superblock
  h2 sa[NT], ca[NT];         // operand scale / offset, steps s < 2
  h2 sb[NT], cb[NT];         // steps s >= 2
  h2 sla[NT], cla[NT], slb[NT], clb[NT];  // Q6_K low-scale operands
  h8 bmin[NT];               // K-quant mins of the superblock (lane groups 0, 1)
  lt_rsrc_t wrs;             // the workgroup's weight rows from its first superblock
  LtVo vo[NT];
  int acol[4];               // byte offset of step s's A chunk in a staged row
  int lane, wave, j, g;

  // the packed bytes of step i (half H = i & 1) into fr[H]
  template <int H>
  __device__ __forceinline__ void load_w(int i) {
    const uint32_t so = (uint32_t)(i >> 1) * FmtTraits<FMT>::bytes;
#pragma unroll
    for (int t = 0; t < NT; t++) lt_load<H>(fr[H][t], wrs, vo[t], so);
  }

  // The superblock's 8 mins as exact fp16 for lane groups 0 and 1 (zero
  // elsewhere), from the header of the second half's fragment.
  __device__ __forceinline__ h8 mins(int t) const {
    const u4v& hd = fr[1][t].hdr;
    const uint32_t m03 = hd.z & 0x3F3F3F3Fu;
    const uint32_t m47 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
    const h2 one = hsplat(1.0f), off = hsplat(-1024.0f);
    uint32_t u[4] = {pk_fma(perm(C64, m03, SEL_B0_E_B1_E), one, off), pk_fma(perm(C64, m03, SEL_B2_E_B3_E), one, off),
                     pk_fma(perm(C64, m47, SEL_B0_E_B1_E), one, off), pk_fma(perm(C64, m47, SEL_B2_E_B3_E), one, off)};
#pragma unroll
    for (int i = 0; i < 4; i++) u[i] = g < 2 ? u[i] : 0u;
    return mk_h8(u[0], u[1], u[2], u[3]);
  }

  // Operand constants of the step (half H) for tile t; at a superblock's
  // first half also its new units.  Returns the rescale factor for acc.
  template <int H>
  __device__ __forceinline__ float prep(int t) {
    float r = 1.0f;
    if constexpr (!Q6) {
      const u4v& hd = fr[H][t].hdr;
      if (H == 0) {
        const float d = f16_bits_to_f32(hd.x), dmin = f16_bits_to_f32(hd.x >> 16);
        live[t] = d != 0.0f;
        const float dn = live[t] ? d : deff[t];
        const float inv = __builtin_amdgcn_rcpf(dn);  // 1 ulp: far below the fp32 accumulation error
        r = deff[t] * inv;
        deff[t] = dn;
        kk[t] = -64.0f * dmin * inv;
      }
      // sub-blocks 4H + 2(g>>1) (low nibbles) and the next (high nibbles)
      const int e0 = 4 * H + 2 * (g >> 1);
      uint32_t sc0, sc1, mn;
      lt_scale_min<H>(e0, hd, sc0, mn);
      lt_scale_min<H>(e0 + 1, hd, sc1, mn);
      const float f0 = live[t] ? (float)sc0 : 0.0f, f1 = live[t] ? (float)sc1 : 0.0f;
      sa[t] = hsplat(f0);
      ca[t] = hsplat(-1024.0f * f0);       // (1024 + q) * sc - 1024 sc
      sb[t] = hsplat(f1 * 0.0625f);
      cb[t] = hsplat(-64.0f * f1);         // (1024 + 16 q) * sc/16 - 64 sc
      if (H == 1 && !LEAN) bmin[t] = mins(t);
    } else {
      if (H == 0) {
        const float d = f16_bits_to_f32(fr[H][t].d);
        live[t] = d != 0.0f;
        const float dn = live[t] ? 16.0f * d : deff[t];
        r = deff[t] * __builtin_amdgcn_rcpf(dn);
        deff[t] = dn;
      }
      // scale index (g>>1) + 2t within the half: t = g&1 (s < 2), t + 2 (s >= 2)
      const uint32_t sh = 8 * ((g >> 1) + 2 * (g & 1));
      const int sc_a = live[t] ? (int)(int8_t)(fr[H][t].sc.x >> sh) : 0;
      const int sc_b = live[t] ? (int)(int8_t)(fr[H][t].sc.y >> sh) : 0;
      const int ha = sc_a >> 4, la = sc_a & 15, hb = sc_b >> 4, lb = sc_b & 15;
      // s < 2: value 1024 + v6;  s >= 2: 1024 + 16*v6
      sa[t] = hsplat((float)ha);
      ca[t] = hsplat(-1056.0f * (float)ha);
      sla[t] = hsplat((float)la * 0.0625f);
      cla[t] = hsplat(-66.0f * (float)la);
      sb[t] = hsplat((float)hb * 0.0625f);
      cb[t] = hsplat(-96.0f * (float)hb);
      slb[t] = hsplat((float)lb * 0.00390625f);
      clb[t] = hsplat(-6.0f * (float)lb);
    }
    return r;
  }

  // B operand(s) of step s for tile t.  Q4_K: steps s and s+2 use the same
  // bytes (low / high nibbles), decoded together at s < 2.
  template <int H>
  __device__ __forceinline__ void decode(int t, int s, h8& b, h8& b2, h8& bl) const {
    const Frag& f = fr[H][t];
    const int wi = 2 * (s & 1);
    if constexpr (FMT == CQ_Q4_K) {
      const uint32_t w0 = u4_at(f.q, wi), w1 = u4_at(f.q, wi + 1);
      const uint32_t p0 = perm(C64, w0, SEL_B0_E_B1_E), p1 = perm(C64, w0, SEL_B2_E_B3_E);
      const uint32_t p2 = perm(C64, w1, SEL_B0_E_B1_E), p3 = perm(C64, w1, SEL_B2_E_B3_E);
      b = mk_h8(pk_fma(p0 & 0x640F640Fu, sa[t], ca[t]), pk_fma(p1 & 0x640F640Fu, sa[t], ca[t]),
                pk_fma(p2 & 0x640F640Fu, sa[t], ca[t]), pk_fma(p3 & 0x640F640Fu, sa[t], ca[t]));
      b2 = mk_h8(pk_fma(p0 & 0x64F064F0u, sb[t], cb[t]), pk_fma(p1 & 0x64F064F0u, sb[t], cb[t]),
                 pk_fma(p2 & 0x64F064F0u, sb[t], cb[t]), pk_fma(p3 & 0x64F064F0u, sb[t], cb[t]));
    } else if constexpr (FMT == CQ_Q5_K) {
      const int bit = 4 * H + 2 * (g >> 1) + (s >> 1);  // sub-block = qh bit
      uint32_t u[4];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const uint32_t wq = u4_at(f.q, wi + e), hq = u4_at(f.qh, wi + e);
        if (s < 2) {
          // qh bit -> bit 4 of each byte, under the low nibble
          const uint32_t z = bfi(0x10101010u, rotr(hq, (bit - 4) & 31), wq);
          u[2 * e] = pk_fma(perm(C64, z, SEL_B0_E_B1_E) & 0x641F641Fu, sa[t], ca[t]);
          u[2 * e + 1] = pk_fma(perm(C64, z, SEL_B2_E_B3_E) & 0x641F641Fu, sa[t], ca[t]);
        } else {
          // high nibble at bits 4-7 of the half, qh bit at bit 8 under 0x64
          const uint32_t hx = ((hq >> bit) & 0x01010101u) | C64;
          u[2 * e] = pk_fma(perm(hx, wq, SEL_X_B01) & 0x65F065F0u, sb[t], cb[t]);
          u[2 * e + 1] = pk_fma(perm(hx, wq, SEL_X_B23) & 0x65F065F0u, sb[t], cb[t]);
        }
      }
      b = mk_h8(u[0], u[1], u[2], u[3]);
    } else {
      uint32_t uh[4], ul[4];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const uint32_t wq = u4_at(f.ql, wi + e), hq = u4_at(f.qh, wi + e);
        uint32_t v0, v1;
        if (s < 2) {
          // quadrant t = g&1: qh bits 2t, 2t+1 -> bits 4, 5 under the low nibble
          const uint32_t z = bfi(0x30303030u, hq << (4 - 2 * (g & 1)), wq);
          v0 = perm(C64, z, SEL_B0_E_B1_E) & 0x643F643Fu;
          v1 = perm(C64, z, SEL_B2_E_B3_E) & 0x643F643Fu;
          uh[2 * e] = pk_fma(v0, sa[t], ca[t]);
          uh[2 * e + 1] = pk_fma(v1, sa[t], ca[t]);
          ul[2 * e] = pk_fma(v0, sla[t], cla[t]);
          ul[2 * e + 1] = pk_fma(v1, sla[t], cla[t]);
        } else {
          // quadrant t = 2 + (g&1): high nibble, qh bits 2t, 2t+1 at bits 8, 9
          const uint32_t hx = ((hq >> (4 + 2 * (g & 1))) & 0x03030303u) | C64;
          v0 = perm(hx, wq, SEL_X_B01) & 0x67F067F0u;
          v1 = perm(hx, wq, SEL_X_B23) & 0x67F067F0u;
          uh[2 * e] = pk_fma(v0, sb[t], cb[t]);
          uh[2 * e + 1] = pk_fma(v1, sb[t], cb[t]);
          ul[2 * e] = pk_fma(v0, slb[t], clb[t]);
          ul[2 * e + 1] = pk_fma(v1, slb[t], clb[t]);
        }
      }
      b = mk_h8(uh[0], uh[1], uh[2], uh[3]);
      bl = mk_h8(ul[0], ul[1], ul[2], ul[3]);
    }
  }

  // One step (half H of superblock u) on staged chunk X and, at H == 1, the
  // superblock's sub-block sums S.
  template <int H>
  __device__ __forceinline__ void compute(const _Float16* X, const _Float16* S) {
    float r[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) r[t] = prep<H>(t);
    const char* xr = (const char*)(X + j * LT_KC);
    // A fragments: a ring of HR registers (MT/2, at most 4).  Tile tm's
    // fragment of step s sits in slot tm % HR; once its MFMAs are issued the
    // slot is reloaded with the fragment needed HR tiles later (tile tm + HR
    // of this step, or tile tm + HR - MT of the next), NT * HR MFMAs ahead of
    // its use.
    constexpr int HR = LEAN ? 2 : MT / 2 < 4 ? MT / 2 : 4;
    auto afrag = [&](int s, int tm) { return *(const h8*)(xr + tm * 16 * LT_KC * 2 + acol[s]); };
    h8 av[HR];
#pragma unroll
    for (int i = 0; i < HR; i++) av[i] = afrag(0, i);
    h8 bsave[2][NT];  // Q4_K: high-nibble operands of steps 2, 3
#pragma unroll
    for (int s = 0; s < 4; s++) {
      h8 b[NT], bl[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        if (FMT == CQ_Q4_K && s >= 2 && LEAN) {
          h8 lo;
          decode<H>(t, s - 2, lo, b[t], bl[t]);  // the same bytes' high nibbles
        } else if (FMT == CQ_Q4_K && s >= 2) {
          b[t] = bsave[s & 1][t];
        } else {
          h8 b2;
          decode<H>(t, s, b[t], b2, bl[t]);
          if (FMT == CQ_Q4_K && !LEAN) bsave[s & 1][t] = b2;
        }
      }
#pragma unroll
      for (int tm = 0; tm < MT; tm++) {
        const int slot = tm % HR;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if (H == 0 && s == 0) {
#pragma unroll
            for (int q = 0; q < 4; q++) acc[t][tm][q] *= r[t];
          }
          acc[t][tm] = mfma(av[slot], b[t], acc[t][tm]);
        }
        if constexpr (Q6) {
#pragma unroll
          for (int t = 0; t < NT; t++) acc[t][tm] = mfma(av[slot], bl[t], acc[t][tm]);
        }
        if (tm + HR < MT) av[slot] = afrag(s, tm + HR);
        else if (s < 3) av[slot] = afrag(s + 1, tm + HR - MT);
        // LEAN: no fragment read moves above its ring slot's last use
        if constexpr (LEAN) __builtin_amdgcn_sched_barrier(0);
      }
      // keep each step's decode next to its MFMAs
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!Q6) {
      if (H == 1) {
        // min term: lane group 0 reads the sums' hi halves, group 1 the lo
        // halves (groups 2, 3 meet zero mins)
        const f4 zero4 = {0, 0, 0, 0};
#pragma unroll
        for (int tm = 0; tm < MT; tm++) {
          const h8 as = *(const h8*)(S + (16 * tm + j) * 16 + 8 * (g & 1));
#pragma unroll
          for (int t = 0; t < NT; t++) {
            const f4 cm = mfma(as, LEAN ? mins(t) : bmin[t], zero4);
#pragma unroll
            for (int q = 0; q < 4; q++) acc[t][tm][q] = __builtin_fmaf(kk[t], cm[q], acc[t][tm][q]);
          }
        }
      }
    }
  }
};

// Workgroup -> tile map.  Consecutive workgroup ids go to different XCDs
// (round robin over 8); remapping so that each XCD walks a contiguous run of
// tiles in activation-block-major order keeps an activation block hot in
// that XCD's L2 while its weight tiles stream past.
__device__ __forceinline__ void lt_tile(int& bx, int& by) {
  const int nx = gridDim.x, total = nx * gridDim.y;
  int id = blockIdx.x + nx * blockIdx.y;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  bx = id % nx;
  by = id / nx;
}

template <int FMT, int YT, int NT, int MT, int NW>
__device__ __forceinline__ void gemm2_body(const LtArgs& a) {
  // Distinct arrays, sized for this MT (so MT = 8 leaves room for two
  // workgroups per compute unit): the compiler can then see that reading one
  // buffer never aliases a pending DMA into another and inserts no wait.
  __shared__ __attribute__((aligned(16))) _Float16 lt_x0[16 * MT * LT_KC];
  __shared__ __attribute__((aligned(16))) _Float16 lt_x1[16 * MT * LT_KC];
  __shared__ __attribute__((aligned(16))) _Float16 lt_s0[16 * MT * 16];
  __shared__ __attribute__((aligned(16))) _Float16 lt_s1[16 * MT * 16];
  LtGemm<FMT, YT, NT, MT> s;
  s.lane = threadIdx.x & 63;
  s.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  s.j = s.lane & 15;
  s.g = s.lane >> 4;
  int bx, by;
  lt_tile(bx, by);
  const int n0 = (bx * NW + s.wave) * 16 * NT;
  const int m0 = by * 16 * MT;
  // K slice of this workgroup: superblocks [ub, ub + nu)
  const int ub = blockIdx.z * a.usplit;
  const int nu = min(a.usplit, a.units - ub);
  const int wg_row0 = bx * NW * 16 * NT;  // < N: the grid covers the rows
  s.wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + (size_t)wg_row0 * a.row_bytes + (size_t)ub * FmtTraits<FMT>::bytes), (short)0, 0x7fffffff,
      LT_RSRC_FLAGS);
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int row = min(n0 + 16 * t + s.j, a.N - 1);
    s.vo[t] = lt_vo<FMT>((uint32_t)((row - wg_row0) * a.row_bytes), s.g);
    s.deff[t] = 1.0f;
    s.kk[t] = 0.0f;
    s.live[t] = true;
#pragma unroll
    for (int tm = 0; tm < MT; tm++) s.acc[t][tm] = f4{0, 0, 0, 0};
  }
  const int swj = lt_sw<FMT>(s.j);
#pragma unroll
  for (int q = 0; q < 4; q++) s.acol[q] = 16 * (lt_chunk<FMT>(s.g, q) ^ swj);

  // Activation DMA: instruction i moves staged rows 4i .. 4i+3 (16 lanes x
  // 16 B each); this wave issues i = wave + NW ii.  Lane (row r, slot v)
  // fetches the row's chunk v ^ lt_sw(r); r & 15 does not depend on ii.
  // 32-bit offsets (M * K * 2 < 2^31 is checked by the host) from a uniform
  // base.  global_load_lds, not the buffer form: with it the compiler sees
  // which LDS array a DMA writes and lets the reads of the other array run
  // while it is in flight (for buffer-to-LDS loads it waits for them).
  const uint32_t K2 = (uint32_t)a.K * 2;
  const uint32_t dr = 4 * s.wave + (s.lane >> 4);
  const uint32_t dsw = 16 * ((s.lane & 15) ^ lt_sw<FMT>(dr));
  const uint32_t xoff0 = (m0 + dr) * K2 + dsw, xmax = (uint32_t)(a.M - 1) * K2 + dsw;
  auto dma_x = [&](_Float16* buf, int step) {
    const char* base = (const char*)a.x + (2 * ub + step) * (LT_KC * 2);
#pragma unroll
    for (int ii = 0; ii < 4 * MT / NW; ii++) {
      const uint32_t off = min(xoff0 + ii * 4 * NW * K2, xmax);
      __builtin_amdgcn_global_load_lds((lt_glb_t*)(base + off), (lt_lds_t*)(buf + (s.wave + NW * ii) * 512), 16, 0, 0);
    }
  };
  // Sums DMA: 32 rows (2 x 16 B each) per instruction, MT/2 instructions.
  const int srow = s.lane >> 1;
  auto dma_s = [&](_Float16* buf, int u) {
#pragma unroll
    for (int ii = 0; ii < (MT / 2 + NW - 1) / NW; ii++) {
      const int i = s.wave + NW * ii;
      if (i < MT / 2) {
        const int row = min(m0 + 32 * i + srow, a.M - 1);
        const _Float16* src = a.xs + ((size_t)row * a.units + ub + u) * 16 + 8 * (s.lane & 1);
        __builtin_amdgcn_global_load_lds((lt_glb_t*)src, (lt_lds_t*)(buf + i * 512), 16, 0, 0);
      }
    }
  };
  const bool kq = FMT != CQ_Q6_K;
  dma_x(lt_x0, 0);
  if (kq) dma_s(lt_s0, 0);
  s.template load_w<0>(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int steps = 2 * nu;
  // One step: prefetch the next (activation DMA, its sums at a superblock
  // boundary, the weight bytes), compute this one, then wait and barrier.
  auto step = [&](auto hc, auto pc, int i) {
    constexpr int H = decltype(hc)::value, P = decltype(pc)::value;  // half, superblock parity
    _Float16* xc = H ? lt_x1 : lt_x0;
    _Float16* xn = H ? lt_x0 : lt_x1;
    const bool more = i + 1 < steps;
    if (more) {
      dma_x(xn, i + 1);
      if (kq && H == 1) dma_s(P ? lt_s0 : lt_s1, (i + 1) >> 1);
      s.template load_w<1 - H>(i + 1);
    }
    s.template compute<H>(xc, P ? lt_s1 : lt_s0);
    if (more) {
      // this wave's DMA for step i+1 has landed (the weight loads issued
      // behind it were issued a whole step ago and are normally complete)
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
  };
  typedef std::integral_constant<int, 0> I0;
  typedef std::integral_constant<int, 1> I1;
  for (int i = 0; i < steps; i += 4) {
    step(I0{}, I0{}, i);
    step(I1{}, I0{}, i + 1);
    if (i + 2 < steps) {
      step(I0{}, I1{}, i + 2);
      step(I1{}, I1{}, i + 3);
    }
  }
  // (Q5_K with two weight tiles sits at the 256-VGPR limit: a second store
  // path spills a value that its K loop reloads, so it keeps the per-store
  // epilogue below.)
  constexpr bool EPI_T = !(FMT == CQ_Q5_K && NT == 2 && MT == 8);
  // Epilogue (bias, gated act(v) * aux): cq_store_tiles_epi picks the
  // activation once and loads every bias / aux value ahead of the stores.
  // Carrying all three activations at each of a thread's 64 unrolled stores,
  // with each aux load waiting for the stores before it, made the gated
  // gate / up prefill 18944 x 3584 at m = 512 take 159 us for gate's launch
  // against 119 without the epilogue (now within 1 us of it).
  if (EPI_T && !a.part && (a.epi.bias || a.epi.aux) &&
      cq_store_tiles_epi<YT, NT, MT>(a.epi, a.y, a.M, a.N, m0, n0, s.g, s.j, s.acc, s.deff))
    return;
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int tm = 0; tm < MT; tm++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * tm + 4 * s.g + r, n = n0 + 16 * t + s.j;
        if (m < a.M && n < a.N) {
          const float v = s.deff[t] * s.acc[t][tm][r];
          if (a.part) a.part[((size_t)blockIdx.z * a.M + m) * a.N + n] = v;
          else cq_store<YT>(a.y, a.epi, v, (size_t)m * a.N + n, n);
        }
      }
    }
  }
}

// Sub-block sums of fp16 activations for the K-quant min term:
// xs[m][u][sb] = hi, xs[m][u][8 + sb] = lo, hi + lo = sum(x[m][256u + 32sb ..
// +32]) / 64 (the 1/64 keeps sums of up to 32 * 65504 inside fp16).  One
// thread per (m, u, sb).
__device__ __forceinline__ void xsums_body(const _Float16* x, _Float16* xs, int M, int K) {
  const int units = K / 256;
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (long long)M * units * 8) return;
  const int sb = (int)(tid & 7);
  const long long mu = tid >> 3;
  const int u = (int)(mu % units);
  const long long m = mu / units;
  const uint8_t* p = (const uint8_t*)(x + m * K + 256 * u + 32 * sb);
  const h2 one = {1, 1};
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const u4v v = ld_u128(p + 16 * q);
    acc = __builtin_amdgcn_fdot2(as_h2(v.x), one, acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(v.y), one, acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(v.z), one, acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(v.w), one, acc, false);
  }
  acc *= 0.015625f;
  const _Float16 hi = (_Float16)acc;
  _Float16* o = xs + mu * 16;
  o[sb] = hi;
  o[8 + sb] = (_Float16)(acc - (float)hi);
}

// Split-K epilogue: y = sum over the slices' fp32 partials, in slice order.
template <int YT>
__device__ __forceinline__ void splitk_reduce_body(const float* part, void* y, int splits, long long mn, int N,
                                                   CqEpi epi) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= mn) return;
  float v = 0.0f;
  for (int z = 0; z < splits; z++) v += part[z * mn + i];
  cq_store<YT>(y, epi, v, (size_t)i, (int)(i % N));
}

// Decode GEMV for a few fp16 activation rows (2 <= m <= 16), K-quant
// weights, with every activation fragment loaded once per workgroup
// (cq_gemvq_*): y[m, n] = sum_k x[m, k] * W[n, k].
// Replaces qmatmul.rs:881-930 (Q4_K), :1064-1117 (Q5_K) and :1184-1229
// (Q6_K) for batched decode.
//
// Why.  In the MFMA operand layout a lane holds 8 consecutive activations of
// one row, so a 16-byte-per-lane load of A fragments touches 16 rows x 4
// k-groups = 64 distinct 128-byte lines per instruction; reading the m x K
// activation block that way once per 16-row tile (cq_gemvd) is bound by
// cache-line traffic, not bytes (measured: the activation loads alone of a
// 14336 x 4096 weight at m = 16 take 7 us).  And a tile's weight bytes,
// fetched as 16-byte pieces of 16 rows at a row stride, stream poorly.
//
// Work mapping.
//   - Wave u of a workgroup owns superblock column cb + u of a slice of at
//     most 16 columns (rows of up to 16 superblocks are one slice; longer
//     rows are split into slices over blockIdx.y, whose fp32 partials
//     cq_splitk_reduce_* adds in slice order).  Its activations (m rows x 256 values)
//     arrive once, by LDS DMA (global_load_lds, whole 512-byte row pieces,
//     two rows per instruction) through its ring, and are read into
//     registers in the operand layout (8 x 16 bytes per lane), where they
//     stay for the whole launch.
//   - The workgroup walks a contiguous range of 16-row tiles (the grid is
//     at most one workgroup per compute unit, the tiles split as evenly as
//     floor division allows).  Each wave streams its column of every tile
//     (16 rows x one superblock, each row's bytes from the 16-byte boundary
//     at or below the superblock) through a ring of R slots of its own by
//     LDS DMA, waiting for a slot by position in the in-order load counter,
//     so no wave waits for another while loading.  Dynamic LDS per wave:
//     the ring (R x NI KB), then 1 KB of the workgroup's partial sums.
//   - Each wave keeps its 16 x 16 partial blocks (4 fp32 per lane) of
//     TC tiles (as many as LDS allows: 1 to 4) in registers; then they
//     are added across the waves in LDS in wave order, one thread per
//     output (one barrier pair per chunk), and stored through the epilogue.
//     (Reducing after every tile made every wave wait for the slowest
//     wave's weight bytes once per tile: 13.2 against 10.3 us with no
//     reduction at all, Q4_K 14336 x 4096 at m = 2.)
//   - Superblock arithmetic is the MFMA GEMV's (cq_gemv.h: exact q * sc
//     fp16 operands, d / dmin on the fp32 results, the K-quant min term as
//     an MFMA against the 6-bit mins).
// Activation rows >= m are read as row m - 1 (their outputs are not
// stored); weight rows >= n are read as row n - 1 (likewise).
#pragma once
#include "cq_gemvd.h"
#include "cq_gemv1.h"

#define GVQ_MAX_WAVES 16
#define GVQ_MAX_SEG 4  // weights of one launch

// Segments: the weights of one launch (same format and K, one activation
// block): segment s owns global tiles [segt[s], segt[s + 1]) of 16 of its
// rows.  Gated (two segments, gate and up of the same shape): every tile
// is 8 gate rows and the same 8 up rows, and the output is act(gate) * up.
struct GvqArgs {
  const _Float16* x;  // [M][K]
  float* part;        // split (one segment): [slices][M][N] fp32 partial sums, else null
  long long row_bytes;
  int M, K, units;    // units = K / 256
  int tiles;          // tiles of all segments
  int nseg, gated;
  int segt[GVQ_MAX_SEG + 1];
  const uint8_t* segw[GVQ_MAX_SEG];  // packed weight, [N rows][row_bytes]
  void* segy[GVQ_MAX_SEG];           // [M][N] fp32 or fp16
  int segn[GVQ_MAX_SEG];             // N
  long long segwb[GVQ_MAX_SEG];      // weight bytes (the DMA never reads past them)
  CqEpi epi;          // one segment only (gated: epi.act)
};

// A column is 256 values of a row: one K-quant superblock, or 8 blocks of a
// 32-value format.  Per wave a ring of two slots, each 16 rows x PR
// 16-byte pieces (a column from the 16-byte boundary at or below its start;
// DMA lanes past the last piece are masked off), rounded up to 256 bytes,
// then TC KB of partial sums, within a 10 KB share of the 160 KB.
template <int FMT>
struct GvqShape {
  static constexpr bool KQ = FmtTraits<FMT>::vals == 256;
  static constexpr int CB = KQ ? FmtTraits<FMT>::bytes : 8 * FmtTraits<FMT>::bytes / LB;  // column bytes per row
  static constexpr int PR = CB % 16 == 0 ? CB / 16 : (CB + 15) / 16 + 1;
  static constexpr int P = 16 * PR;                 // pieces per slot
  static constexpr int NI = (P + 63) / 64;          // DMA instructions per slot
  static constexpr int SLOT = (16 * P + 255) / 256 * 256;  // bytes
  static constexpr int R = 2;
  // tiles per cross-wave reduction (their partial sums in registers, then
  // LDS): what LDS leaves, at most 4 (2 for Q6_K's larger decode state)
  static constexpr int TC_LDS = (10240 - R * SLOT) / 1024;
  static constexpr int TC = TC_LDS < (FMT == CQ_Q6_K ? 2 : 4) ? TC_LDS : (FMT == CQ_Q6_K ? 2 : 4);
  // activation row pairs of 1 KB that slot 1 and the partial sums carry
  static constexpr int PH = (10240 - SLOT) / 1024;
  static constexpr int WAVE_BYTES = 10240;
  static_assert(TC >= 1 && PH >= 1, "column too large for the LDS share");
};

// A fragment s of lane group g of a column, as 16-byte pieces p0 (and, for
// the 4-bit / 5-bit legacy formats, the second half of a split fragment at
// byte offset o1 of piece p1): the k layout the format's B operands use.
template <int FMT>
__device__ __forceinline__ void gvq_apos(int g, int s, int& p0, int& o0, int& p1, int& o1) {
  if constexpr (FmtTraits<FMT>::vals == 256) {
    p0 = (gvd_abase<FMT>(g) + gvd_aoff<FMT>(s)) >> 3;  // 8 values = one piece
    o0 = 0;
    p1 = -1;
    o1 = 0;
  } else if constexpr (FMT == CQ_Q8_0) {
    p0 = 4 * s + g;  // block s, k = 32 s + 8 g .. + 7
    o0 = 0;
    p1 = -1;
    o1 = 0;
  } else {
    // block s: k = 32 s + 4 g .. + 3, then 32 s + 16 + 4 g .. + 3
    p0 = 4 * s + (g >> 1);
    o0 = 8 * (g & 1);
    p1 = 4 * s + 2 + (g >> 1);
    o1 = 8 * (g & 1);
  }
}

// Q4_K / Q5_K min term: the wave's column is fixed for the launch, so its
// sub-block activation sums are formed once (as sum / 64, fp16 hi + lo, so
// no fp16 overflows), in the A layout of a 16x16x16 MFMA: lane group 0 / 1
// holds the hi halves of sub-blocks 0-3 / 4-7, group 2 / 3 the lo halves.
// Lane (row j, group g) of the fragments holds k = 64 g + 8 s: sub-block 2g
// (s < 4) and 2g + 1 (s >= 4); the rearrangement is two lane shuffles.
__device__ __forceinline__ h4 gvq_xsums(const h8 (&xa)[8], int lane) {
  const h2 one = {1, 1};
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const u4v v = __builtin_bit_cast(u4v, xa[s]);
    float t = __builtin_amdgcn_fdot2(as_h2(v.x), one, 0.0f, false);
    t = __builtin_amdgcn_fdot2(as_h2(v.y), one, t, false);
    t = __builtin_amdgcn_fdot2(as_h2(v.z), one, t, false);
    t = __builtin_amdgcn_fdot2(as_h2(v.w), one, t, false);
    if (s < 4) s0 += t;
    else s1 += t;
  }
  const int j = lane & 15, g = lane >> 4, hh = g & 1;
  // sub-blocks 4 hh + 0, 1 from group 2 hh; 4 hh + 2, 3 from group 2 hh + 1
  const int la = 16 * (2 * hh) + j, lb = la + 16;
  const float v[4] = {__shfl(s0, la, 64) * 0.015625f, __shfl(s1, la, 64) * 0.015625f,
                      __shfl(s0, lb, 64) * 0.015625f, __shfl(s1, lb, 64) * 0.015625f};
  h4 r;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const _Float16 hi = (_Float16)v[e];
    r[e] = g < 2 ? hi : (_Float16)(v[e] - (float)hi);
  }
  return r;
}
// B operand for that MFMA: the 6-bit mins of sub-blocks 4 (g & 1) + 0..3 as
// exact fp16 (1024 + m under the fp16 exponent, less 1024).
__device__ __forceinline__ h4 gvq_mins(const u4v& hdr, int g) {
  const uint32_t m03 = hdr.z & 0x3F3F3F3Fu;
  const uint32_t m47 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
  const uint32_t mm = (g & 1) ? m47 : m03;
  const h2 one = hsplat(1.0f), off = hsplat(-1024.0f);
  const uint32_t a = pk_fma(perm(C64, mm, SEL_B0_E_B1_E), one, off);
  const uint32_t b = pk_fma(perm(C64, mm, SEL_B2_E_B3_E), one, off);
  return __builtin_bit_cast(h4, u2v{a, b});
}

// One column of one 16-row tile against the lane's 8 A fragments (legacy:
// block s meets fragment s; every block's fp16 scale, and the affine
// formats' min times the block's activation sum, applied to fp32 results).
template <int FMT, bool MSUM>
__device__ __forceinline__ f4 gvq_column(const uint8_t* wp, const h8 (&xa)[8], const h4& xs, int g) {
  if constexpr (FMT == CQ_Q6_K) {
    typename FmtTraits<FMT>::Frag f;
    load_unit<FMT>(f, wp, g, 0);
    return gvd_superblock<FMT>(f, xa, g);
  } else if constexpr (FmtTraits<FMT>::vals == 256) {
    if constexpr (!MSUM) {
      // min term by 8 MFMAs against the mins (no sums set-up)
      typename FmtTraits<FMT>::Frag f;
      load_unit<FMT>(f, wp, g, 0);
      return gvd_superblock<FMT>(f, xa, g);
    }
    // main term by 8 MFMAs on the exact q*sc operands; the min term
    // sum_sb m_sb * sum(x in sb) by one 16x16x16 MFMA against the column's
    // sub-block sums / 64
    typename FmtTraits<FMT>::Frag f;
    load_unit<FMT>(f, wp, g, 0);
    DecKQ o;
    if constexpr (FMT == CQ_Q4_K) decode_q4k(f, g, o);
    else decode_q5k(f, g, o);
    f4 c = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; s++) c = mfma(xa[s], o.b[s], c);
    const f4 cm = __builtin_amdgcn_mfma_f32_16x16x16f16(xs, gvq_mins(f.hdr, g), f4{0, 0, 0, 0}, 0, 0, 0);
    f4 res;
#pragma unroll
    for (int r = 0; r < 4; r++) res[r] = __builtin_fmaf(-64.0f * o.dmin, cm[r], o.d * c[r]);
    return res;
  } else {
    f4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < 2; h++) {
      typename FmtTraits<FMT>::Frag f;
      load_unit<FMT>(f, wp + h * LB * FmtTraits<FMT>::bytes / LB, g, LB);
#pragma unroll
      for (int i = 0; i < LB; i++) {
        const h8 b = legacy_b(f, i, g);
        const h8 a = xa[LB * h + i];
        if constexpr (FMT == CQ_Q4_1 || FMT == CQ_Q5_1) {
          affine_block<0>(A8<0>{a, a}, b, legacy_d(f, i), acc);
        } else {
          const f4 c = mfma(a, b, f4{0, 0, 0, 0});
          const float d = f16_bits_to_f32(legacy_d(f, i));
#pragma unroll
          for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(d, c[r], acc[r]);
        }
      }
    }
    return acc;
  }
}

// MODE 0: one weight (segment 0); 1: segments; 2: gated pair.  MSUM (Q4_K /
// Q5_K): the min term by one MFMA against the column's sub-block sums, whose
// set-up pays from two tiles per workgroup on (Q4_K 14336 x 4096, 3-4
// tiles: 12.0-12.5 -> 11.6 us at m = 2; 4096 x 4096, one tile: 6.5 -> 7.0);
// the host picks it when every workgroup has at least two.
// EPI (one weight only): apply the bias / gated epilogue at the store.  Its
// argument fields otherwise stay live in scalar registers through the tile
// loop and spill (8-30 SGPRs), so launches without an epilogue take the
// kernels built without it.
template <int FMT, int YT, int MODE, bool MSUM, bool EPI>
__device__ __forceinline__ void gemvq_body(const GvqArgs& a) {
  static_assert(!EPI || MODE == 0, "the epilogue is for one-weight launches");
  static_assert(!MSUM || FMT == CQ_Q4_K || FMT == CQ_Q5_K, "sums for the K-quant min term only");
  typedef GvqShape<FMT> S;
  constexpr int CB = S::CB, PR = S::PR, P = S::P, NI = S::NI, SLOT = S::SLOT, R = S::R, TC = S::TC;
  extern __shared__ __attribute__((aligned(16))) u4v gq_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  // superblock columns [cb, cb + cols) of this slice (blockIdx.y); waves
  // past the last column only take part in the reductions
  const int cb = (int)blockIdx.y * nw;
  const int cols = min(nw, a.units - cb);
  const bool live = wave < cols;
  const int j = lane & 15, g = lane >> 4;
  u4v* ring = gq_lds + wave * (S::WAVE_BYTES / 16);
  // partial sums of wave w, tile tt of a chunk: TC KB after w's ring
  auto red_at = [&](int w, int tt, int r, int ln) -> float& {
    return ((float*)((uint8_t*)gq_lds + w * S::WAVE_BYTES + R * SLOT))[(tt * 4 + r) * 64 + ln];
  };
  const uint32_t rb = gv3_lds_addr(ring);
  // this workgroup's tiles [t0, t0 + nmine)
  const int G = (int)gridDim.x;
  const int t0 = (int)((long long)blockIdx.x * a.tiles / G);
  const int nmine = (int)((long long)(blockIdx.x + 1) * a.tiles / G) - t0;

  // Weight pieces of this lane: piece q = 64 i + lane of a slot is piece
  // q % PR of row q / PR's column (from its 16-byte boundary); q >= P is
  // not loaded.
  int prow[NI], poff[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int q = min(64 * i + lane, P - 1);
    prow[i] = q / PR;
    poff[i] = 16 * (q - prow[i] * PR);
  }
  const size_t col = (size_t)(cb + wave) * CB;
  // the segment holding global tile t (uniform), picked by a compare chain on
  // t: a select on a segment index is folded back into a dynamic index into
  // the kernel arguments, which the compiler then copies to scratch
  struct Seg {
    const uint8_t* w;
    void* y;
    size_t wlast;
    int t0, n;
  };
  auto seg_at = [&](int t) {
    Seg sg{a.segw[0], a.segy[0], (size_t)a.segwb[0] - 16, 0, a.segn[0]};
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 1; k < GVQ_MAX_SEG; k++)
        if (k < a.nseg && t >= a.segt[k]) sg = Seg{a.segw[k], a.segy[k], (size_t)a.segwb[k] - 16, a.segt[k], a.segn[k]};
    }
    return sg;
  };
  // weight, and byte offset in it, of row r (0..15) of global tile t's
  // column: gated tiles take rows 0-7 from the gate weight and 8-15 from the
  // up weight, 8 rows of each per tile
  auto row_src = [&](int t, int r, const uint8_t*& w, size_t& wlast) -> size_t {
    const Seg sg = seg_at(t);
    int row;
    w = sg.w;
    wlast = sg.wlast;
    if constexpr (MODE == 2) {
      row = 8 * t + (r & 7);
      if (r >= 8) {
        w = a.segw[1];
        wlast = (size_t)a.segwb[1] - 16;
      }
    } else {
      row = 16 * (t - sg.t0) + r;
    }
    return (size_t)min(row, sg.n - 1) * (size_t)a.row_bytes + col;
  };
  auto dma = [&](int t) {  // tile t0 + t into slot t % R
    const uint32_t lb = rb + SLOT * (t % R);
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const uint8_t* w;
      size_t wlast;
      const size_t s = row_src(t0 + t, prow[i], w, wlast);
      if (P % 64 == 0 || i + 1 < NI || 64 * i + lane < P)
        gv3_dma16(w + min((s & ~(size_t)15) + poff[i], wlast), lb + 1024 * i);
    }
  };
  // the lane's row within a slot: byte offset of its column
  auto my_off = [&](int t) {
    const uint8_t* w;
    size_t wlast;
    return (int)(row_src(t0 + t, j, w, wlast) & 15);
  };
  // Activations of column `wave`, carried by the wave's LDS after slot 0
  // (slot 1 and the partial sums' space) in phases of PH row pairs while
  // tile 0's weights land in slot 0 (their HBM latency hides the first
  // phase's; one phase up to 14 rows, 12 for Q6_K): DMA instruction p brings rows 2p
  // (even lanes) and 2p + 1 (odd lanes), piece (lane >> 1) ^ p of each
  // row's 32 16-byte pieces, so that the 16 rows' reads of one fragment
  // fall on 16 distinct 16-byte bank groups.
  constexpr int PH = S::PH;
  if (live) dma(0);
  const int pairs = live ? (a.M + 1) >> 1 : 0;
  const int xr = min(j, a.M - 1), xp = xr >> 1;  // the lane's activation row and its pair
  h8 xa[8] = {};
  for (int p0 = 0; p0 < pairs; p0 += PH) {
    const int pe = min(p0 + PH, pairs);
    for (int p = p0; p < pe; p++) {
      const int r = min(2 * p + (lane & 1), a.M - 1);
      gv3_dma16(a.x + (size_t)r * a.K + 256 * (cb + wave) + 8 * ((lane >> 1) ^ p), rb + SLOT + 1024 * (p - p0));
    }
    gv3_wait_vm<0>();
    if (xp >= p0 && xp < pe) {
      const uint8_t* base = (const uint8_t*)ring + SLOT + 1024 * (xp - p0) + 16 * (xr & 1);
#pragma unroll
      for (int s = 0; s < 8; s++) {
        int p0s, o0s, p1s, o1s;
        gvq_apos<FMT>(g, s, p0s, o0s, p1s, o1s);  // fragment s of lane group g
        if (p1s < 0) {
          xa[s] = __builtin_bit_cast(h8, ld_u128(base + 32 * (p0s ^ xp)));
        } else {
          const u2v lo = ld_u64(base + 32 * (p0s ^ xp) + o0s), hi = ld_u64(base + 32 * (p1s ^ xp) + o1s);
          xa[s] = __builtin_bit_cast(h8, u4v{lo.x, lo.y, hi.x, hi.y});
        }
      }
    }
    // the slots are reused only after these reads have completed
#pragma unroll
    for (int s = 0; s < 8; s++) asm volatile("" ::"v"(xa[s]));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
  }

  // MSUM: the column's sub-block sums for the K-quant min term (all lanes:
  // shuffles)
  h4 xs = {};
  if constexpr (MSUM) xs = gvq_xsums(xa, lane);
  for (int t = 1; live && t < R - 1 && t < nmine; t++) dma(t);
  // Tiles in chunks of TC: each wave keeps its partial sums of a chunk
  // in registers and the chunk is added across waves afterwards, so that
  // within a chunk no wave waits for another.
  for (int c0 = 0; c0 < nmine; c0 += TC) {
    f4 acc[TC];
#pragma unroll
    for (int tt = 0; tt < TC; tt++) {
      const int t = c0 + tt;
      acc[tt] = f4{0, 0, 0, 0};
      if (live && t < nmine) {
        // refill the slot of tile t - 1 (read completely) with tile
        // t + R - 1; near the end nothing is refilled and every load still
        // in flight is waited for
        if (t + R - 1 < nmine) {
          dma(t + R - 1);
          gv3_wait_vm<NI * (R - 1)>();  // tile t landed; tiles t + 1 .. t + R - 1 may be in flight
        } else {
          gv3_wait_vm<0>();
        }
        const uint8_t* wp = (const uint8_t*)ring + SLOT * (t % R) + 16 * PR * j + my_off(t);
        acc[tt] = gvq_column<FMT, MSUM>(wp, xa, xs, g);
        // this slot is refilled in a later iteration: its reads must be done
        __builtin_amdgcn_s_waitcnt(0xC07F);
        asm volatile("" ::: "memory");
      }
    }
    // the chunk's partial sums, [wave][tile][r][lane], added by one thread
    // per output: all partials in flight at once, then summed in wave order
#pragma unroll
    for (int tt = 0; tt < TC; tt++)
      if (c0 + tt < nmine)
#pragma unroll
        for (int r = 0; r < 4; r++) red_at(wave, tt, r, lane) = acc[tt][r];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256 * TC; idx += blockDim.x) {
      const int tt = idx >> 8, r = (idx >> 6) & 3, ln = idx & 63;
      if (c0 + tt < nmine) {
        float v[GVQ_MAX_WAVES];
#pragma unroll
        for (int w2 = 0; w2 < GVQ_MAX_WAVES; w2++) v[w2] = w2 < cols ? red_at(w2, tt, r, ln) : 0.0f;
        float s = v[0];
#pragma unroll
        for (int w2 = 1; w2 < GVQ_MAX_WAVES; w2++)
          if (w2 < cols) s += v[w2];
        const int m = 4 * (ln >> 4) + r, t = t0 + c0 + tt, c = ln & 15;
        if constexpr (MODE == 2) {
          // columns c < 8: gate row 8 t + c; its up row is column c + 8
          const int n = 8 * t + c, N = a.segn[0];
          float u = 0.0f;
          if (c < 8) {
#pragma unroll
            for (int w2 = 0; w2 < GVQ_MAX_WAVES; w2++) v[w2] = w2 < cols ? red_at(w2, tt, r, ln + 8) : 0.0f;
            u = v[0];
#pragma unroll
            for (int w2 = 1; w2 < GVQ_MAX_WAVES; w2++)
              if (w2 < cols) u += v[w2];
          }
          if (c < 8 && m < a.M && n < N) cq_store_raw<YT>(a.segy[0], cq_gated<YT>(s, u, a.epi.act), (size_t)m * N + n);
        } else {
          const Seg sg = seg_at(t);
          const int n = 16 * (t - sg.t0) + c, N = sg.n;
          void* const y = sg.y;
          if (m < a.M && n < N) {
            if (a.part) a.part[((size_t)blockIdx.y * a.M + m) * N + n] = s;
            else if constexpr (EPI) cq_store<YT>(y, a.epi, s, (size_t)m * N + n, n);
            else cq_store_raw<YT>(y, s, (size_t)m * N + n);
          }
        }
      }
    }
    __syncthreads();  // partial sums read before the next chunk writes them
  }
  gv3_wait_vm<0>();  // no LDS DMA may still be landing when the workgroup ends
}

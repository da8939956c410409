// Decode GEMV for a few fp16 activation rows (2 <= m <= 16), K-quant
// weights, with the activation block shared through LDS and the K range
// split over workgroups (cq_gemvs_*): y[m, n] = sum_k x[m, k] * W[n, k].
// Replaces qmatmul.rs:881-930 (Q4_K), :1064-1117 (Q5_K) and :1184-1229
// (Q6_K) for batched decode.
//
// Why: with one 16-row weight tile per workgroup (cq_gemvd), every tile
// reads the whole m x K activation block (16 x 14336 fp16 = 458 KB per
// 16 rows of a 4096 x 14336 weight: 3.5 times the weight's own bytes) and
// few bytes of weights are in flight per compute unit.  Here:
//   - a workgroup is 8 waves x one 16-row tile each = 128 weight rows, over
//     a slice of the superblocks (blockIdx.y; the slices' fp32 partials are
//     added by cq_splitk_reduce_* in slice order), so the grid still fills
//     the chip while each superblock's activations (16 rows x 256 values,
//     8 KB) are read once per 128 rows;
//   - every step (one superblock) arrives by LDS DMA (global_load_lds,
//     issued as inline assembly so that the kernel alone decides which
//     loads to wait for): the activation chunk, two half-wave instructions
//     per wave, and each wave's 16 rows of weight bytes, NI instructions;
//     a ring of R = 4 slots keeps three steps in flight while one is
//     computed, one barrier per step;
//   - the superblock arithmetic is the MFMA GEMV's (cq_gemv.h: exact q * sc
//     fp16 operands, d / dmin on the fp32 results, the K-quant min term as
//     an MFMA against the 6-bit mins), reading the weight fields and the A
//     fragments from LDS.
// Activation rows >= m are staged as row m - 1 (those outputs are not
// stored); steps past a slice's end re-load its last superblock into the
// unused slot, so every wave issues the same loads in the same order and
// the wait counts stay exact.
#pragma once
#include "cq_gemv1.h"

struct GvsArgs {
  const uint8_t* w;    // packed superblocks, [N rows][row_bytes]
  const _Float16* x;   // [M][K]
  void* y;             // [M][N] fp32 or fp16 (no split)
  float* part;         // split: [splits][M][N] fp32 partial sums, else null
  long long row_bytes;
  long long wbytes;    // weight bytes (a multiple of 16)
  int M, N, K, units, usplit;
  CqEpi epi;
};

#define GVS_WAVES 8
#define GVS_R 4      // ring slots (steps in LDS)
#define GVS_XS 264   // halves per staged activation row (256 + 8: spreads the A-fragment reads over the banks)

// 16-byte pieces per row slot: the superblock from the 16-byte boundary at
// or below its start (Q6_K's 210-byte superblocks start at any even offset).
template <int FMT>
constexpr int gvs_pr() {
  return FmtTraits<FMT>::bytes % 16 == 0 ? FmtTraits<FMT>::bytes / 16 : 14;
}
template <int FMT>
constexpr int gvs_ni() {
  return (16 * gvs_pr<FMT>() + 63) / 64;
}

template <int FMT, int YT>
__device__ __forceinline__ void gemvs_body(const GvsArgs& a) {
  constexpr int PR = gvs_pr<FMT>(), SP = 16 * PR, NI = gvs_ni<FMT>();
  constexpr int BB = FmtTraits<FMT>::bytes;
  constexpr int PER = 2 + NI;  // DMA instructions per wave and step
  __shared__ __attribute__((aligned(16))) _Float16 gs_x[GVS_R][16 * GVS_XS];
  __shared__ __attribute__((aligned(16))) u4v gs_w[GVS_R][GVS_WAVES][SP];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int n0 = (int)blockIdx.x * 16 * GVS_WAVES + 16 * wave;
  const int ub = (int)blockIdx.y * a.usplit;
  const int nu = min(a.usplit, a.units - ub);
  // weight pieces of this lane: piece q = 64 i + lane of the wave's slot,
  // row q / PR of the tile, piece q % PR of that row's superblock
  size_t wrow[NI];
  int wpc[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int q = min(64 * i + lane, SP - 1);
    wrow[i] = (size_t)min(n0 + q / PR, a.N - 1) * (size_t)a.row_bytes;
    wpc[i] = q % PR;
  }
  const size_t wlast = (size_t)a.wbytes - 16;
  const int xr = 2 * wave + (lane >> 5);  // activation row this lane's DMA fetches
  const _Float16* xsrc = a.x + (size_t)min(xr, a.M - 1) * a.K + 8 * (lane & 31);
  auto dma = [&](int slot, int u) {
    u = min(u, nu - 1);
    const size_t sb = (size_t)(ub + u) * BB;
    const _Float16* xs = xsrc + (size_t)(ub + u) * 256;
    if (lane < 32) gv3_dma16(xs, gv3_lds_addr(&gs_x[slot][(2 * wave) * GVS_XS]));
    if (lane >= 32) gv3_dma16(xs, gv3_lds_addr(&gs_x[slot][(2 * wave + 1) * GVS_XS]) - 512);
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const size_t s = wrow[i] + sb;
      const uint8_t* src = a.w + min((s & ~(size_t)15) + 16 * (size_t)wpc[i], wlast);
      if (SP % 64 == 0 || i + 1 < NI || 64 * i + lane < SP) gv3_dma16(src, gv3_lds_addr(&gs_w[slot][wave][64 * i]));
    }
  };
  // the lane's row: byte offset of its superblock within the row slot
  const size_t my_row = (size_t)min(n0 + j, a.N - 1) * (size_t)a.row_bytes;
#pragma unroll
  for (int s = 0; s < GVS_R - 1; s++) dma(s, s);
  f4 acc = {0, 0, 0, 0};
  for (int i = 0; i < nu; i++) {
    gv3_wait_vm<PER * (GVS_R - 2)>();  // step i landed (this wave's part)
    __syncthreads();                    // every wave's part of step i landed, step i - 1 consumed
    dma((i + GVS_R - 1) % GVS_R, i + GVS_R - 1);
    const int slot = i % GVS_R;
    const int o = (int)((my_row + (size_t)(ub + i) * BB) & 15);
    const uint8_t* wp = (const uint8_t*)&gs_w[slot][wave][0] + j * PR * 16 + o;
    typename FmtTraits<FMT>::Frag f;
    load_unit<FMT>(f, wp, g, 0);
    const XRow<0> xrow(&gs_x[slot][0], &gs_x[slot][0], j, GVS_XS, 0, j < a.M);
    compute_unit<FMT, 0>(f, xrow, 0, g, 0, acc);
  }
  gv3_wait_vm<0>();  // no LDS DMA may still be landing when the workgroup ends
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int m = 4 * g + r, n = n0 + j;
    if (m < a.M && n < a.N) {
      if (a.part) a.part[((size_t)blockIdx.y * a.M + m) * a.N + n] = acc[r];
      else cq_store<YT>(a.y, a.epi, acc[r], (size_t)m * a.N + n, n);
    }
  }
}

// Decode GEMV for a few fp16 activation rows (2 <= m <= 16), K-quant
// weights, with the activations read straight from global memory:
// y[m, n] = sum_k x[m, k] * W[n, k].
// Replaces qmatmul.rs:881-930 (Q4_K), :1064-1117 (Q5_K) and :1184-1229
// (Q6_K) for batched decode.
//
// Work mapping.  A workgroup owns 16 * NT consecutive weight rows over the
// whole K range; its NW waves split the row's superblocks (wave w takes
// superblocks w, w + NW, ...) and their partial sums are added in LDS in
// wave order at the end.  Lane l of a wave owns weight row (l & 15) of each
// of its NT row tiles and k-group g = l >> 4, the operand layout of
// v_mfma_f32_16x16x32_f16 (A = activation rows, B = weight rows), so one
// MFMA yields 16 activation rows x 16 weight rows.
//
// Why no LDS staging: the whole activation block (m x K fp16, at most
// 16 x 16384 x 2 = 512 KB) sits in L2, every byte of it is used by exactly
// one wave of a workgroup, and each wave reuses its A fragments for all NT
// row tiles.  Loading the fragments into registers together with the weight
// bytes they meet keeps every wave streaming on its own, with no barrier and
// no LDS limit on the number of resident workgroups.  Each wave keeps D
// superblocks of loads (weights for NT tiles + 8 A fragments) in flight.
// Activation rows >= m are read as row m - 1 (same cache lines; those output
// rows are never stored).
//
// Superblock arithmetic is the MFMA GEMV's (exact q * sc fp16 operands, fp16
// d / dmin applied to the fp32 results, K-quant min term as an MFMA against
// the 6-bit mins).
#pragma once
#include "cq_gemv.h"

#define GVD_MAX_WAVES 8

struct GvdArgs {
  const uint8_t* w;   // packed superblocks, [N rows][row_bytes]
  const _Float16* x;  // [M][K]
  void* y;            // [M][N] fp32 or fp16
  long long row_bytes;
  int M, N, K, units;  // units = K / 256
  CqEpi epi;
};

// Element offset (within its superblock) of A fragment s of lane group g:
// Q4_K / Q5_K step s covers k = 64g + 8s .. +7; Q6_K step st covers
// q6k_koff(g, st).
template <int FMT>
__device__ __forceinline__ int gvd_abase(int g) {
  if constexpr (FMT == CQ_Q6_K) return 128 * (g >> 1) + 16 * (g & 1);
  return 64 * g;
}
template <int FMT>
__device__ __forceinline__ constexpr int gvd_aoff(int s) {
  if constexpr (FMT == CQ_Q6_K) return 32 * (s >> 1) + 8 * (s & 1);
  return 8 * s;
}

// One superblock of one 16-row tile against the lane's 8 A fragments: the
// fp32 contribution to the lane's 4 outputs.
template <int FMT>
__device__ __forceinline__ f4 gvd_superblock(const typename FmtTraits<FMT>::Frag& f, const h8 (&xa)[8], int g) {
  f4 res;
  if constexpr (FMT == CQ_Q6_K) {
    DecQ6 o;
    decode_q6k(f, g, o);
    f4 chi = {0, 0, 0, 0}, clo = {0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < 8; st++) {
      chi = mfma(xa[st], o.bh[st], chi);
      clo = mfma(xa[st], o.bl[st], clo);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) res[r] = o.d * __builtin_fmaf(16.0f, chi[r], clo[r]);
  } else {
    DecKQ o;
    if constexpr (FMT == CQ_Q4_K) decode_q4k(f, g, o);
    else decode_q5k(f, g, o);
    const h8 bm0 = mk_h8(o.um0, o.um0, o.um0, o.um0), bm1 = mk_h8(o.um1, o.um1, o.um1, o.um1);
    f4 c = {0, 0, 0, 0}, cm = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; s++) {
      c = mfma(xa[s], o.b[s], c);
      cm = mfma(xa[s], s < 4 ? bm0 : bm1, cm);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) res[r] = __builtin_fmaf(-o.dmin, cm[r], o.d * c[r]);
  }
  return res;
}

// Grid: x = ceil(N / (16 NT)).  Block: 64 * NW threads, NW <= units and
// NW <= GVD_MAX_WAVES (checked by the host).
template <int FMT, int YT, int NT, int D>
__device__ __forceinline__ void gemvd_body(const GvdArgs& a) {
  typedef FmtTraits<FMT> T;
  typedef typename T::Frag Frag;
  __shared__ float red[GVD_MAX_WAVES][4][64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const uint8_t* wr[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) wr[t] = a.w + (size_t)min(n0 + 16 * t + j, a.N - 1) * a.row_bytes;
  // byte offsets of x fit 31 bits (checked on the host)
  const uint8_t* xr = (const uint8_t*)a.x + 2u * (uint32_t)(min(j, a.M - 1) * a.K + gvd_abase<FMT>(g));
  const int mine = (a.units - 1 - wave) / nw + 1;  // this wave's superblocks (wave < units)

  Frag f[D][NT];
  h8 xa[D][8];
  auto load = [&](int d, int i) {
    const int u = wave + nw * min(i, mine - 1);  // past the end: reload the last, its result is dropped
#pragma unroll
    for (int t = 0; t < NT; t++) load_unit<FMT>(f[d][t], wr[t] + (size_t)u * T::bytes, g, 0);
    const uint8_t* xp = xr + (uint32_t)u * 512u;
#pragma unroll
    for (int s = 0; s < 8; s++) xa[d][s] = __builtin_bit_cast(h8, ld_u128(xp + 2 * gvd_aoff<FMT>(s)));
  };
  f4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = f4{0, 0, 0, 0};
#pragma unroll
  for (int d = 0; d < D; d++) load(d, d);
  for (int i = 0; i < mine; i += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const bool live = i + d < mine;  // uniform; a dead slot's result is discarded by a select
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const f4 p = gvd_superblock<FMT>(f[d][t], xa[d], g);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = live ? acc[t][r] + p[r] : acc[t][r];
      }
      load(d, i + d + D);
    }
  }
  // Cross-wave sum in wave order, one row tile at a time.
#pragma unroll
  for (int t = 0; t < NT; t++) {
    if (t > 0) __syncthreads();  // previous tile's sums have been read
#pragma unroll
    for (int r = 0; r < 4; r++) red[wave][r][lane] = acc[t][r];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256; idx += blockDim.x) {
      const int r = idx >> 6, ln = idx & 63;
      float s = red[0][r][ln];
      for (int w2 = 1; w2 < nw; w2++) s += red[w2][r][ln];
      const int m = 4 * (ln >> 4) + r, n = n0 + 16 * t + (ln & 15);
      if (m < a.M && n < a.N) cq_store<YT>(a.y, a.epi, s, (size_t)m * a.N + n, n);
    }
  }
}

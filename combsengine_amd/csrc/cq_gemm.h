// Prefill dequant-GEMM over K-quant weights on CDNA4 MFMA:
//   y[m, n] = sum_k x[m, k] * W[n, k],  m >= 17 (chunked prefill).
// Replaces the reference's tiled/untiled fused kernels for m > 1
// (engine/core/combs-models/src/qmatmul.rs:939-993 for Q4_K; Q5_K/Q6_K ran
// their untiled kernels, :1064-1117, :1184-1229).
//
// Work mapping.  A workgroup owns 16*nw weight rows (one 16-row tile per
// wave) and a block of MB = 16*MT activation rows.  It walks K one 256-value
// superblock at a time:
//   - the activation chunk x[m0 .. m0+MB)[256 values] is double-buffered in
//     LDS (row pitch 264 halves, so the 16 rows an MFMA reads fall in
//     distinct banks), together with per-row sums of each 32-value sub-block
//     (as fp16 hi + lo) for the K-quant min term;
//   - each wave decodes its tile's superblock once into exact fp16 MFMA B
//     operands (q*sc) and reuses them for all MT activation tiles;
//   - the next superblock's weights (registers) and activations (registers,
//     then LDS) are loaded while the current one is computed.
// Per superblock and tile: y += d * C - dmin * Cmin, with Cmin one MFMA of
// the sub-block sums against the 6-bit mins.  Q6_K: y += d * (16 Chi + Clo).
#pragma once
#include "cq_gemv.h"

struct GemmArgs {
  const uint8_t* w;
  const void* x;
  void* y;
  long long row_bytes;
  int M, N, K;
  int units;  // superblocks per row
  CqEpi epi;
};

#define GM_KC 256           // K values per step (one superblock)
#define GM_XP GM_KC         // LDS row pitch of the activation chunk (halves)
#define GM_XS_REG 8         // 16-byte activation vectors a thread stages per step

// LDS bank swizzle of the activation chunk.  Row r keeps its 16-byte chunk c
// at position c ^ gm_sw(r).  An MFMA A read is served 32 lanes at a time on
// gfx950 (16 rows x 2 k-groups whose chunks differ by 8); gm_sw takes 16
// values whose pairwise XOR never equals 8, so those 32 reads land on 32
// distinct 16-byte bank groups of the 512-byte LDS row.
__device__ __forceinline__ int gm_sw(int r) { return (r & 7) | ((r & 8) << 1); }

template <int XT>
struct GmStage {
  u4v v[GM_XS_REG][XT ? 2 : 1];
};

// Issue the global loads of activation chunk [kc0, kc0+256) for rows
// m0 .. m0+MB (rows past M re-read row M-1; their outputs are never stored).
template <int XT, int MB>
__device__ __forceinline__ void gm_issue(const GemmArgs& a, GmStage<XT>& st, int m0, int kc0) {
  constexpr int total = MB * (GM_KC / 8);
#pragma unroll
  for (int q = 0; q < GM_XS_REG; q++) {
    const int i = threadIdx.x + q * blockDim.x;
    if (i < total) {
      const int r = i >> 5, v = i & 31;
      const int m = min(m0 + r, a.M - 1);
      const uint32_t src = (uint32_t)(m * a.K + kc0 + 8 * v) * (XT ? 4u : 2u);
      st.v[q][0] = ld_u128((const uint8_t*)a.x + src);
      if (XT) st.v[q][XT] = ld_u128((const uint8_t*)a.x + src + 16);
    }
  }
}

// Convert and store a staged chunk; also the sub-block sums (4 consecutive
// threads hold the 4 vectors of one 32-value sub-block of one row).
template <int XT, int MB>
__device__ __forceinline__ void gm_commit(const GmStage<XT>& st, _Float16 (*xh)[GM_XP], _Float16 (*xl)[GM_XP],
                                          _Float16 (*xsum)[16]) {
  constexpr int total = MB * (GM_KC / 8);
#pragma unroll
  for (int q = 0; q < GM_XS_REG; q++) {
    const int i = threadIdx.x + q * blockDim.x;
    if (q * (int)blockDim.x >= total) break;  // later slots are empty for every thread
    h8 vh, vl;
    float sum;
    if (!XT) {
      vh = __builtin_bit_cast(h8, st.v[q][0]);
      // exact products by 1.0, f32 accumulation (v_dot2_f32_f16)
      const h2 one = {1, 1};
      sum = __builtin_amdgcn_fdot2(as_h2(st.v[q][0].x), one, 0.0f, false);
      sum = __builtin_amdgcn_fdot2(as_h2(st.v[q][0].y), one, sum, false);
      sum = __builtin_amdgcn_fdot2(as_h2(st.v[q][0].z), one, sum, false);
      sum = __builtin_amdgcn_fdot2(as_h2(st.v[q][0].w), one, sum, false);
    } else {
      float f[8];
      __builtin_memcpy(f, &st.v[q][0], 16);
      __builtin_memcpy(f + 4, &st.v[q][XT], 16);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        vh[e] = (_Float16)f[e];
        vl[e] = (_Float16)(f[e] - (float)vh[e]);
      }
      sum = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
    }
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if (i < total) {
      const int r = i >> 5, v = i & 31;
      const int pv = 8 * (v ^ gm_sw(r & 15));
      *(h8*)&xh[r][pv] = vh;
      if (XT) *(h8*)&xl[r][pv] = vl;
      if ((v & 3) == 0) {
        const _Float16 hi = (_Float16)sum;
        xsum[r][2 * (v >> 2)] = hi;
        xsum[r][2 * (v >> 2) + 1] = (_Float16)(sum - (float)hi);
      }
    }
  }
}

// Min-term B operand for lane group g: k index = 2*sb + part over sub-blocks
// sb = 4g .. 4g+3 (groups 0, 1), zeros for groups 2, 3.
__device__ __forceinline__ h8 kq_min_operand(const u4v& hdr, int g) {
  uint32_t u[4] = {0, 0, 0, 0};
  if (g < 2) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t sc, mn;
      scale_min_k4(4 * g + i, hdr.y, hdr.z, hdr.w, sc, mn);
      u[i] = as_u32(hsplat((float)mn));
    }
  }
  return mk_h8(u[0], u[1], u[2], u[3]);
}

template <int FMT, int XT, int YT>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
  constexpr int MT = XT ? 2 : 4;  // activation tiles per workgroup
  constexpr int MB = 16 * MT;
  typedef typename FmtTraits<FMT>::Frag Frag;
  __shared__ __attribute__((aligned(16))) _Float16 xh[2][MB][GM_XP];
  __shared__ __attribute__((aligned(16))) _Float16 xl[XT ? 2 : 1][XT ? MB : 1][GM_XP];
  __shared__ __attribute__((aligned(16))) _Float16 xsum[2][MB][16];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * nw + wave) * 16;
  const int m0 = blockIdx.y * MB;
  const int row = min(n0 + j, a.N - 1);
  const uint8_t* wr = a.w + (size_t)row * a.row_bytes;
  f4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = f4{0, 0, 0, 0};
  // swizzled column (halves) of this lane's 8 A values for each MFMA step
  const int swj = gm_sw(j);
  int acol[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const int c = (FMT == CQ_Q6_K) ? q6k_koff(g, s) / 8 : 8 * g + s;
    acol[s] = 8 * (c ^ swj);
  }

  GmStage<XT> st;
  gm_issue<XT, MB>(a, st, m0, 0);
  Frag cur, nxt;
  load_unit<FMT>(cur, wr, g, 0);
  gm_commit<XT, MB>(st, xh[0], xl[0], xsum[0]);
  __syncthreads();

  for (int u = 0; u < a.units; u++) {
    const int b = u & 1;
    const bool more = u + 1 < a.units;
    if (more) {
      gm_issue<XT, MB>(a, st, m0, (u + 1) * GM_KC);
      load_unit<FMT>(nxt, wr + (size_t)(u + 1) * FmtTraits<FMT>::bytes, g, 0);
    }
    const _Float16(*xb)[GM_XP] = xh[b];
    const _Float16(*xbl)[GM_XP] = xl[XT ? b : 0];
    // Steps outer, activation tiles inner: the MT accumulation chains are
    // independent, so consecutive MFMAs never wait on each other.
    if constexpr (FMT == CQ_Q6_K) {
      DecQ6 o;
      decode_q6k(cur, g, o);
      f4 chi[MT], clo[MT];
#pragma unroll
      for (int t = 0; t < MT; t++) chi[t] = clo[t] = f4{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < 8; s++) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const h8 av = *(const h8*)&xb[16 * t + j][acol[s]];
          chi[t] = mfma(av, o.bh[s], chi[t]);
          clo[t] = mfma(av, o.bl[s], clo[t]);
          if (XT) {
            const h8 al = *(const h8*)&xbl[16 * t + j][acol[s]];
            chi[t] = mfma(al, o.bh[s], chi[t]);
            clo[t] = mfma(al, o.bl[s], clo[t]);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[t][r] = __builtin_fmaf(o.d, __builtin_fmaf(16.0f, chi[t][r], clo[t][r]), acc[t][r]);
    } else {
      DecKQ o;
      if constexpr (FMT == CQ_Q4_K) decode_q4k(cur, g, o);
      else decode_q5k(cur, g, o);
      const h8 bmin = kq_min_operand(cur.hdr, g);
      const h8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
      f4 c[MT];
#pragma unroll
      for (int t = 0; t < MT; t++) c[t] = f4{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < 8; s++) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
          c[t] = mfma(*(const h8*)&xb[16 * t + j][acol[s]], o.b[s], c[t]);
          if (XT) c[t] = mfma(*(const h8*)&xbl[16 * t + j][acol[s]], o.b[s], c[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const h8 as = g < 2 ? *(const h8*)&xsum[b][16 * t + j][8 * g] : zero;
        const f4 cm = mfma(as, bmin, f4{0, 0, 0, 0});
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = __builtin_fmaf(-o.dmin, cm[r], __builtin_fmaf(o.d, c[t][r], acc[t][r]));
      }
    }
    if (more) {
      gm_commit<XT, MB>(st, xh[b ^ 1], xl[XT ? (b ^ 1) : 0], xsum[b ^ 1]);
      cur = nxt;
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < MT; t++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = m0 + 16 * t + 4 * g + r, n = n0 + j;
      if (m < a.M && n < a.N) cq_store<YT>(a.y, a.epi, acc[t][r], (size_t)m * a.N + n, n);
    }
  }
}

// Prefill dequant-GEMM for the 32-value block formats (Q4_0, Q5_0, Q8_0,
// Q4_1, Q5_1), fp16 activations (cq_gemml_*): y[m, n] = sum_k x[m, k] * W[n, k].
// Replaces the reference's tiled Q8_0 kernel (qmatmul.rs:481-527, chosen for
// m > 1 at :701-703) and its untiled Q4_0 / Q5_0 kernels for prefill.
//
// Work mapping (the prefill GEMM's, cq_gemm2.h, at block granularity):
//   - workgroup: 4 waves x NT 16-row weight tiles each, x 128 activation rows
//     (MT = 8 tiles of 16; 64 rows, MT = 4, for short prefills); a step is
//     four 32-value blocks (128 K values);
//   - the activation chunk of a step (16*MT rows x 128 halves, 32 KB at MT = 8) arrives
//     by global_load_lds one step ahead into the other of two LDS buffers;
//     16-byte chunk c of row r is stored in slot c ^ (r & 15), so the 16
//     rows of an A-fragment read hit 16 distinct bank groups;
//   - each wave decodes its NT tiles' blocks from registers into exact fp16
//     MFMA operands (the decode GEMV's, cq_gemv.h legacy_b) and reuses each
//     for MT MFMAs, one per activation tile;
//   - a block's MFMA starts from zero and its fp32 result is scaled by the
//     block's fp16 d into the accumulator (every 32 K values carry their own
//     scale, so nothing can be folded into the operands exactly); Q4_1 /
//     Q5_1 add m * sum(x of the block), the sum by one more MFMA against B = 1
//     (once per activation tile, shared by the NT weight tiles);
//   - when the tile grid leaves compute units idle (few weight rows or
//     activation rows), the steps are split over blockIdx.z; each slice
//     writes fp32 partials and cq_splitk_reduce_* sums them in slice order.
#pragma once
#include <type_traits>
#include "cq_gemm2.h"

struct LgArgs {
  const uint8_t* w;    // packed blocks, [N rows][row_bytes]
  const _Float16* x;   // [M][K]
  void* y;             // [M][N] fp32 or fp16 (no split)
  float* part;         // split: [slices][M][N] fp32 partial sums, else null
  long long row_bytes;
  int M, N, K, blocks; // blocks = K / 32
  int ssteps;          // steps (4 blocks) per slice (blockIdx.z)
  CqEpi epi;
};

#define LG_KC 128  // K values per step (four blocks)

template <int FMT>
constexpr bool lg_affine() {
  return FMT == CQ_Q4_1 || FMT == CQ_Q5_1;
}

template <int FMT, int YT, int NT, int NW, int MT = 8>
__device__ __forceinline__ void gemml_body(const LgArgs& a) {
  typedef FmtTraits<FMT> T;  // unit = LB = 4 blocks = one step
  typedef typename T::Frag Frag;
  constexpr int BB = T::bytes / LB;  // bytes per block
  __shared__ __attribute__((aligned(16))) _Float16 lg_x0[16 * MT * LG_KC];
  __shared__ __attribute__((aligned(16))) _Float16 lg_x1[16 * MT * LG_KC];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  int bx, by;
  lt_tile(bx, by);
  const int n0 = (bx * NW + wave) * 16 * NT;
  const int m0 = by * 16 * MT;
  const uint8_t* wr[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) wr[t] = a.w + (size_t)min(n0 + 16 * t + j, a.N - 1) * (size_t)a.row_bytes;
  f4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int tm = 0; tm < MT; tm++) acc[t][tm] = f4{0, 0, 0, 0};

  // Activation DMA: instruction I = wave + NW ii moves rows 4I .. 4I+3; lane
  // (row r = 4I + (lane >> 4), slot v = lane & 15) fetches the row's chunk
  // v ^ (r & 15).  Rows >= M re-read row M - 1, chunks past K re-read the
  // row's last chunk (neither is used).
  const int steps = (a.blocks + LB - 1) / LB;
  const int st0 = (int)blockIdx.z * a.ssteps, st1 = min(steps, st0 + a.ssteps);  // this slice's steps
  auto dma_x = [&](_Float16* buf, int step) {
#pragma unroll
    for (int ii = 0; ii < 4 * MT / NW; ii++) {
      const int I = wave + NW * ii;
      const int r = 4 * I + (lane >> 4);
      const int c = (lane & 15) ^ (r & 15);
      const int col = min(LG_KC * step + 8 * c, a.K - 8);
      const _Float16* src = a.x + (size_t)min(m0 + r, a.M - 1) * a.K + col;
      __builtin_amdgcn_global_load_lds((lt_glb_t*)src, (lt_lds_t*)(buf + I * 512), 16, 0, 0);
    }
  };
  Frag cur[NT], nxt[NT];
  auto load_w = [&](Frag* f, int step) {
    const int nb = min(LB, a.blocks - LB * step);
#pragma unroll
    for (int t = 0; t < NT; t++) load_unit<FMT>(f[t], wr[t] + (size_t)step * LB * BB, g, nb);
  };
  // A fragment of block i, activation tile tm: row 16 tm + j, halves
  // (32 i + 4g .. +3, 32 i + 16 + 4g .. +3), or 32 i + 8g .. +7 for Q8_0.
  auto afrag = [&](const _Float16* buf, int tm, int i) {
    const _Float16* row = buf + (16 * tm + j) * LG_KC;
    if constexpr (FMT == CQ_Q8_0) {
      const int c = 4 * i + g;
      return *(const h8*)(row + 8 * (c ^ j));
    } else {
      const int c0 = 4 * i + (g >> 1), c1 = 4 * i + 2 + (g >> 1), o = 4 * (g & 1);
      const h4 p = *(const h4*)(row + 8 * (c0 ^ j) + o), q = *(const h4*)(row + 8 * (c1 ^ j) + o);
      return (h8)__builtin_shufflevector(p, q, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  dma_x(lg_x0, st0);
  load_w(cur, st0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const uint32_t ones = 0x3C003C00u;
  const h8 bones = mk_h8(ones, ones, ones, ones);
  for (int step = st0; step < st1; step++) {
    const _Float16* xc = ((step - st0) & 1) ? lg_x1 : lg_x0;
    _Float16* xn = ((step - st0) & 1) ? lg_x0 : lg_x1;
    const bool more = step + 1 < st1;
    if (more) {
      dma_x(xn, step + 1);
      load_w(nxt, step + 1);
    }
    const int nb = min(LB, a.blocks - LB * step);
#pragma unroll
    for (int i = 0; i < LB; i++) {
      if (i >= nb) break;
      h8 b[NT];
      float d[NT], mm[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        b[t] = legacy_b(cur[t], i, g);
        const uint32_t dw = legacy_d(cur[t], i);
        d[t] = f16_bits_to_f32(dw);
        mm[t] = f16_bits_to_f32(dw >> 16);
      }
#pragma unroll
      for (int tm = 0; tm < MT; tm++) {
        const h8 av = afrag(xc, tm, i);
        f4 sx = {0, 0, 0, 0};
        if constexpr (lg_affine<FMT>()) sx = mfma(av, bones, f4{0, 0, 0, 0});
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const f4 c = mfma(av, b[t], f4{0, 0, 0, 0});
#pragma unroll
          for (int r = 0; r < 4; r++) acc[t][tm][r] = __builtin_fmaf(d[t], c[r], acc[t][tm][r]);
          if constexpr (lg_affine<FMT>()) {
#pragma unroll
            for (int r = 0; r < 4; r++) acc[t][tm][r] = __builtin_fmaf(mm[t], sx[r], acc[t][tm][r]);
          }
        }
      }
    }
    if (more) {
#pragma unroll
      for (int t = 0; t < NT; t++) cur[t] = nxt[t];
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
  }
  // bias / gated epilogue: the activation chosen once, the values loaded
  // ahead of the stores (cq_store_tiles_epi)
  if (!a.part && (a.epi.bias || a.epi.aux)) {
    float one[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) one[t] = 1.0f;
    if (cq_store_tiles_epi<YT, NT, MT>(a.epi, a.y, a.M, a.N, m0, n0, g, j, acc, one)) return;
  }
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int tm = 0; tm < MT; tm++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * tm + 4 * g + r, n = n0 + 16 * t + j;
        if (m < a.M && n < a.N) {
          if (a.part) a.part[((size_t)blockIdx.z * a.M + m) * a.N + n] = acc[t][tm][r];
          else cq_store<YT>(a.y, a.epi, acc[t][tm][r], (size_t)m * a.N + n, n);
        }
      }
}

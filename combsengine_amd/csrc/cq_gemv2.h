// Decode GEMV for a single fp16 activation row, streaming variant for the
// K-quants:  y[n] = sum_k x[k] * W[n, k].
//
// Why a second single-row kernel: cq_gemv1 gives each lane a whole superblock
// (144-210 bytes), so a wave task is 9-13 KB and a wave holds only one or two
// tasks of a 33 MB weight.  The last task's arithmetic then runs after the
// weight stream has ended, and that tail is a large part of the launch.
// Here the unit of work is a quarter superblock per lane:
//   - lane l of a wave takes quarter p = l & 3 of superblock slot s = l >> 2:
//     Q4_K / Q5_K: the 64-value group p (sub-blocks 2p, 2p+1), i.e. the
//       16-byte header (+ the 32 qh bytes for Q5_K) and qs bytes [32p, 32p+32);
//     Q6_K: half h = p >> 1, ql column c = p & 1: ql bytes 64h + 32c .. +32
//       (values 128h + 32c + l and 128h + 32(c+2) + l), the half's 32 qh
//       bytes, its 8 scales and d;
//   - a step is 16 superblocks: the next 16 of one row (rows of more than 16
//     superblocks take several steps), or R = 16 / units whole rows when
//     units is a power of two below 16 (otherwise one shorter row);
//   - each wave owns a contiguous range of rows (balanced to within one row)
//     and streams its steps with the weight loads D steps ahead of the
//     arithmetic, in a ring of D register buffers; the last step's arithmetic
//     is small, so the tail after the stream is short;
//   - the activation row is staged once per workgroup in LDS as three int8
//     parts (Gv1XStage), and the inner products are exact int32 v_dot4
//     sums, as in cq_gemv1;
//   - per-lane partial sums accumulate over a row's steps and are reduced
//     across the wave (fixed order, deterministic) when the row is done.
// Replaces qmatmul.rs:881-930 (Q4_K), :1064-1117 (Q5_K), :1184-1229 (Q6_K)
// for m = 1.
#pragma once
#include "cq_gemv1.h"

struct Gv2Args {
  const uint8_t* w;
  const _Float16* x;
  void* y;
  long long row_bytes;  // units * block bytes
  int N, K, units;
  int R;                // rows per step: 16 / units for units = 1, 2, 4, 8; else 1
  int C;                // steps per row (ceil(units / 16)), 1 when R > 1
  int cinv;             // ceil(65536 / C): step / C = (step * cinv) >> 16
  int waves;            // waves in the grid
  CqEpi epi;
};

// Per-lane weight bytes of one step, as 16-byte chunks (+ a 16-bit tail).
template <int FMT> struct Gv2Frag;
template <> struct Gv2Frag<CQ_Q4_K> {
  u4v hd, q0, q1;
  __device__ __forceinline__ void load(const uint8_t* sb, int p) {
    hd = ld_u128(sb);
    q0 = ld_u128(sb + 16 + 32 * p);
    q1 = ld_u128(sb + 32 + 32 * p);
  }
};
template <> struct Gv2Frag<CQ_Q5_K> {
  u4v hd, h0, h1, q0, q1;
  __device__ __forceinline__ void load(const uint8_t* sb, int p) {
    hd = ld_u128(sb);
    h0 = ld_u128(sb + 16);
    h1 = ld_u128(sb + 32);
    q0 = ld_u128(sb + 48 + 32 * p);
    q1 = ld_u128(sb + 64 + 32 * p);
  }
};
template <> struct Gv2Frag<CQ_Q6_K> {
  u4v l0, l1, h0, h1;
  u2v sc;
  uint32_t d;
  __device__ __forceinline__ void load(const uint8_t* sb, int p) {
    const int hh = p >> 1, c = p & 1;
    l0 = ld_u128(sb + 64 * hh + 32 * c);
    l1 = ld_u128(sb + 64 * hh + 32 * c + 16);
    h0 = ld_u128(sb + 128 + 32 * hh);
    h1 = ld_u128(sb + 128 + 32 * hh + 16);
    sc = ld_u64(sb + 192 + 8 * hh);
    d = ld_u16(sb + 208);
  }
};

__device__ __forceinline__ float gv2_combine(int ih, int il, int ie) {
  // |il| * 254 + |ie| stays far inside int32: combine exactly, then convert once
  return __builtin_fmaf((float)(254 * il + ie), 1.0f / 64516.0f, (float)ih);
}

// Partial dot product of quarter p of a superblock of unit u with the staged
// activations (ux: byte offset u * GV1_XSTRIDE; xb: 32-value block index of
// the unit's first value).
template <int FMT>
__device__ __forceinline__ float gv2_quarter(const Gv2Frag<FMT>& f, int p, int ux, int xb) {
  if constexpr (FMT == CQ_Q4_K || FMT == CQ_Q5_K) {
    // group p: sub-block 2p = low nibbles of qs[32p .. 32p+32), 2p+1 = high
    uint32_t sc0, m0, sc1, m1;
    scale_min_k4(2 * p, f.hd.y, f.hd.z, f.hd.w, sc0, m0);
    scale_min_k4(2 * p + 1, f.hd.y, f.hd.z, f.hd.w, sc1, m1);
    const int8_t* xh = gv_xh + ux + 64 * p;
    const int8_t* xl = gv_xl + ux + 64 * p;
    const int8_t* xe = gv_xe + ux + 64 * p;
    int ih0 = 0, il0 = 0, ie0 = 0, ih1 = 0, il1 = 0, ie1 = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {  // qs bytes [16h, 16h+16): values 16h .. 16h+15
      const u4v q = h ? f.q1 : f.q0;
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
      const u4v h0 = *(const u4v*)(xh + 16 * h), l0 = *(const u4v*)(xl + 16 * h), e0 = *(const u4v*)(xe + 16 * h);
      const u4v h1 = *(const u4v*)(xh + 32 + 16 * h), l1 = *(const u4v*)(xl + 32 + 16 * h),
                e1 = *(const u4v*)(xe + 32 + 16 * h);
      const uint32_t xh0[4] = {h0.x, h0.y, h0.z, h0.w}, xl0[4] = {l0.x, l0.y, l0.z, l0.w};
      const uint32_t xe0[4] = {e0.x, e0.y, e0.z, e0.w};
      const uint32_t xh1[4] = {h1.x, h1.y, h1.z, h1.w}, xl1[4] = {l1.x, l1.y, l1.z, l1.w};
      const uint32_t xe1[4] = {e1.x, e1.y, e1.z, e1.w};
      uint32_t hb[4] = {0, 0, 0, 0};
      if constexpr (FMT == CQ_Q5_K) {
        const u4v qh = h ? f.h1 : f.h0;
        hb[0] = qh.x; hb[1] = qh.y; hb[2] = qh.z; hb[3] = qh.w;
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
        if constexpr (FMT == CQ_Q5_K) {
          // 5th bits: qh bit 2p (low values), 2p+1 (high values) -> bit 4 of each byte
          lo |= ((hb[i] >> (2 * p)) & 0x01010101u) << 4;
          hi |= ((hb[i] >> (2 * p + 1)) & 0x01010101u) << 4;
        }
        ih0 = dot4(lo, xh0[i], ih0);
        il0 = dot4(lo, xl0[i], il0);
        ie0 = dot4(lo, xe0[i], ie0);
        ih1 = dot4(hi, xh1[i], ih1);
        il1 = dot4(hi, xl1[i], il1);
        ie1 = dot4(hi, xe1[i], ie1);
      }
    }
    const float d = f16_bits_to_f32(f.hd.x), dmin = f16_bits_to_f32(f.hd.x >> 16);
    const int b0 = xb + 2 * p;
    float acc = (float)sc0 * gv_xs[b0] * gv2_combine(ih0, il0, ie0);
    acc = __builtin_fmaf((float)sc1 * gv_xs[b0 + 1], gv2_combine(ih1, il1, ie1), acc);
    const float macc = __builtin_fmaf((float)m0, gv_s[b0], (float)m1 * gv_s[b0 + 1]);
    return d * acc - dmin * macc;
  } else {
    // Q6_K (gguf.rs:968-999): half hh, ql column c; quadrant t = c (low
    // nibbles, qh bits 2c) and t = c + 2 (high nibbles, qh bits 2c + 4).
    // Value (hh, t, l) = (q - 32) * sc[8hh + l/16 + 2t]; the -32 is applied
    // as -32 * sum(x) per 16-value group.
    const int hh = p >> 1, c = p & 1;
    const uint32_t scw[2] = {f.sc.x, f.sc.y};
    const uint32_t lw[8] = {f.l0.x, f.l0.y, f.l0.z, f.l0.w, f.l1.x, f.l1.y, f.l1.z, f.l1.w};
    const uint32_t hw[8] = {f.h0.x, f.h0.y, f.h0.z, f.h0.w, f.h1.x, f.h1.y, f.h1.z, f.h1.w};
    float acc = 0.0f, cacc = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
      const int t = c + 2 * tt;
      const int ko = ux + 64 * (2 * hh + c) + 32 * tt;  // staged byte offset of this quadrant (permuted layout)
      int ih[2] = {0, 0}, il[2] = {0, 0}, ie[2] = {0, 0};
#pragma unroll
      for (int g = 0; g < 2; g++) {  // 16-value group l/16
        const u4v xh = *(const u4v*)(gv_xh + ko + 16 * g), xl = *(const u4v*)(gv_xl + ko + 16 * g),
                  xe = *(const u4v*)(gv_xe + ko + 16 * g);
        const uint32_t xhw[4] = {xh.x, xh.y, xh.z, xh.w}, xlw[4] = {xl.x, xl.y, xl.z, xl.w};
        const uint32_t xew[4] = {xe.x, xe.y, xe.z, xe.w};
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {  // 4 values l = 16g + 4jj ..
          const int j = 4 * g + jj;
          const uint32_t q = ((lw[j] >> (4 * tt)) & 0x0F0F0F0Fu) | (((hw[j] >> (2 * t)) & 0x03030303u) << 4);
          ih[g] = dot4(q, xhw[jj], ih[g]);
          il[g] = dot4(q, xlw[jj], il[g]);
          ie[g] = dot4(q, xew[jj], ie[g]);
        }
      }
      const float sblk = gv_xs[xb + 4 * hh + t];
#pragma unroll
      for (int g = 0; g < 2; g++) {
        const int si = g + 2 * t;  // scale index within the half
        const float scf = (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
        acc = __builtin_fmaf(scf * sblk, gv2_combine(ih[g], il[g], ie[g]), acc);
        cacc = __builtin_fmaf(scf, gv_s16[2 * xb + 8 * hh + 2 * t + g], cacc);
      }
    }
    return f16_bits_to_f32(f.d) * __builtin_fmaf(-32.0f, cacc, acc);
  }
}

template <int FMT>
constexpr int gv2_block_bytes() {
  return FMT == CQ_Q4_K ? 144 : FMT == CQ_Q5_K ? 176 : 210;
}

// Grid: one workgroup of NW waves per slot (up to a few per compute unit);
// wave w of the grid owns rows [w N / W, (w + 1) N / W).  EPI = 1 applies
// the output epilogue, its bias / gate values for the wave's first 64 rows
// loaded (lane l: row row0 + l) before anything else.
template <int FMT, int YT, int NW, int D, int EPI>
__device__ __forceinline__ void gemv2_body(const Gv2Args& a) {
  constexpr int BB = gv2_block_bytes<FMT>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wg = blockIdx.x * NW + wave;
  const int row0 = (int)(((long long)wg * a.N) / a.waves);
  const int row1 = (int)(((long long)(wg + 1) * a.N) / a.waves);
  const int nrows = row1 - row0;
  const int nsteps = a.R > 1 ? (nrows + a.R - 1) / a.R : nrows * a.C;
  const int s = lane >> 2, p = lane & 3;
  // R > 1: the lane's row within the step and its unit are fixed
  const int rr = a.R > 1 ? s / a.units : 0;
  const int ur = a.R > 1 ? s - rr * a.units : 0;
  // Lane's superblock for step st (clamped to a valid one; the caller skips
  // the arithmetic of slots that are not real).
  auto slot = [&](int st, int& row, int& u) -> bool {
    if (a.R > 1) {
      row = row0 + st * a.R + rr;
      u = ur;
      return rr < a.R && row < row1;
    }
    const int q = (int)(((uint32_t)st * (uint32_t)a.cinv) >> 16);  // st / C
    row = row0 + q;
    u = 16 * (st - q * a.C) + s;
    return u < a.units;
  };
  auto ptr = [&](int st) {
    int row, u;
    st = max(0, min(st, nsteps - 1));  // (prologue only: waves with fewer than D steps)
    const bool ok = slot(st, row, u);
    row = min(row, a.N - 1);  // (a wave without rows loads row N - 1 and never uses it)
    u = ok ? u : a.units - 1;
    return a.w + (size_t)row * a.row_bytes + (size_t)u * BB;
  };

  float pb = 0.0f, pa = 0.0f;
  if constexpr (EPI) {
    const int r = min(row0 + lane, a.N - 1);
    pb = cq_epi_bias(a.epi, r);
    pa = cq_epi_aux(a.epi, r);
  }
  Gv1XStage<NW, FMT == CQ_Q6_K> xst;
  xst.issue(a.x, a.K);
  Gv2Frag<FMT> f[D];
  // (unconditional, so that the staging below waits for the x loads only)
#pragma unroll
  for (int d = 0; d < D; d++) f[d].load(ptr(d), p);
  __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the staging
  xst.commit(a.K);
  __syncthreads();
  if (nsteps <= 0) return;

  float acc = 0.0f;
  // Output of row `row` (j = row - row0), the epilogue's values from lane j;
  // called by every lane (the shuffles need them), stored by `leader`.
  auto finish = [&](float v, int row, bool leader) {
    if constexpr (EPI) {
      const int j = row - row0;
      float b = __shfl(pb, j & 63, 64), u = __shfl(pa, j & 63, 64);
      if (j >= 64) {
        b = cq_epi_bias(a.epi, min(row, a.N - 1));
        u = cq_epi_aux(a.epi, min(row, a.N - 1));
      }
      v = cq_epi_apply<YT>(a.epi, v, b, u);
    }
    if (leader) cq_store_raw<YT>(a.y, v, row);
  };
  // Arithmetic of step st from buffer fb, then the row bookkeeping.
  auto step = [&](const Gv2Frag<FMT>& fb, int st) {
    int row, u;
    const bool ok = slot(st, row, u);
    if (ok) acc += gv2_quarter<FMT>(fb, p, u * GV1_XSTRIDE, 8 * u);
    if (a.R > 1) {
      // R rows of `units` superblocks: reduce within each group of 4 units lanes
      const float v = lane_group_sum(acc, 4 * a.units);
      finish(v, row, ok && (lane & (4 * a.units - 1)) == 0);
      acc = 0.0f;
    } else if (16 * (st - (int)(((uint32_t)st * (uint32_t)a.cinv) >> 16) * a.C) + 16 >= a.units) {
      // last step of this row: reduce the whole wave
      const float v = lane_group_sum(acc, 64);
      finish(v, row, lane == 0);
      acc = 0.0f;
    }
  };
  // Steady state: every buffer is refilled D steps ahead, no conditions on
  // the loads (so the load counters stay exact); then the last < 2D steps.
  int i = 0;
  for (; i + 2 * D <= nsteps; i += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      step(f[d], i + d);
      f[d].load(ptr(i + d + D), p);
    }
  }
#pragma unroll
  for (int d = 0; d < D; d++) {
    if (i + d < nsteps) step(f[d], i + d);
    if (i + d + D < nsteps) f[d].load(ptr(i + d + D), p);
  }
#pragma unroll
  for (int d = 0; d < D; d++)
    if (i + D + d < nsteps) step(f[d], i + D + d);
}

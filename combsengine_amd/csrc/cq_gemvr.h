// Decode GEMV for one fp16 activation row, rows split across the lanes of a
// wave (cq_gemvr_*): y[n] = sum_k x[k] * W[n, k].
//
// Work mapping.  A row's superblocks are cut into quarters of 64 values (a
// K-quant superblock's sub-block pair: 32 qs bytes and the 16-byte header);
// quarter s of a row belongs to lane s % 64 of wave s / 64 of a row group of
// C = ceil(4 units / 64) waves.  Each lane keeps its quarter's 64
// activations in 32 registers for the whole launch, and a wave walks its
// row group's rows one after another, D rows of loads in flight: three
// 16-byte loads per lane and row, which together read the row's bytes
// contiguously (measured at the speed of a flat read of the same bytes).
// Compared with one superblock per lane (cq_gemv1), the activation set-up is
// a quarter as large, a row is 1/4 of a task, and no LDS hand-over of the
// weights is needed.
//
// Row sums: each lane's partial goes into a batch of RB = 4 rows, which a
// transposed butterfly reduces across the 64 lanes (7 cross-lane adds per 4
// rows); with C > 1 the waves of a row group add their partials in LDS in
// wave order, so a row's result does not depend on the grid.
// Replaces qmatmul.rs:881-930 (q4_k_matmul_kernel) for m = 1.
#pragma once
#include "cq_gemv1.h"

struct GvrArgs {
  const uint8_t* w;
  const _Float16* x;
  void* y;
  long long row_bytes;
  int N, K, units;
  int C;        // waves per row group: ceil(4 units / 64)
  int G;        // row groups per workgroup
  int iters;    // rows per row group: ceil(N / (gridDim.x * G))
  CqEpi epi;
};

#define GVR_RB 4          // rows per reduction batch
#define GVR_XSTRIDE 72    // halves per staged 64-value quarter (64 + 8 pad: spreads the quarter reads over the banks)
#define GVR_MAXK 32768
#define GVR_MAXW 8        // waves per workgroup


// The 4 values of a batch summed over the 64 lanes: afterwards lane l holds
// the total of row ((l >> 5) & 1) * 2 + ((l >> 4) & 1).
__device__ __forceinline__ float gvr_reduce4(const float (&v)[GVR_RB], int lane) {
  const bool b5 = lane & 32, b4 = lane & 16;
  float t2[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const float keep = b5 ? v[k + 2] : v[k], send = b5 ? v[k] : v[k + 2];
    t2[k] = keep + __shfl_xor(send, 32, 64);
  }
  float t = (b4 ? t2[1] : t2[0]) + __shfl_xor(b4 ? t2[0] : t2[1], 16, 64);
  return lane_group_sum(t, 16);
}
__device__ __forceinline__ int gvr_row_of_lane(int lane) { return ((lane >> 5) & 1) * 2 + ((lane >> 4) & 1); }

// One row's bytes for this lane: two 16-byte pieces of qs and the header.
struct GvrLoad {
  u4v q0, q1, hd;
};

// Q4_K quarter j of a superblock against the lane's 64 activations
// (xe[2m] = (x[4m], x[4m+2]), xe[2m+1] = (x[4m+1], x[4m+3]) for the low
// sub-block's 32 values m = 0..7, then the high sub-block's at 16 + ...),
// with the sub-blocks' activation sums xs_lo, xs_hi.
__device__ __forceinline__ float gvr_quarter_q4k(const GvrLoad& L, int j, const uint32_t (&xe)[32], float xs_lo,
                                                 float xs_hi) {
  uint32_t sc0, m0, sc1, m1;
  scale_min_k4(2 * j, L.hd.y, L.hd.z, L.hd.w, sc0, m0);
  scale_min_k4(2 * j + 1, L.hd.y, L.hd.z, L.hd.w, sc1, m1);
  const float d = f16_bits_to_f32(L.hd.x), dmin = f16_bits_to_f32(L.hd.x >> 16);
  const uint32_t w[8] = {L.q0.x, L.q0.y, L.q0.z, L.q0.w, L.q1.x, L.q1.y, L.q1.z, L.q1.w};
  float lo0 = 0.0f, lo1 = 0.0f, hi0 = 0.0f, hi1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t ws = w[i] >> 8;
    lo0 = fdot2u(w[i] & 0x000F000Fu, xe[2 * i], lo0);
    lo1 = fdot2u(ws & 0x000F000Fu, xe[2 * i + 1], lo1);
    hi0 = fdot2u(w[i] & 0x00F000F0u, xe[16 + 2 * i], hi0);
    hi1 = fdot2u(ws & 0x00F000F0u, xe[16 + 2 * i + 1], hi1);
  }
  const float s = __builtin_fmaf((float)sc1 * 0.0625f, hi0 + hi1, (float)sc0 * (lo0 + lo1));
  const float mterm = __builtin_fmaf((float)m1, xs_hi, (float)m0 * xs_lo);
  return d * (s * 16777216.0f) - dmin * mterm;
}

// XR: 16-byte activation pieces per thread when staging the row
// (ceil(K / 8 / threads) rounded up to 1, 2, 4 or 8).  D: rows of loads in
// flight per wave (a multiple of RB).  Measured on 14336 x 4096 (one
// workgroup of 8 waves per compute unit): the arithmetic alone takes about
// 5 us and the loads alone about 7, and the two overlap only in part; D = 8
// was slower than D = 4 at every shape.
template <int YT, int XR, int D>
__device__ __forceinline__ void gvr_q4k_body(const GvrArgs& a) {
  static_assert(D % GVR_RB == 0, "D must be a multiple of the reduction batch");
  __shared__ __attribute__((aligned(16))) _Float16 gvr_x[GVR_MAXK / 64 * GVR_XSTRIDE];
  __shared__ float gvr_red[2][GVR_MAXW][GVR_RB];  // [batch parity][wave][row of batch]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = a.C;
  const int g = wave / C, c = wave - g * C;
  const int slots = 4 * a.units;
  const int slot = 64 * c + lane;
  const bool valid = slot < slots;
  const int sl = min(slot, slots - 1);
  const int u = sl >> 2, j = sl & 3;
  const int gid = (int)blockIdx.x * a.G + g;
  const int gstride = (int)gridDim.x * a.G;
  const uint8_t* wq = a.w + (size_t)u * 144 + 16 + 32 * j;
  const uint8_t* wh = a.w + (size_t)u * 144;
  auto load_row = [&](GvrLoad& L, int i) {
    const int r = min(gid + i * gstride, a.N - 1);
    const size_t off = (size_t)r * (size_t)a.row_bytes;
    L.q0 = ld_u128(wq + off);
    L.q1 = ld_u128(wq + off + 16);
    L.hd = ld_u128(wh + off);
  };
  // activation row: 16-byte pieces, issued before the first weight loads
  const int pieces = a.K >> 3;  // 8 halves each
  const int nthreads = blockDim.x;
  u4v xv[XR];
#pragma unroll
  for (int q = 0; q < XR; q++) {
    const int p = min((int)threadIdx.x + q * nthreads, pieces - 1);
    xv[q] = ld_u128((const uint8_t*)(a.x + 8 * p));
  }
  GvrLoad ring[D];
#pragma unroll
  for (int d = 0; d < D; d++) load_row(ring[d], d);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < XR; q++) {
    const int p = (int)threadIdx.x + q * nthreads;
    if (p < pieces) *(u4v*)(gvr_x + (p >> 3) * GVR_XSTRIDE + 8 * (p & 7)) = xv[q];
  }
  __syncthreads();
  // this lane's 64 activations as dot2 pairs, and its two sub-block sums
  uint32_t xe[32];
  float xs_lo = 0.0f, xs_hi = 0.0f;
  {
    const _Float16* src = gvr_x + sl * GVR_XSTRIDE;
    const h2 one = {1, 1};
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const u4v v = *(const u4v*)(src + 8 * q);
      const int b = 4 * (q & 3) + 16 * (q >> 2);
      xe[b + 0] = perm(v.y, v.x, 0x05040100u);
      xe[b + 1] = perm(v.y, v.x, 0x07060302u);
      xe[b + 2] = perm(v.w, v.z, 0x05040100u);
      xe[b + 3] = perm(v.w, v.z, 0x07060302u);
      float s = __builtin_amdgcn_fdot2(as_h2(v.x), one, 0.0f, false);
      s = __builtin_amdgcn_fdot2(as_h2(v.y), one, s, false);
      s = __builtin_amdgcn_fdot2(as_h2(v.z), one, s, false);
      s = __builtin_amdgcn_fdot2(as_h2(v.w), one, s, false);
      if (q < 4) xs_lo += s;
      else xs_hi += s;
    }
    if (!valid) xs_lo = xs_hi = 0.0f;
  }
  const int rrow = gvr_row_of_lane(lane);
  // D rows per iteration, each reduced in batches of RB: ring slot k holds
  // row i0 + k; once computed it is refilled with row i0 + k + D, or, in
  // the last iteration, with its own row again (a cache hit, so that no
  // branch disturbs the compiler's count of loads in flight).
  for (int i0 = 0; i0 < a.iters; i0 += D) {
    const bool more = i0 + D < a.iters;
#pragma unroll
    for (int b = 0; b < D; b += GVR_RB) {
      float part[GVR_RB];
#pragma unroll
      for (int k = 0; k < GVR_RB; k++) {
        const float p = gvr_quarter_q4k(ring[b + k], j, xe, xs_lo, xs_hi);
        part[k] = valid ? p : 0.0f;
        load_row(ring[b + k], more ? i0 + b + k + D : i0 + b + k);
      }
      const float tot = gvr_reduce4(part, lane);
      const int ib = i0 + b;
      const int r = gid + (ib + rrow) * gstride;
      if (C == 1) {
        if ((lane & 15) == 0 && ib + rrow < a.iters && r < a.N) cq_store_raw<YT>(a.y, tot, r);
      } else {
        const int par = (ib / GVR_RB) & 1;
        if ((lane & 15) == 0) gvr_red[par][wave][rrow] = tot;
        __syncthreads();
        if (c == 0 && lane < GVR_RB) {
          float sacc = 0.0f;
          for (int cc = 0; cc < C; cc++) sacc += gvr_red[par][wave + cc][lane];
          const int rr = gid + (ib + lane) * gstride;
          if (ib + lane < a.iters && rr < a.N) cq_store_raw<YT>(a.y, sacc, rr);
        }
      }
    }
  }
}

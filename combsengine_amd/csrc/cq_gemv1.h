// Decode GEMV for a single activation row (m = 1), every format (K-quant
// superblocks; legacy blocks eight at a time):
// y[n] = sum_k x[k] * W[n, k], streamed at HBM speed.
//
// Why not the MFMA GEMV here: with one activation row an MFMA computes 16
// rows of which one is used, and its lane = weight-row layout makes every
// wave gather 16 separate 16-byte streams.  This kernel gives each lane one
// whole unit (superblock) instead:
//   - a wave task is R = max(1, 64 / units) consecutive rows, i.e. one
//     contiguous span of at most 64 units; lane l computes unit l of the
//     span (row l / units, unit l % units);
//   - the span is read as consecutive 16-byte pieces, piece 64 i + l by
//     lane l in load instruction i, so each instruction is one contiguous
//     1 KB read (64 strided 16-byte pieces, one unit per lane, measured
//     8.5 us against 6.6 us for a 33 MB read), and handed to the owning
//     lanes through a per-wave LDS slice;
//   - a persistent grid of one 8- or 4-wave workgroup per compute unit,
//     each wave walking ~N/(R * waves) tasks with the next task's loads in
//     flight while the current one is computed.
// Two activation paths:
//   - Q4_K (the fp16 register path): the row is staged once per workgroup
//     in LDS as fp16 and every lane keeps its unit's 256 values in registers
//     for the whole launch (a lane's unit is the same in every task), so the
//     only LDS traffic per task is the weight hand-over; weights arrive by
//     LDS DMA into two slices per wave.  Nibbles masked in place are fp16
//     subnormals q * 2^-24, so v_dot2_f32_f16 forms exact products q * x.
//   - the other formats: each 32-value activation block is staged as three
//     int8 parts, x = s * (h + l/254 + e/254^2) with s = max|x|/127 (about
//     22 bits relative to the block maximum, error <= max|x| * 3.9e-8; two
//     parts, 15 bits, fail the 1e-3 bar on outputs that cancel), and each
//     lane masks its nibbles in place (q = 0..15 / 0..31 per byte) and
//     accumulates v_dot4_i32_i8 against h, l and e, exactly in int32; per
//     sub-block the three sums become one fp32 value scaled by d * sc * s.
// In both, the K-quant min term uses fp32 sums of the fp16 activations and
// the lanes of a row are summed with cross-lane adds.
// Replaces qmatmul.rs:92-125 (Q4_0), :386-423 (Q5_0), :440-470 (Q8_0),
// :881-930 (Q4_K), :1064-1117 (Q5_K) and :1184-1229 (Q6_K) for m = 1.
#pragma once
#include <type_traits>
#include "cq_gemv.h"

#define GV1_XMAX 16384                       // largest K staged
#define GV1_XSTRIDE 272                      // bytes per staged 256-value unit (16 pad)

// Timeline hook of the fp16-register path: measurement builds define it to
// record a timestamp per wave at each numbered point; the library build
// compiles it to nothing.
#ifndef GV1_MARK
#define GV1_MARK(ev)
#endif

struct Gv1Args {
  const uint8_t* w;
  const uint8_t* w2;    // EPI = 2: the up projection (same format and shape as w, the gate)
  const _Float16* x;
  void* y;
  long long row_bytes;  // units * block bytes
  int N, K, units;
  int rows;             // lane rows per wave task (R)
  int tasks;            // ceil(N / R), or ceil(N / (R / 2)) for EPI = 2
  int prefetch2;        // 1: when every wave has at most two tasks, load both before staging x
  int wave_major;       // 1: task t runs on wave t / grid of workgroup t % grid (balanced), 0: on workgroup t / NW
  int span;             // 1: load each task as a contiguous span (formats with whole 16-byte units)
  CqEpi epi;
  // EPI = 3: up to GV1_MSEG weights of one format and K against the same
  // activation row, one output each; task t belongs to weight i when
  // mt0[i] <= t < mt0[i + 1] (each weight's rows a multiple of R, so no task
  // straddles two)
  const uint8_t* mw[4];
  void* my[4];
  int mt0[5];
  int mn[4];
  int nseg;
};
#define GV1_MSEG 4

__shared__ __attribute__((aligned(16))) int8_t gv_xh[GV1_XMAX / 256 * GV1_XSTRIDE];
__shared__ __attribute__((aligned(16))) int8_t gv_xl[GV1_XMAX / 256 * GV1_XSTRIDE];
__shared__ __attribute__((aligned(16))) int8_t gv_xe[GV1_XMAX / 256 * GV1_XSTRIDE];
__shared__ float gv_xs[GV1_XMAX / 32];  // s of each 32-value block
__shared__ float gv_s[GV1_XMAX / 32];   // sum of each 32-value block (fp32 of the fp16 values)
__shared__ float gv_s16[GV1_XMAX / 16]; // sum of each 16-value half block

// Staging of the fp16 activation row into LDS as three int8 parts per
// 32-value block (gv_xh/gv_xl/gv_xe), with each block's scale (gv_xs), sum
// (gv_s) and 16-value half sums (gv_s16).  issue() loads the row into
// registers (16-byte chunks, thread c holds chunks c, c + 64 NW, ...);
// commit() quantises and stores them.  Branch-free: indices past the end are
// clamped, so chunks may be loaded twice with the same value (control-flow
// joins would make the compiler wait for every outstanding load).  The
// caller issues its weight loads between the two and synchronises after
// commit().
// Q6P = 1 permutes each unit's eight 32-value quadrants (half h, quadrant t)
// to slot 2 (2h + (t & 1)) + (t >> 1), the layout of cq_gemv2's Q6_K reads
// (lanes h, c = t & 1 of one slot then fall on different LDS banks); the
// scale and sum arrays keep the value order.
template <int NW, int Q6P = 0>
struct Gv1XStage {
  static constexpr int XL = GV1_XMAX / 8 / (64 * NW);  // chunks per thread, at most
  u4v xv[XL];
  __device__ __forceinline__ void issue(const _Float16* x, int K) {
    const int xc_last = K / 8 - 1;
#pragma unroll
    for (int i = 0; i < XL; i++) {
      const int c = min((int)threadIdx.x + 64 * NW * i, xc_last);
      xv[i] = ld_u128((const uint8_t*)(x + 8 * c));
    }
  }
  // Thread c holds chunk c (8 values); the 4 threads of a 32-value block
  // share its max and sum.  Threads past the end hold a copy of the last
  // chunk and store nothing.
  __device__ __forceinline__ void commit(int K) {
    const int xc_last = K / 8 - 1;
#pragma unroll
    for (int i = 0; i < XL; i++) {
      if (64 * NW * i > xc_last) break;  // uniform
      const int craw = (int)threadIdx.x + 64 * NW * i;
      const int c = min(craw, xc_last);
      const uint32_t wv[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      float v[8], mx = 0.0f, sm = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = (float)as_h2(wv[e])[0];
        v[2 * e + 1] = (float)as_h2(wv[e])[1];
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        mx = fmaxf(mx, fabsf(v[e]));
        sm += v[e];
      }
      mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
      sm += __shfl_xor(sm, 1, 64);
      const float sm16 = sm;  // this thread pair's 16 values
      sm += __shfl_xor(sm, 2, 64);
      const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
      uint32_t hw[2] = {0, 0}, lw[2] = {0, 0}, ew[2] = {0, 0};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        // y = x/s in [-127, 127]; residuals after each rounding are in [-0.5, 0.5]
        const float y = v[e] * inv;
        const float hv = __builtin_rintf(y);
        const float r1 = (y - hv) * 254.0f;
        const float lv = __builtin_rintf(r1);
        const float ev = __builtin_rintf((r1 - lv) * 254.0f);
        const int sh = 8 * (e & 3);
        hw[e >> 2] |= (uint32_t)((int)hv & 0xFF) << sh;
        lw[e >> 2] |= (uint32_t)((int)lv & 0xFF) << sh;
        ew[e >> 2] |= (uint32_t)((int)ev & 0xFF) << sh;
      }
      if (craw <= xc_last) {
        int q = (c & 31) >> 2;  // quadrant of the unit: 4 h + t
        if (Q6P) q = 2 * (2 * (q >> 2) + (q & 1)) + ((q >> 1) & 1);
        const int off = (c >> 5) * GV1_XSTRIDE + 32 * q + 8 * (c & 3);
        *(u2v*)(gv_xh + off) = u2v{hw[0], hw[1]};
        *(u2v*)(gv_xl + off) = u2v{lw[0], lw[1]};
        *(u2v*)(gv_xe + off) = u2v{ew[0], ew[1]};
        if ((c & 3) == 0) {
          gv_xs[c >> 2] = mx * (1.0f / 127.0f);
          gv_s[c >> 2] = sm;
        }
        if ((c & 1) == 0) gv_s16[c >> 1] = sm16;
      }
    }
  }
};

// The 8 scales and mins of a K-quant superblock header as floats.
__device__ __forceinline__ void gv1_scales(const u4v& hd, float sc[8], float mn[8]) {
  // All eight 6-bit scales (mins) as the four bytes of two words: sub-blocks
  // 0-3 are the low six bits of bytes 0-3 of hd.y (hd.z); 4-7 take the low
  // (high) nibble of hd.w's byte and, above it, the top two bits of hd.y's
  // (hd.z's) byte (get_scale_min_k4), one bit-field insert per word.
  uint32_t s47, m47;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(s47) : "v"(0x0F0F0F0Fu), "v"(hd.w), "v"(hd.y >> 2));
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(m47) : "v"(0x0F0F0F0Fu), "v"(hd.w >> 4), "v"(hd.z >> 2));
  const uint32_t w[4] = {hd.y & 0x3F3F3F3Fu, hd.z & 0x3F3F3F3Fu, s47 & 0x3F3F3F3Fu, m47 & 0x3F3F3F3Fu};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    sc[j] = (float)((w[0] >> (8 * j)) & 0xFFu);
    mn[j] = (float)((w[1] >> (8 * j)) & 0xFFu);
    sc[4 + j] = (float)((w[2] >> (8 * j)) & 0xFFu);
    mn[4 + j] = (float)((w[3] >> (8 * j)) & 0xFFu);
  }
}

// Bytes of a lane's unit of 256 values: one K-quant superblock, or eight
// consecutive 32-value blocks of a legacy format (144 / 176 / 272 bytes, so
// units stay 16-byte aligned whenever rows are).
template <int FMT>
constexpr int gv1_unit_bytes() {
  return FmtTraits<FMT>::vals == 256 ? FmtTraits<FMT>::bytes : 8 * (FmtTraits<FMT>::bytes / LB);
}

// One unit in registers, as 16-byte chunks.
template <int FMT>
struct Gv1Block {
  static constexpr int NC = gv1_unit_bytes<FMT>() / 16;
  static constexpr bool TAIL = gv1_unit_bytes<FMT>() % 16 != 0;  // Q6_K: d in the last 2 bytes
  u4v c[NC];
  uint32_t tail;
  __device__ __forceinline__ void load(const uint8_t* p) {
#pragma unroll
    for (int i = 0; i < NC; i++) c[i] = ld_u128(p + 16 * i);
    if (TAIL) tail = ld_u16(p + 16 * NC);
  }
  // Either one unit per lane (span = 0: chunk i of the unit at p), or the
  // wave's span of units as consecutive 16-byte pieces (span = 1: chunk i
  // is piece q = 64 i + lane; pieces q < seg come from b0, at most lim0 of
  // them, the rest from b1, at most lim1; a piece past a limit re-reads the
  // last valid one).  Both are 16-byte loads; the span form makes each load
  // instruction one contiguous 1 KB read, which the memory pipeline serves
  // far faster than 64 strided 16-byte pieces.
  __device__ __forceinline__ void load_any(bool span, const uint8_t* p, const uint8_t* b0, int seg, int lim0,
                                           const uint8_t* b1, int lim1) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < NC; i++) {
      const int q = 64 * i + lane;
      const uint8_t* sp = q < seg ? b0 + 16 * min(q, lim0 - 1) : b1 + 16 * min(q - seg, lim1 - 1);
      c[i] = ld_u128(span ? sp : p + 16 * i);
    }
    if (TAIL) tail = ld_u16(p + 16 * NC);
  }
};
// Units whose bytes are whole 16-byte chunks can be loaded as a contiguous
// span and handed to their lanes through LDS (K-quants but Q6_K, and the
// legacy formats up to 12 chunks; Q8_0's 17 would not fit with 8 waves).
template <int FMT>
constexpr bool gv1_spannable() {
  return gv1_unit_bytes<FMT>() % 16 == 0 && gv1_unit_bytes<FMT>() / 16 <= 12;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Partial dot product of one superblock with the staged activations of its
// unit (xh, xl, xe: 256 int8 each; xs, su: 8 block scales / sums).
template <int FMT>
__device__ __forceinline__ float gv1_superblock(const Gv1Block<FMT>& b, const int8_t* xh, const int8_t* xl,
                                                const int8_t* xe, const float* xs, const float* su) {
  const u4v hd = b.c[0];
  float sc[8], mn[8];
  gv1_scales(hd, sc, mn);
  const float d = f16_bits_to_f32(hd.x), dmin = f16_bits_to_f32(hd.x >> 16);
  constexpr int QC = FMT == CQ_Q5_K ? 3 : 1;  // first qs chunk
  float acc = 0.0f, macc = 0.0f;
#pragma unroll
  for (int p = 0; p < 4; p++) {  // sub-block pair: 2p (low nibbles), 2p+1 (high)
    int ih0 = 0, il0 = 0, ie0 = 0, ih1 = 0, il1 = 0, ie1 = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {  // bytes [16h, 16h+16) of the pair: values 16h .. 16h+15
      const u4v q = b.c[QC + 2 * p + h];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
      const int o0 = 64 * p + 16 * h, o1 = o0 + 32;
      const u4v h0 = *(const u4v*)(xh + o0), l0 = *(const u4v*)(xl + o0);
      const u4v h1 = *(const u4v*)(xh + o1), l1 = *(const u4v*)(xl + o1);
      const u4v e0 = *(const u4v*)(xe + o0), e1 = *(const u4v*)(xe + o1);
      const uint32_t xh0[4] = {h0.x, h0.y, h0.z, h0.w}, xl0[4] = {l0.x, l0.y, l0.z, l0.w};
      const uint32_t xh1[4] = {h1.x, h1.y, h1.z, h1.w}, xl1[4] = {l1.x, l1.y, l1.z, l1.w};
      const uint32_t xe0[4] = {e0.x, e0.y, e0.z, e0.w}, xe1[4] = {e1.x, e1.y, e1.z, e1.w};
      uint32_t hb[4] = {0, 0, 0, 0};
      if constexpr (FMT == CQ_Q5_K) {
        const u4v qh = b.c[1 + h];
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
    // |il| * 254 + |ie| stays far inside int32: combine exactly, then one conversion
    const float f0 = __builtin_fmaf((float)(254 * il0 + ie0), 1.0f / 64516.0f, (float)ih0);
    const float f1 = __builtin_fmaf((float)(254 * il1 + ie1), 1.0f / 64516.0f, (float)ih1);
    acc = __builtin_fmaf(sc[2 * p] * xs[2 * p], f0, acc);
    acc = __builtin_fmaf(sc[2 * p + 1] * xs[2 * p + 1], f1, acc);
    macc = __builtin_fmaf(mn[2 * p], su[2 * p], macc);
    macc = __builtin_fmaf(mn[2 * p + 1], su[2 * p + 1], macc);
  }
  return d * acc - dmin * macc;
}

__device__ __forceinline__ uint32_t u4_word(const u4v& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Q6_K (gguf.rs:968-999): value (half hh, quadrant t, l) is
// (ql nibble | 2 qh bits << 4) - 32 with scale sc[8hh + l/16 + 2t]; the ql
// byte is 64hh + 32(t&1) + l (nibble t>>1), the qh byte 32hh + l (bits 2t).
// The 6-bit q (0..63) goes into v_dot4 as is; the -32 is applied as
// -32 * sum(x) per 16-value group.  xs16: sums of the unit's 16 groups.
__device__ __forceinline__ float gv1_superblock_q6k(const Gv1Block<CQ_Q6_K>& b, const int8_t* xh, const int8_t* xl,
                                                   const int8_t* xe, const float* xs, const float* xs16) {
  const float d = f16_bits_to_f32(b.tail);
  const u4v sc0 = b.c[12];
  const uint32_t scw[4] = {sc0.x, sc0.y, sc0.z, sc0.w};
  float acc = 0.0f, cacc = 0.0f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int ih[2] = {0, 0}, il[2] = {0, 0}, ie[2] = {0, 0};
      const int ko = 128 * hh + 32 * t;  // staged byte offset of this quadrant
#pragma unroll
      for (int j = 0; j < 8; j++) {   // 4 values l = 4j .. 4j+3
        const uint32_t qlw = u4_word(b.c[4 * hh + 2 * (t & 1) + (j >> 2)], j & 3);
        const uint32_t qhw = u4_word(b.c[8 + 2 * hh + (j >> 2)], j & 3);
        const uint32_t q = ((qlw >> (4 * (t >> 1))) & 0x0F0F0F0Fu) | (((qhw >> (2 * t)) & 0x03030303u) << 4);
        const int g = j >> 2;  // 16-value group l/16
        ih[g] = dot4(q, *(const uint32_t*)(xh + ko + 4 * j), ih[g]);
        il[g] = dot4(q, *(const uint32_t*)(xl + ko + 4 * j), il[g]);
        ie[g] = dot4(q, *(const uint32_t*)(xe + ko + 4 * j), ie[g]);
      }
      const float sblk = xs[4 * hh + t];
#pragma unroll
      for (int g = 0; g < 2; g++) {
        const int si = 8 * hh + g + 2 * t;
        const float scf = (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
        const float f = __builtin_fmaf((float)(254 * il[g] + ie[g]), 1.0f / 64516.0f, (float)ih[g]);
        acc = __builtin_fmaf(scf * sblk, f, acc);
        cacc = __builtin_fmaf(scf, xs16[8 * hh + 2 * t + g], cacc);
      }
    }
  }
  return d * __builtin_fmaf(-32.0f, cacc, acc);
}

// 32-bit word at even byte offset o of a unit in registers (o is a
// compile-time constant once unrolled; odd halfword offsets cost one
// v_alignbit).
template <int NC>
__device__ __forceinline__ uint32_t gv1_word(const u4v (&c)[NC], int o) {
  const int wi = o >> 2;
  const uint32_t w0 = u4_word(c[wi >> 2], wi & 3);
  if ((o & 3) == 0) return w0;
  const uint32_t w1 = u4_word(c[(wi + 1) >> 2], (wi + 1) & 3);
  return __builtin_amdgcn_alignbit(w1, w0, 16);
}
template <int NC>
__device__ __forceinline__ uint32_t gv1_half(const u4v (&c)[NC], int o) {
  const int wi = o >> 2;
  return (u4_word(c[wi >> 2], wi & 3) >> (8 * (o & 2))) & 0xFFFFu;
}

// Legacy 32-value blocks, eight per unit (block b = values 32b .. 32b+31):
// Q4_0 (gguf.rs:755-774) value j = low nibble of qs byte j, j + 16 = its high
// nibble, (q - 8) * d; Q5_0 (gguf.rs:825-847) adds qh bit j / j + 16 as the
// 5th bit, (q - 16) * d; Q8_0 (gguf.rs:779-794) q = signed byte j, q * d.
// The offsets -8 / -16 are applied as -8 / -16 * sum(x) of the block.
// Q4_1 / Q5_1 (gguf.rs:798-820, 851-874) are Q4_0 / Q5_0 with a min m after
// the scale and no offset: value = q * d + m, the m term m * sum(x).
template <int FMT>
__device__ __forceinline__ float gv1_unit_legacy(const Gv1Block<FMT>& b, const int8_t* xh, const int8_t* xl,
                                                 const int8_t* xe, const float* xs, const float* su) {
  constexpr int BB = FmtTraits<FMT>::bytes / LB;  // bytes per 32-value block
  float acc = 0.0f;
#pragma unroll
  for (int blk = 0; blk < 8; blk++) {
    const int o = BB * blk;
    const float d = f16_bits_to_f32(gv1_half(b.c, o));
    int ih = 0, il = 0, ie = 0;
    const int xo = 32 * blk;
    if constexpr (FMT == CQ_Q8_0) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t q = gv1_word(b.c, o + 2 + 4 * i);
        ih = dot4(q, *(const uint32_t*)(xh + xo + 4 * i), ih);
        il = dot4(q, *(const uint32_t*)(xl + xo + 4 * i), il);
        ie = dot4(q, *(const uint32_t*)(xe + xo + 4 * i), ie);
      }
    } else {
      constexpr bool Q5 = FMT == CQ_Q5_0 || FMT == CQ_Q5_1;
      constexpr int HO = FMT == CQ_Q5_1 ? 4 : 2;                                    // qh offset
      constexpr int QO = FMT == CQ_Q5_0 ? 6 : FMT == CQ_Q4_1 ? 4 : FMT == CQ_Q5_1 ? 8 : 2;  // qs offset
      uint32_t qh = 0;
      if constexpr (Q5) qh = gv1_word(b.c, o + HO);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t w = gv1_word(b.c, o + QO + 4 * i);
        uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        if constexpr (Q5) {
          lo |= spread4(qh >> (4 * i)) << 4;
          hi |= spread4(qh >> (16 + 4 * i)) << 4;
        }
        ih = dot4(lo, *(const uint32_t*)(xh + xo + 4 * i), ih);
        il = dot4(lo, *(const uint32_t*)(xl + xo + 4 * i), il);
        ie = dot4(lo, *(const uint32_t*)(xe + xo + 4 * i), ie);
        ih = dot4(hi, *(const uint32_t*)(xh + xo + 16 + 4 * i), ih);
        il = dot4(hi, *(const uint32_t*)(xl + xo + 16 + 4 * i), il);
        ie = dot4(hi, *(const uint32_t*)(xe + xo + 16 + 4 * i), ie);
      }
    }
    const float f = __builtin_fmaf((float)(254 * il + ie), 1.0f / 64516.0f, (float)ih);
    float v = xs[blk] * f;
    if constexpr (FMT == CQ_Q4_0) v = __builtin_fmaf(-8.0f, su[blk], v);
    if constexpr (FMT == CQ_Q5_0) v = __builtin_fmaf(-16.0f, su[blk], v);
    acc = __builtin_fmaf(d, v, acc);
    if constexpr (FMT == CQ_Q4_1 || FMT == CQ_Q5_1) acc = __builtin_fmaf(f16_bits_to_f32(gv1_half(b.c, o + 2)), su[blk], acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// fp16-activation variant (Q4_K): the activation row is staged once per
// workgroup in LDS as fp16 (a plain copy, with fp32 sums of each 32-value
// block), and every lane then keeps its unit's 256 values in registers for
// the whole launch: a lane's unit is lane % units in every task, so after
// the start the only LDS traffic left is the hand-over of the weight span.
// The inner products use v_dot2_f32_f16 on nibbles masked in place: in a
// 16-bit half, q (0..15) or 16 q are the fp16 subnormals q * 2^-24 and
// 16 q * 2^-24, exact, so each product q * x is exact in fp32.  Masking the
// word w and w >> 8 pairs bytes (0, 2) and (1, 3), so the lane's values are
// kept as pairs (x[4m], x[4m+2]) and (x[4m+1], x[4m+3]).
typedef __attribute__((address_space(3))) void gv_lds_t;
typedef __attribute__((address_space(1))) void gv_glb_t;

// LDS DMA of 16 bytes per lane (global_load_lds_dwordx4: lane l's bytes
// land at LDS byte address m0 + 16 l), issued as inline assembly so that the
// compiler's wait-count pass does not see it: the kernel waits for these
// loads itself (gv3_wait_vm), by position in the in-order vector-memory
// counter.  The compiler treats any pending LDS DMA conservatively and would
// otherwise wait for every load in flight before each LDS read.
__device__ __forceinline__ void gv3_dma16(const void* src, uint32_t lds_byte_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_byte_addr)
               : "memory", "m0");
}
// s_waitcnt vmcnt(N) (other counters unconstrained), then a compiler barrier
// so that no LDS read moves above it.
template <int N>
__device__ __forceinline__ void gv3_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ uint32_t gv3_lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(gv_lds_t*)p);
}

// A lane's 256 activations of unit u as the pairs described above
// (xe[2m] = (x[4m], x[4m+2]), xe[2m+1] = (x[4m+1], x[4m+3])), read from the
// staged row x16p (units at a 264-value stride), and its 8 block sums
// (computed per lane: measured faster than one thread per block through
// LDS).
struct Gv3XRegs {
  uint32_t xe[128];
  float su[16];  // sums of the 16 16-value groups (Q6_K) or of the 8 32-value blocks (Q4_K, su[0..7])
  __device__ __forceinline__ void load(int u, const _Float16* x16p) {
    const _Float16* src = x16p + 264 * u;
#pragma unroll
    for (int q = 0; q < 32; q++) {
      const u4v v = *(const u4v*)(src + 8 * q);
      xe[4 * q + 0] = perm(v.y, v.x, 0x05040100u);
      xe[4 * q + 1] = perm(v.y, v.x, 0x07060302u);
      xe[4 * q + 2] = perm(v.w, v.z, 0x05040100u);
      xe[4 * q + 3] = perm(v.w, v.z, 0x07060302u);
    }
  }
  // fp32 sums of 16-value groups (G = 16) or 32-value blocks (G = 32):
  // group j's pairs are xe[G/2 j .. G/2 j + G/2)
  template <int G>
  __device__ __forceinline__ void lane_sums() {
    const h2 one = {1, 1};
#pragma unroll
    for (int j = 0; j < 256 / G; j++) {
      float a = 0.0f, b = 0.0f;
#pragma unroll
      for (int e = 0; e < G / 2; e += 2) {
        a = __builtin_amdgcn_fdot2(as_h2(xe[G / 2 * j + e]), one, a, false);
        b = __builtin_amdgcn_fdot2(as_h2(xe[G / 2 * j + e + 1]), one, b, false);
      }
      su[j] = a + b;
    }
  }
};

__device__ __forceinline__ float fdot2u(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// Q4_K superblock against the lane's registers: per sub-block pair p the
// low nibbles (sub-block 2p) meet x[64p + j], the high nibbles (2p + 1)
// x[64p + 32 + j]; sums are in units of 2^-24 (low) and 2^-20 (high).
__device__ __forceinline__ float gv3_superblock_q4k(const u4v* pc, const Gv3XRegs& xr) {
  const u4v hd = pc[0];
  float sc[8], mn[8];
  gv1_scales(hd, sc, mn);
  const float d = f16_bits_to_f32(hd.x), dmin = f16_bits_to_f32(hd.x >> 16);
  float acc = 0.0f, macc = 0.0f;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    float lo0 = 0.0f, lo1 = 0.0f, hi0 = 0.0f, hi1 = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const u4v q = pc[1 + 2 * p + h];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ws = w[i] >> 8;
        const int m = 16 * p + 4 * h + i;
        lo0 = fdot2u(w[i] & 0x000F000Fu, xr.xe[2 * m], lo0);
        lo1 = fdot2u(ws & 0x000F000Fu, xr.xe[2 * m + 1], lo1);
        hi0 = fdot2u(w[i] & 0x00F000F0u, xr.xe[2 * m + 16], hi0);
        hi1 = fdot2u(ws & 0x00F000F0u, xr.xe[2 * m + 17], hi1);
      }
    }
    acc = __builtin_fmaf(sc[2 * p], lo0 + lo1, acc);
    acc = __builtin_fmaf(sc[2 * p + 1] * 0.0625f, hi0 + hi1, acc);
    macc = __builtin_fmaf(mn[2 * p], xr.su[2 * p], macc);
    macc = __builtin_fmaf(mn[2 * p + 1], xr.su[2 * p + 1], macc);
  }
  return d * (acc * 16777216.0f) - dmin * macc;
}

// Q6_K superblock (gguf.rs:968-999) against the lane's registers, read from
// an LDS slice at any 2-byte alignment (210-byte superblocks; unaligned LDS
// reads are supported on gfx950).  Value (half hh, quadrant t, l) =
// (ql nibble | 2 qh bits << 4) - 32 at x[128 hh + 32 t + l] with scale
// sc[8 hh + l/16 + 2 t]; the 6-bit q of four consecutive l are built as
// bytes, split into the pairs (l, l+2), (l+1, l+3) as fp16 subnormals, and
// the -32 is applied as -32 * (sum of the 16-value group).
__device__ __forceinline__ float gv3_superblock_q6k(const uint8_t* sb, const Gv3XRegs& xr) {
  const u4v sc0 = ld_u128(sb + 192);
  const uint32_t scw[4] = {sc0.x, sc0.y, sc0.z, sc0.w};
  const float d = f16_bits_to_f32(ld_u16(sb + 208));
  float acc = 0.0f, cacc = 0.0f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    u4v qh4[2];
    qh4[0] = ld_u128(sb + 128 + 32 * hh);
    qh4[1] = ld_u128(sb + 144 + 32 * hh);
#pragma unroll
    for (int c = 0; c < 2; c++) {  // ql column: quadrants t = c (low nibbles), c + 2 (high)
      u4v ql4[2];
      ql4[0] = ld_u128(sb + 64 * hh + 32 * c);
      ql4[1] = ld_u128(sb + 64 * hh + 32 * c + 16);
#pragma unroll
      for (int tt = 0; tt < 2; tt++) {
        const int t = c + 2 * tt;
#pragma unroll
        for (int g = 0; g < 2; g++) {  // 16-value group l / 16
          float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {  // l = 16 g + 4 jj .. +3
            const uint32_t qlw = u4_word(ql4[g], jj), qhw = u4_word(qh4[g], jj);
            // per byte: bits 0-3 the ql nibble, 4-5 quadrant t's two qh
            // bits (shifted there; bits 6-7 are left over from other
            // fields), one bit-field insert; the 0x3F masks below drop 6-7
            const uint32_t nl = tt ? qlw >> 4 : qlw;
            const uint32_t hb = t == 0 ? qhw << 4 : t == 1 ? qhw << 2 : t == 2 ? qhw : qhw >> 2;
            uint32_t q;  // (opaque to the compiler, which otherwise re-derives the fields with more operations)
            asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(q) : "v"(0x0F0F0F0Fu), "v"(nl), "v"(hb));
            const int m = 32 * hh + 8 * t + 4 * g + jj;
            s0 = fdot2u(q & 0x003F003Fu, xr.xe[2 * m], s0);
            s1 = fdot2u((q >> 8) & 0x003F003Fu, xr.xe[2 * m + 1], s1);
          }
          const int si = 8 * hh + g + 2 * t;
          const float scf = (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
          acc = __builtin_fmaf(scf, s0 + s1, acc);
          cacc = __builtin_fmaf(scf, xr.su[8 * hh + 2 * t + g], cacc);
        }
      }
    }
  }
  return d * __builtin_fmaf(16777216.0f, acc, -32.0f * cacc);
}

// Q5_K superblock (gguf.rs:929-961) against the lane's registers: as Q4_K,
// plus the 5th bit of value (pair p, byte l) = bit 2p (low nibble) or
// 2p + 1 (high nibble) of qh[l], moved to bit 4 of the low value's half
// (q = nib | bit << 4) or bit 8 of the high one's (16 q = 16 nib | bit << 8),
// both still fp16 subnormals.  Layout: header 16 bytes, qh 32, qs 128.
__device__ __forceinline__ float gv3_superblock_q5k(const u4v* pc, const Gv3XRegs& xr) {
  const u4v hd = pc[0];
  float sc[8], mn[8];
  gv1_scales(hd, sc, mn);
  const float d = f16_bits_to_f32(hd.x), dmin = f16_bits_to_f32(hd.x >> 16);
  float acc = 0.0f, macc = 0.0f;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    float lo0 = 0.0f, lo1 = 0.0f, hi0 = 0.0f, hi1 = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const u4v q = pc[3 + 2 * p + h], qh = pc[1 + h];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ws = w[i] >> 8;
        // bit 2p of qh bytes 0, 2 (1, 3) to bits 4, 20 and bit 2p + 1 to
        // bits 8, 24 of the pair (0, 2) ((1, 3))
        const uint32_t tl0 = p < 2 ? hw[i] << (4 - 2 * p) : hw[i] >> (2 * p - 4), tl1 = hw[i] >> (2 * p + 4);
        const uint32_t th0 = hw[i] << (7 - 2 * p), th1 = hw[i] >> (2 * p + 1);
        const int m = 16 * p + 4 * h + i;
        lo0 = fdot2u((w[i] & 0x000F000Fu) | (tl0 & 0x00100010u), xr.xe[2 * m], lo0);
        lo1 = fdot2u((ws & 0x000F000Fu) | (tl1 & 0x00100010u), xr.xe[2 * m + 1], lo1);
        hi0 = fdot2u((w[i] & 0x00F000F0u) | (th0 & 0x01000100u), xr.xe[2 * m + 16], hi0);
        hi1 = fdot2u((ws & 0x00F000F0u) | (th1 & 0x01000100u), xr.xe[2 * m + 17], hi1);
      }
    }
    acc = __builtin_fmaf(sc[2 * p], lo0 + lo1, acc);
    acc = __builtin_fmaf(sc[2 * p + 1] * 0.0625f, hi0 + hi1, acc);
    macc = __builtin_fmaf(mn[2 * p], xr.su[2 * p], macc);
    macc = __builtin_fmaf(mn[2 * p + 1], xr.su[2 * p + 1], macc);
  }
  return d * (acc * 16777216.0f) - dmin * macc;
}

// Legacy units (eight 32-value blocks) against the lane's registers.  Q4_0
// (gguf.rs:755-774): block b at byte 18 b, [d][16 qs]; value j = low nibble
// of qs[j] at x[32 b + j], j + 16 = its high nibble; (q - 8) d, the -8 as
// -8 * (block sum).  Q8_0 (gguf.rs:779-794): block b at 34 b, [d][32 qs];
// q = qs[j] signed at x[32 b + j], fed as the byte q + 128 (a subnormal)
// with -128 * (block sum).  Block fields are 2-byte aligned in LDS.
template <int FMT>
__device__ __forceinline__ float gv3_unit_legacy(const uint8_t* up, const Gv3XRegs& xr) {
  float acc = 0.0f;
#pragma unroll
  for (int blk = 0; blk < 8; blk++) {
    float s0 = 0.0f, s1 = 0.0f;
    if constexpr (FMT == CQ_Q4_0) {
      const uint8_t* bp = up + 18 * blk;
      const u4v q = ld_u128(bp + 2);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
      float h0 = 0.0f, h1 = 0.0f;  // high nibbles, seen as 16 q
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t ws = w[i] >> 8;
        const int m = 8 * blk + i;  // low nibbles: x[32 blk + 4 i ..]; high nibbles: 16 values on
        s0 = fdot2u(w[i] & 0x000F000Fu, xr.xe[2 * m], s0);
        s1 = fdot2u(ws & 0x000F000Fu, xr.xe[2 * m + 1], s1);
        h0 = fdot2u(w[i] & 0x00F000F0u, xr.xe[2 * m + 8], h0);
        h1 = fdot2u(ws & 0x00F000F0u, xr.xe[2 * m + 9], h1);
      }
      const float d = f16_bits_to_f32(ld_u16(bp));
      const float sq = __builtin_fmaf(0.0625f, h0 + h1, s0 + s1);
      acc = __builtin_fmaf(d, __builtin_fmaf(16777216.0f, sq, -8.0f * xr.su[blk]), acc);
    } else {
      const uint8_t* bp = up + 34 * blk;
      u4v q[2];
      q[0] = ld_u128(bp + 2);
      q[1] = ld_u128(bp + 18);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t w = u4_word(q[i >> 2], i & 3) ^ 0x80808080u;
        const int m = 8 * blk + i;
        s0 = fdot2u(w & 0x00FF00FFu, xr.xe[2 * m], s0);
        s1 = fdot2u(perm(w, w, 0x0C030C01u), xr.xe[2 * m + 1], s1);  // bytes 1, 3 to the low bytes of the halves
      }
      const float d = f16_bits_to_f32(ld_u16(bp));
      acc = __builtin_fmaf(d, __builtin_fmaf(16777216.0f, s0 + s1, -128.0f * xr.su[blk]), acc);
    }
  }
  return acc;
}

// Activation mode of cq_gemv1 per format: 1 = fp16 registers (Q4_K), 0 =
// int8 three-part LDS staging.
template <int FMT>
constexpr int gv1_xmode() {
  return FMT == CQ_Q4_K || FMT == CQ_Q5_K || FMT == CQ_Q6_K || FMT == CQ_Q4_0 || FMT == CQ_Q8_0 ? 1 : 0;
}

// Waves per workgroup: 8 (two per SIMD) where the register budget allows it
// without spilling (Q4_K / Q5_K), else 4.
template <int FMT>
constexpr int gv1_waves() {
  return FMT == CQ_Q4_K || FMT == CQ_Q4_0 ? 8 : 4;
}

// EPI = 0: no epilogue (a.epi empty), no loads at store time; EPI = 1: the
// epilogue's loads happen at each store (they wait for the weight loads in
// flight; a slower path kept for outputs with a bias or a gate); EPI = 2:
// the gated MLP input in one launch, y = act(x . W^T) * (x . W2^T) — a task
// holds floor(R / 2) rows of the gate W and the same rows of the up W2
// (R >= 2: units <= 32), so both share one activation staging and the
// product is formed across lanes.
// The gated Q6_K kernel keeps the int8 path and 4 waves.
template <int FMT, int EPI>
constexpr int gv1_kernel_waves() {
  return EPI == 2 && FMT == CQ_Q6_K ? 4 : gv1_waves<FMT>();
}
// EPI = 3: several weights against one activation row (Gv1Args::mw / my),
// fp16-register path only.
template <int FMT, int YT, int EPI, int NW = gv1_kernel_waves<FMT, EPI>(),
          int XM = (EPI == 2 && FMT == CQ_Q6_K) ? 0 : gv1_xmode<FMT>()>
__device__ __forceinline__ void gemv1_body(const Gv1Args& a) {
  static_assert(EPI != 3 || XM == 1, "several weights per launch: fp16-register path only");
  constexpr int BB = gv1_unit_bytes<FMT>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lanes_used = a.rows * a.units;
  const int myrow = lane / a.units, myunit = lane - myrow * a.units;
  const int stride = gridDim.x * NW;
  // lane's superblock of task t (lanes past the task's rows reread its first)
  const int half = a.rows >> 1;  // EPI = 2: output rows per task
  auto block_ptr = [&](int t) {
    if constexpr (EPI == 2) {
      const int up = myrow >= half;
      const int row = min(t * half + myrow - (up ? half : 0), a.N - 1);
      return (up ? a.w2 : a.w) + ((size_t)row * a.units + myunit) * BB;
    }
    const int r0 = t * a.rows;
    const int nsb = min(a.rows, a.N - r0) * a.units;
    return a.w + ((size_t)r0 * a.units + (lane < nsb ? lane : 0)) * BB;
  };
  // Span loads: a task's units are R consecutive rows (gate rows then up
  // rows for EPI = 2), i.e. one or two contiguous byte ranges; each wave
  // passes its pieces to the owning lanes through its own LDS slice.
  constexpr bool SPANOK = gv1_spannable<FMT>();
  constexpr int NC = Gv1Block<FMT>::NC;
  __shared__ __attribute__((aligned(16))) u4v gv_tw[SPANOK ? NW * 64 * NC : 1];
  const bool span = SPANOK && (XM == 1 || a.span);
  auto load_task = [&](Gv1Block<FMT>& blk, int t) {
    const uint8_t* p = block_ptr(t);
    if constexpr (EPI == 2) {
      // lanes [0, half * units) hold gate rows, the rest the same up rows
      const int r0 = t * half, lim = min(half, a.N - r0) * a.units * NC;
      const size_t off = (size_t)r0 * a.units * BB;
      blk.load_any(span, p, a.w + off, half * a.units * NC, lim, a.w2 + off, lim);
    } else {
      const int r0 = t * a.rows, lim = min(a.rows, a.N - r0) * a.units * NC;
      const uint8_t* b0 = a.w + (size_t)r0 * a.units * BB;
      blk.load_any(span, p, b0, 1 << 30, lim, b0, lim);
    }
  };
  Gv3XRegs xregs;  // XM = 1 only
  // Row sums across the lanes of each row, then the store (and epilogue).
  auto task_store = [&](float part, int tt, void* yv, int N) {
    const int r0 = tt * (EPI == 2 ? half : a.rows);
    const int nrows = min(EPI == 2 ? half : a.rows, N - r0);
    const int rq = EPI == 2 && myrow >= half ? myrow - half : myrow;  // output row of this lane
    if ((a.units & (a.units - 1)) == 0) {
      // a row's lanes form an aligned group of `units` lanes: sum within it
      part = lane_group_sum(part, a.units);
      if constexpr (EPI == 2) {
        // up row rq sits half * units lanes after its gate row
        const float upv = __shfl(part, (lane + half * a.units) & 63, 64);
        if (myunit == 0 && myrow < half && rq < nrows)
          cq_store_raw<YT>(yv, cq_gated<YT>(part, upv, a.epi.act), r0 + rq);
      } else if (myunit == 0 && myrow < nrows) {
        if constexpr (EPI == 1) cq_store<YT>(yv, a.epi, part, r0 + myrow, r0 + myrow);
        else cq_store_raw<YT>(yv, part, r0 + myrow);
      }
    } else if constexpr (EPI == 2) {
      // gate row q and its up row q + half, each summed over the wave
      for (int q = 0; q < half; q++) {
        const float v = lane_group_sum(myrow == q ? part : 0.0f, 64);
        const float u = lane_group_sum(myrow == q + half ? part : 0.0f, 64);
        if (lane == 0 && q < nrows) cq_store_raw<YT>(yv, cq_gated<YT>(v, u, a.epi.act), r0 + q);
      }
    } else {
      for (int q = 0; q < a.rows; q++) {
        const float v = lane_group_sum(myrow == q ? part : 0.0f, 64);
        if (lane == 0 && q < nrows) {
          if constexpr (EPI == 1) cq_store<YT>(yv, a.epi, v, r0 + q, r0 + q);
          else cq_store_raw<YT>(yv, v, r0 + q);
        }
      }
    }
    };
  auto task_compute = [&](const Gv1Block<FMT>& blk_in, int tt) {
    Gv1Block<FMT> blk = blk_in;
    if constexpr (SPANOK) {
      if (span) {
        // piece 64 i + lane -> LDS; then lane reads its unit (pieces NC lane ..)
        // (one wave's LDS operations complete in order: no barrier needed)
        u4v* tw = gv_tw + wave * 64 * NC;
#pragma unroll
        for (int i = 0; i < NC; i++) tw[64 * i + lane] = blk_in.c[i];
#pragma unroll
        for (int i = 0; i < NC; i++) blk.c[i] = tw[NC * lane + i];
      }
    }
    const int r0 = tt * (EPI == 2 ? half : a.rows);
    const int nrows = min(EPI == 2 ? half : a.rows, a.N - r0);
    const int rq = EPI == 2 && myrow >= half ? myrow - half : myrow;  // output row of this lane
    float part = 0.0f;
    if (lane < lanes_used && rq < nrows) {
      if constexpr (XM == 1) {
        part = 0.0f;  // (served by the XM = 1 loop below)
      } else {
      const int8_t* xh = gv_xh + myunit * GV1_XSTRIDE;
      const int8_t* xl = gv_xl + myunit * GV1_XSTRIDE;
      const int8_t* xe = gv_xe + myunit * GV1_XSTRIDE;
      if constexpr (FMT == CQ_Q6_K) part = gv1_superblock_q6k(blk, xh, xl, xe, gv_xs + 8 * myunit, gv_s16 + 16 * myunit);
      else if constexpr (FmtTraits<FMT>::vals != 256)
        part = gv1_unit_legacy<FMT>(blk, xh, xl, xe, gv_xs + 8 * myunit, gv_s + 8 * myunit);
      else part = gv1_superblock<FMT>(blk, xh, xl, xe, gv_xs + 8 * myunit, gv_s + 8 * myunit);
      }
    }
    task_store(part, tt, a.y, a.N);
  };
  // Load order matters (the vector-memory counter retires in order): the
  // activation chunks first, then the first task's weights, so that staging
  // x into LDS waits only for x while the weights' HBM latency runs on.
  Gv1XStage<NW> xst;  // XM = 0 only
  if constexpr (XM == 0) xst.issue(a.x, a.K);
  // Tasks go wave-major over the grid (task t: wave t / grid of workgroup
  // t % grid), so when tasks do not divide evenly every compute unit still
  // gets the same share within one task per wave.
  int t = a.wave_major ? wave * (int)gridDim.x + (int)blockIdx.x : blockIdx.x * NW + wave;
  if constexpr (XM == 1) {
    // Each task's span goes straight to LDS by DMA (global_load_lds, 1 KB
    // per instruction, piece 64 i + lane at 16 (64 i + lane)), two slices
    // per wave in distinct arrays: task j + 1 lands in one while task j is
    // computed from the other, its lane reading its superblock at BB lane.
    // A span's last piece may run into the next task's bytes; the host
    // checks that the weight's byte size is a multiple of 16, so no piece
    // runs past the weight.
    // Two span slices per wave (the 64 lanes' units, 64 BB bytes, packed)
    // in distinct arrays, so the compiler sees reads of one never alias a
    // DMA into the other.  The fp16 activation row is staged in the second
    // before any DMA uses it.
    constexpr int SP = 64 * BB / 16;        // 16-byte pieces per wave slice
    constexpr int NI = (SP + 63) / 64;      // DMA instructions (1 KB) per task
    __shared__ __attribute__((aligned(16))) u4v gv_sa[NW * SP];
    __shared__ __attribute__((aligned(16))) u4v gv_sb[NW * SP];
    static_assert(NW * SP * 16 >= GV1_XMAX / 256 * 528, "the staged row fits in gv_sb");
    const int n = t < a.tasks ? (a.tasks - 1 - t) / stride + 1 : 0;
    // task tt -> (weight, output, rows, task within the weight): the launch's
    // own for EPI != 3, weight i's for EPI = 3 (uniform over the wave)
    struct View {
      const uint8_t* w;
      void* y;
      int N, t;
    };
    auto view = [&](int tt) -> View {
      if constexpr (EPI == 3) {
        int i = 0;
#pragma unroll
        for (int q = 1; q < GV1_MSEG; q++) i += (q < a.nseg && tt >= a.mt0[q]) ? 1 : 0;
        return View{a.mw[i], a.my[i], a.mn[i], tt - a.mt0[i]};
      }
      return View{a.w, a.y, a.N, tt};
    };
    auto dma_task = [&](u4v* arr, int tt) {
      const uint8_t *b0, *b1;
      int seg, lim0, lim1;
      if constexpr (EPI == 2) {
        // (BB is a multiple of 16 here: EPI = 2 runs this path for Q4_K only)
        const int r0 = tt * half, lim = min(half, a.N - r0) * a.units * (BB / 16);
        const size_t off = (size_t)r0 * a.units * BB;
        b0 = a.w + off, b1 = a.w2 + off, seg = half * a.units * (BB / 16), lim0 = lim1 = lim;
      } else {
        const View v = view(tt);
        const int r0 = v.t * a.rows, lim = (min(a.rows, v.N - r0) * a.units * BB + 15) / 16;
        b0 = b1 = v.w + (size_t)r0 * a.units * BB, seg = 1 << 30, lim0 = lim1 = lim;
      }
      u4v* dst = arr + wave * SP;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const int q = 64 * i + lane;
        const uint8_t* src = q < seg ? b0 + 16 * min(q, lim0 - 1) : b1 + 16 * min(q - seg, lim1 - 1);
        if (SP % 64 == 0 || i + 1 < NI || q < SP) gv3_dma16(src, gv3_lds_addr(dst + 64 * i));  // the slice ends at SP
      }
    };
    auto compute = [&](const u4v* arr, int tt) {
      const View v = view(tt);
      const int r0 = v.t * (EPI == 2 ? half : a.rows);
      const int nrows = min(EPI == 2 ? half : a.rows, v.N - r0);
      const int rq = EPI == 2 && myrow >= half ? myrow - half : myrow;
      float part = 0.0f;
      if (lane < lanes_used && rq < nrows) {
        const uint8_t* sbp = (const uint8_t*)(arr + wave * SP) + BB * lane;
        if constexpr (FMT == CQ_Q6_K) part = gv3_superblock_q6k(sbp, xregs);
        else if constexpr (FMT == CQ_Q4_K) {
          // all nine reads first: one LDS latency per superblock instead of
          // one per group of reads the scheduler would interleave
          u4v sb[9];
#pragma unroll
          for (int q = 0; q < 9; q++) sb[q] = ((const u4v*)sbp)[q];
          __builtin_amdgcn_sched_barrier(0);
          part = gv3_superblock_q4k(sb, xregs);
        }
        else if constexpr (FMT == CQ_Q5_K) part = gv3_superblock_q5k((const u4v*)sbp, xregs);
        else part = gv3_unit_legacy<FMT>(sbp, xregs);
      }
      task_store(part, v.t, v.y, v.N);
    };
    // The activation row (K fp16, a multiple of 8 values) goes to gv_sb by
    // DMA with each 256-value unit at a 264-value (528-byte) stride: units
    // 512 bytes apart would put every lane's read of the same chunk of its
    // unit in one LDS bank.  A unit is one half-wave instruction (32 lanes x
    // 16 bytes); waves take unit pairs in turn.  These DMAs are the older
    // ones in the counter.
    GV1_MARK(0);
    _Float16* x16p = (_Float16*)gv_sb;
    {
      const int nunits = a.K / 256;
      for (int u0 = 2 * wave; u0 < nunits; u0 += 2 * NW) {
        if (lane < 32) gv3_dma16(a.x + 256 * u0 + 8 * lane, gv3_lds_addr(x16p + 264 * u0));
        if (lane >= 32 && u0 + 1 < nunits)
          gv3_dma16(a.x + 256 * (u0 + 1) + 8 * (lane - 32), gv3_lds_addr(x16p + 264 * (u0 + 1)) - 512);
      }
    }
    dma_task(gv_sa, min(t, a.tasks - 1));
    gv3_wait_vm<NI>();
    GV1_MARK(1);
    __syncthreads();
    GV1_MARK(7);
    xregs.load(myunit, x16p);
    xregs.lane_sums<FMT == CQ_Q6_K ? 16 : 32>();  // (Q4_K / legacy: 32-value blocks)
    GV1_MARK(8);
    // The staged row (in gv_sb) fully read before any DMA into gv_sb.  (The
    // second task's DMA goes out only now: issued together with the first,
    // the headline shape measured 11.6 against 10.4 us.)
    __syncthreads();
    GV1_MARK(2);
    for (int j = 0; j < n; j += 2, t += 2 * stride) {
      if (j + 1 < n) {
        dma_task(gv_sb, t + stride);
        gv3_wait_vm<NI>();
      } else {
        gv3_wait_vm<0>();
      }
      GV1_MARK(3 + 2 * j);
      compute(gv_sa, t);
      GV1_MARK(4 + 2 * j);
      if (j + 1 >= n) break;
      if (j + 2 < n) {
        dma_task(gv_sa, t + 2 * stride);
        gv3_wait_vm<NI>();
      } else {
        gv3_wait_vm<0>();
      }
      GV1_MARK(5 + 2 * j);
      compute(gv_sb, t + stride);
      GV1_MARK(6 + 2 * j);
    }
    // no LDS DMA may still be landing when the workgroup's LDS is handed on
    // (a wave without tasks still loaded one into its first slice)
    gv3_wait_vm<0>();
    return;
  } else {
  Gv1Block<FMT> cur, nxt;
  if (a.prefetch2 && a.tasks <= 2 * stride) {
    // At most two tasks per wave (uniform over the grid): both tasks' loads
    // go out before the staging, so the whole weight stream is requested at
    // once; a wave with one task reloads the last task (an L2 hit) and
    // drops it.
    load_task(cur, min(t, a.tasks - 1));
    load_task(nxt, min(t + stride, a.tasks - 1));
    __builtin_amdgcn_sched_barrier(0);
    xst.commit(a.K);
    __syncthreads();
    if (t < a.tasks) task_compute(cur, t);
    if (t + stride < a.tasks) task_compute(nxt, t + stride);
    return;
  }
  load_task(cur, min(t, a.tasks - 1));
  __builtin_amdgcn_sched_barrier(0);  // keep the weight loads ahead of the staging
  xst.commit(a.K);
  __syncthreads();

  // This wave's tasks t, t + stride, ...: n of them.  Loads run one task
  // ahead of the compute, each compute call sits on a path of its own so
  // that the compiler's in-order load counters wait exactly for the task
  // it needs.
  const int n = t < a.tasks ? (a.tasks - 1 - t) / stride + 1 : 0;
  for (int j = 0; j < n; j += 2, t += 2 * stride) {
    if (j + 1 < n) {
      load_task(nxt, t + stride);
      task_compute(cur, t);
      if (j + 2 < n) {
        load_task(cur, t + 2 * stride);
        task_compute(nxt, t + stride);
      } else {
        task_compute(nxt, t + stride);
      }
    } else {
      task_compute(cur, t);
    }
  }
  }
}

// Single-row decode for rows longer than one wave's 64 units (65 to 128
// units, 106 for Q6_K: K from 16640 to 32768, the register-path formats
// other than Q8_0).  A workgroup is two wave pairs; in a pair, wave 2g + p keeps
// the activations of the row's half p (units p * ceil(units / 2) ..) in
// registers and takes that half of every row the pair serves, by LDS DMA
// of its byte range (from the 16-byte boundary at or below its start:
// 210-byte Q6_K units leave half spans at any even offset, which the
// superblock reads accept).  Both halves' sums meet in LDS, one barrier per
// row; the pair's first wave adds them in a fixed order and stores.
constexpr int GV1K_WAVES = 4;
template <int FMT>
constexpr int gv1k_xunits() {
  // units of the staged activation row that fit beside the two slices
  constexpr int sp = 64 * gv1_unit_bytes<FMT>() / 16 + 1;
  constexpr int left = (163840 - 2 * GV1K_WAVES * sp * 16 - 64) / 528;
  return left < 128 ? left : 128;
}
template <int FMT, int YT, int EPI>
__device__ __forceinline__ void gemv1k_body(const Gv1Args& a) {
  constexpr int NW = GV1K_WAVES, G = NW / 2;
  constexpr int BB = gv1_unit_bytes<FMT>();
  constexpr int SP = 64 * BB / 16 + 1;  // pieces per slice: 64 units and a start offset
  constexpr int NI = (SP + 63) / 64;
  constexpr int XU = gv1k_xunits<FMT>();
  __shared__ __attribute__((aligned(16))) u4v gk_sa[NW * SP];
  __shared__ __attribute__((aligned(16))) u4v gk_sb[NW * SP];
  __shared__ __attribute__((aligned(16))) u4v gk_x[XU * 33];
  __shared__ float gk_red[2][NW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int p = wave & 1, g = wave >> 1;
  const int upart = (a.units + 1) >> 1;
  const int u0 = p * upart, cnt = min(upart, a.units - u0);
  const int rstride = (int)gridDim.x * G, rbase = (int)blockIdx.x * G;
  // rows served: rbase + g + i * rstride; every wave of the workgroup runs
  // the same n iterations (group 0's count), so the barriers match
  const int n = rbase < a.N ? (a.N - 1 - rbase) / rstride + 1 : 0;
  if (n == 0) return;
  auto start_of = [&](int i) {
    const int r = min(rbase + g + i * rstride, a.N - 1);
    return (size_t)r * (size_t)a.row_bytes + (size_t)u0 * BB;
  };
  auto dma_task = [&](u4v* arr, int i) {
    const size_t st = start_of(i);
    const uint8_t* b = a.w + (st & ~(size_t)15);
    const int lim = (int)(((st & 15) + (size_t)cnt * BB + 15) >> 4);  // pieces that hold the half
    u4v* dst = arr + wave * SP;
#pragma unroll
    for (int k = 0; k < NI; k++) {
      const int q = 64 * k + lane;
      if (SP % 64 == 0 || k + 1 < NI || q < SP) gv3_dma16(b + 16 * min(q, lim - 1), gv3_lds_addr(dst + 64 * k));
    }
  };
  Gv3XRegs xregs;
  auto compute = [&](const u4v* arr, int i) {
    const int r = rbase + g + i * rstride;
    float part = 0.0f;
    if (lane < cnt) {
      const uint8_t* sbp = (const uint8_t*)(arr + wave * SP) + (start_of(i) & 15) + BB * lane;
      if constexpr (FMT == CQ_Q6_K) part = gv3_superblock_q6k(sbp, xregs);
      else if constexpr (FMT == CQ_Q4_K) part = gv3_superblock_q4k((const u4v*)sbp, xregs);
      else if constexpr (FMT == CQ_Q5_K) part = gv3_superblock_q5k((const u4v*)sbp, xregs);
      else part = gv3_unit_legacy<FMT>(sbp, xregs);
    }
    part = lane_group_sum(part, 64);
    if (lane == 0) gk_red[i & 1][wave] = part;
    __syncthreads();
    if (p == 0 && lane == 0 && r < a.N) {
      const float v = gk_red[i & 1][wave] + gk_red[i & 1][wave + 1];
      if constexpr (EPI == 1) cq_store<YT>(a.y, a.epi, v, r, r);
      else cq_store_raw<YT>(a.y, v, r);
    }
  };
  // activation row -> gk_x (unit u at 528 u bytes), as in cq_gemv1
  _Float16* x16p = (_Float16*)gk_x;
  {
    const int nunits = a.K / 256;
    for (int v0 = 2 * wave; v0 < nunits; v0 += 2 * NW) {
      if (lane < 32) gv3_dma16(a.x + 256 * v0 + 8 * lane, gv3_lds_addr(x16p + 264 * v0));
      if (lane >= 32 && v0 + 1 < nunits)
        gv3_dma16(a.x + 256 * (v0 + 1) + 8 * (lane - 32), gv3_lds_addr(x16p + 264 * (v0 + 1)) - 512);
    }
  }
  dma_task(gk_sa, 0);
  if (n > 1) {
    dma_task(gk_sb, 1);
    gv3_wait_vm<2 * NI>();
  } else {
    gv3_wait_vm<NI>();
  }
  __syncthreads();
  xregs.load(u0 + min(lane, cnt - 1), x16p);
  xregs.lane_sums<FMT == CQ_Q6_K ? 16 : 32>();
  // Invariant at the top: rows i (gk_sa) and i + 1 (gk_sb, if any) issued.
  for (int i = 0; i < n; i += 2) {
    if (i + 1 < n) gv3_wait_vm<NI>();
    else gv3_wait_vm<0>();
    compute(gk_sa, i);
    if (i + 1 >= n) break;
    if (i + 2 < n) {
      dma_task(gk_sa, i + 2);
      gv3_wait_vm<NI>();
    } else {
      gv3_wait_vm<0>();
    }
    compute(gk_sb, i + 1);
    if (i + 3 < n) dma_task(gk_sb, i + 3);
  }
  gv3_wait_vm<0>();
}

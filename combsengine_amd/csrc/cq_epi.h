// Output epilogue of the matmul kernels, shared by the host launcher and the
// device code (plain C layout, the last member of every kernel argument block).
//
// It runs the steps the reference performs right after the quantized op:
//   - the bias add of Linear::forward (qlinear.rs:84-98): v = acc + bias[n];
//   - the gated MLP product act(gate(h)) * up(h) (llama.rs:301-303, with the
//     activations of act.rs:20-30), when `aux` holds up(h) for the same rows:
//     v = act(v) * aux[m][n].
// Either part may be absent (null pointer).  `aux` may be the output buffer
// itself: each output element is read and then written by the same thread.
#pragma once

enum { CQ_EPI_ACT_SILU = 0, CQ_EPI_ACT_GELU_TANH = 1, CQ_EPI_ACT_GELU = 2 };

struct CqEpi {
  const void* bias;  // [N], fp32 or fp16 (bias_f16), or null
  const void* aux;   // [M][N], fp32 or fp16 (aux_f16), or null
  int bias_f16;
  int aux_f16;
  int act;           // CQ_EPI_ACT_*
  int pad_;
};

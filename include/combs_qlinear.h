/*
 * combs_qlinear.h -- C ABI of the MI355X (gfx950) fused GGUF dequant-matmul.
 *
 * Drop-in replacement for the quantized-linear seam of asqrzk/CombsEngine:
 *   trait QuantLinearOp<B> { forward(x [batch,seq,k]) -> [batch,seq,n];
 *                            dims() -> [n,k]; vram_bytes() -> usize }
 *   engine/core/combs-models/src/qlinear.rs:56-63
 * backed by QuantWeight (engine/core/combs-models/src/qmatmul.rs:1601-1689).
 *
 * Conventions
 *   - Weights stay in the unchanged GGUF block layout in device memory:
 *     [n rows][k/QK blocks], blocks along k (gguf.rs:709-748).  No repack.
 *   - y = x . W^T with x [m,k] row-major and y [m,n] row-major; the bias is
 *     not part of the op (the seam adds it outside, qlinear.rs:84-98).
 *   - All launches are asynchronous on the given HIP stream (NULL = the
 *     default stream) and return after the launch, like the reference's
 *     launch-only matmul_device (qmatmul.rs:1674-1688).
 *   - Functions return CQ_OK or an error status and never abort; the last
 *     error message of the calling thread is kept for cq_last_error()
 *     (pattern of combs_last_error, engine/core/combs-ffi/src/lib.rs:55-67).
 *     Shape/format errors are detected on the host before any device work,
 *     so the caller can keep its dense fallback (qlinear.rs:318-325).
 *   - No symbol takes or returns a framework type; device buffers are plain
 *     pointers, streams are hipStream_t passed as void*.
 */
#ifndef COMBS_QLINEAR_H
#define COMBS_QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF block formats with a device kernel; values are the GGML type ids.
 * Replaces combs_formats::QuantFormat (engine/core/combs-formats/src/source.rs:42-55),
 * plus Q4_1 / Q5_1, which the reference decodes only on its dense path
 * (gguf.rs:798-820, 851-874, gguf.rs:1194-1196). */
typedef enum {
  CQ_Q4_0 = 2,  /* 32 values, 18 B: f16 d, 16 nibble bytes          */
  CQ_Q4_1 = 3,  /* 32 values, 20 B: f16 d, f16 m, 16 nibble bytes   */
  CQ_Q5_0 = 6,  /* 32 values, 22 B: f16 d, u32 high bits, 16 bytes  */
  CQ_Q5_1 = 7,  /* 32 values, 24 B: f16 d, f16 m, u32 high bits, 16 B */
  CQ_Q8_0 = 8,  /* 32 values, 34 B: f16 d, 32 x i8                  */
  CQ_Q4_K = 12, /* 256 values, 144 B                                */
  CQ_Q5_K = 13, /* 256 values, 176 B                                */
  CQ_Q6_K = 14  /* 256 values, 210 B                                */
} cq_format;

typedef enum { CQ_F32 = 0, CQ_F16 = 1 } cq_dtype;

typedef enum {
  CQ_OK = 0,
  CQ_ERR_BAD_FORMAT = 1, /* format id not supported                       */
  CQ_ERR_BAD_SHAPE = 2,  /* k not a block multiple, byte count != n,k, m<1 */
  CQ_ERR_BAD_DTYPE = 3,
  CQ_ERR_NULL = 4,       /* a required pointer was NULL                    */
  CQ_ERR_HIP = 5,        /* a HIP runtime call failed (message has detail) */
  CQ_ERR_NO_DEVICE = 6   /* no gfx950 device / code object failed to load */
} cq_status;

typedef struct cq_weight cq_weight;

/* Values per block (32 or 256) and bytes per block, 0 for an unknown format.
 * gguf.rs:709-748 (tensor_byte_size). */
int cq_block_values(int format);
int cq_block_bytes(int format);

/* Packed byte size of an [n, k] weight; CQ_ERR_BAD_SHAPE when k is not a
 * block multiple.  Mirrors the from_gguf_bytes checks, qmatmul.rs:212, 594,
 * 675, 1326-1328, 1444-1446, 1530-1532. */
cq_status cq_tensor_bytes(int format, int64_t n, int64_t k, size_t* out_bytes);

/* Upload a GGUF block stream (host memory) verbatim to the current device and
 * wrap it.  Replaces QuantWeight::from_quant_tensor (qmatmul.rs:1619-1635)
 * and Q*Weight::from_gguf_bytes (e.g. :1318-1344), called from
 * try_quant_linear (qlinear.rs:284-339).  Synchronises `stream` before
 * returning, so `host_bytes` may be freed afterwards. */
cq_status cq_weight_create(int format, const void* host_bytes, size_t nbytes, int64_t n, int64_t k,
                           void* stream, cq_weight** out);

/* Wrap a block stream that already lives in device memory (no copy; the
 * caller keeps ownership and must keep it alive).  Same validation. */
cq_status cq_weight_wrap_device(int format, const void* device_bytes, size_t nbytes, int64_t n, int64_t k,
                                cq_weight** out);

void cq_weight_destroy(cq_weight* w);

/* QuantLinearOp::dims (qlinear.rs:60): [n_out, k]. */
cq_status cq_weight_dims(const cq_weight* w, int64_t* n, int64_t* k);

/* QuantLinearOp::vram_bytes (qlinear.rs:62): bytes of the packed weight in
 * device memory (GGUF-native size; the reference's repacked layout used
 * 20/24/36/148/180/212 B per block instead). */
size_t cq_weight_vram_bytes(const cq_weight* w);

/* Device pointer of the packed blocks. */
const void* cq_weight_device_ptr(const cq_weight* w);

/* Fused dequant-matmul y[m,n] = x[m,k] . dequant(W)^T, fp32 accumulation.
 * Replaces QuantWeight::matmul_device (qmatmul.rs:1674-1688) and the
 * QuantLinearOp::forward it serves (qlinear.rs:58).  x: device, x_dtype
 * CQ_F16 or CQ_F32; y: device, caller-allocated, y_dtype CQ_F32 or CQ_F16.
 * fp32 activations must be finite and below 65504 in magnitude (they are fed
 * to the fp16 matrix cores as a hi+lo pair; at m >= 2 -- m >= 4 for the
 * K-quants -- that split is made once into 2m fp16 rows that the fp16
 * kernels multiply in one pass).  Prefill (m > 16; activation sums, split
 * partials), batched decode (2 <= m <= 16) of rows longer than 4096 values
 * and the fp32 split each take a per-device buffer kept across calls
 * (ordered across streams by an event).  While
 * the stream is being captured into a HIP graph, prefill and batched
 * decode take the device's fixed array instead (see cq_matmul_noalloc),
 * which graphs captured this way share: replays that overlap on one device
 * race; captured fp32 activations run the fp32-x kernels. */
cq_status cq_matmul(const cq_weight* w, const void* x, int x_dtype, int64_t m, void* y, int y_dtype,
                    void* stream);

/* Kernel paths of cq_matmul, for A/B tests (the reference's tiled/untiled
 * choice, qmatmul.rs:1361-1404 and COMBS_NO_TILED_MATMUL, :159-166). */
typedef enum { CQ_PATH_AUTO = 0, CQ_PATH_GEMV = 1, CQ_PATH_GEMM = 2 } cq_path;
cq_status cq_matmul_path(const cq_weight* w, const void* x, int x_dtype, int64_t m, void* y, int y_dtype,
                         int path, void* stream);

/* cq_matmul with the bias add fused into the kernels' epilogue:
 * y[m,n] = x[m,k] . dequant(W)^T + bias[n], one rounding to y_dtype.
 * Replaces the quantized branch of Linear::forward, op.forward(x) followed
 * by `out + b` broadcast over rows (qlinear.rs:84-98).  bias: device [n],
 * bias_dtype CQ_F32 or CQ_F16; NULL means no bias (the reference's None). */
cq_status cq_matmul_bias(const cq_weight* w, const void* x, int x_dtype, int64_t m, const void* bias,
                         int bias_dtype, void* y, int y_dtype, void* stream);

/* Activations of the gated MLP (combs_formats::Activation, applied by
 * act.rs:20-30): SiLU x*sigmoid(x); tanh-approximated GELU; exact (erf) GELU. */
typedef enum { CQ_ACT_SILU = 0, CQ_ACT_GELU_TANH = 1, CQ_ACT_GELU = 2 } cq_act;

/* Gated MLP input projection: y[m,n] = act(x . gate^T) * (x . up^T).
 * Replaces `act::apply(activation, gate.forward(h)) * up.forward(h)`
 * (llama.rs:301-303).  gate and up have the same [n, k] (formats may
 * differ).  Decode with fp16 x and one format for both weights is one
 * launch: m = 1 (K/256 <= 32) and 2 <= m <= 16 (K/256 <= 16, both weights
 * 16-byte aligned).  Otherwise up's product is written to y first, in
 * y_dtype, and gate's kernel epilogue reads it back and overwrites it.
 * No scratch memory on either path. */
cq_status cq_matmul_gate_up(const cq_weight* gate, const cq_weight* up, const void* x, int x_dtype, int64_t m,
                            int act, void* y, int y_dtype, void* stream);

/* Several projections of one input: ys[i][m, n_i] = x[m,k] . dequant(ws[i])^T
 * for i < count (1..4), every weight with the same k.  Replaces consecutive
 * QuantLinearOp::forward calls on one activation, as the attention block's
 * q / k / v projections (llama.rs:261-263).  Decode (m = 1, and
 * 2 <= m <= 16 with K/256 <= 16 and 16-byte aligned weights; fp16 x) of
 * weights of one format streams all of them in a single launch; otherwise
 * one cq_matmul per weight, in order, on `stream`. */
cq_status cq_matmul_multi(int count, const cq_weight* const* ws, const void* x, int x_dtype, int64_t m,
                          void* const* ys, int y_dtype, void* stream);

/* Bit-exact dequantisation of a device block stream to f32 (validation).
 * Replaces dequantize_*_gpu (qmatmul.rs:171-190, 530-573, 1232-1305); the
 * result equals gguf.rs dequantize_* (gguf.rs:755-999) bit for bit. */
cq_status cq_dequantize(int format, const void* device_bytes, size_t nbytes, int64_t n_values,
                        float* device_out, void* stream);

/* Quantise rows of f32 values into GGUF blocks on the host (input
 * generation; the reference has no quantizer, this restates ggml's
 * quantize_row_*_ref).  src [rows][k] -> dst [rows][k/QK blocks].
 * threads <= 0 uses all cores. */
cq_status cq_quantize(int format, const float* src, int64_t rows, int64_t k, void* dst, size_t dst_bytes,
                      int threads);

/* cq_matmul that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as cq_matmul; where cq_matmul takes
 * scratch from the device's buffers kept across calls (the prefill GEMM's
 * activation sums and split-K partials, the batched decode's slice partials
 * of long rows) this uses a
 * fixed 32 MiB device array that the library holds
 * on each device until the process ends, shrinking the K split until the
 * partials fit; a prefill whose activation sums alone (m * K / 8 bytes for
 * Q4_K / Q5_K) exceed it returns CQ_ERR_BAD_SHAPE.  Every call on a device
 * shares that device's array (nothing in it needs to start zeroed), so calls
 * that overlap on one device, on different streams or threads, race.  The
 * first call on a device loads the code objects and looks up the array's
 * address; cq_device_init does that ahead of time. */
cq_status cq_matmul_noalloc(const cq_weight* w, const void* x, int x_dtype, int64_t m, void* y, int y_dtype,
                            void* stream);
cq_status cq_device_init(void);

/* Diagnostics; no counterpart in the reference.
 * cq_matmul_kernels: the comma-separated names of the kernels cq_matmul
 * would launch for this weight, x_dtype, m and y_dtype (a dry run: nothing
 * is launched or allocated; the device's code objects are loaded).
 * cq_reload_options: re-read the COMBS_* tuning variables, which the library
 * otherwise reads once, at its first launch; not to be called while another
 * thread launches. */
cq_status cq_matmul_kernels(const cq_weight* w, int x_dtype, int64_t m, int y_dtype, char* buf, size_t buflen);
void cq_reload_options(void);

/* Message of the calling thread's last error ("" if none). */
const char* cq_last_error(void);

/* Library version string. */
const char* cq_version(void);

#ifdef __cplusplus
}
#endif
#endif /* COMBS_QLINEAR_H */

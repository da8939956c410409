"""Host-side mirror of the reference's quantized-linear seam.

Reference (asqrzk/CombsEngine, Rust):
  engine/core/combs-models/src/qlinear.rs   Linear / QuantLinearOp / try_quant_linear
  engine/core/combs-models/src/qmatmul.rs   QuantWeight, Q*Weight::{from_gguf_bytes,
                                            matmul_device, matmul_host, vram_bytes}
  engine/core/combs-formats/src/source.rs   QuantFormat, QuantTensor

Names, argument meanings and error behaviour follow those files; the compute
is the gfx950 library behind include/combs_qlinear.h.  torch is used only for
device buffers and the current HIP stream.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib as L


class ModelError(Exception):
    """combs_models::ModelError."""


class BadShape(ModelError):
    """ModelError::BadShape { tensor, expected, got } (qmatmul.rs:42-47 etc.)."""

    def __init__(self, tensor: str, expected, got, detail: str = ""):
        self.tensor, self.expected, self.got = tensor, list(expected), list(got)
        super().__init__(f"bad shape for {tensor}: expected {self.expected}, got {self.got}"
                         + (f" ({detail})" if detail else ""))


class QuantFormat(enum.IntEnum):
    """combs_formats::QuantFormat (source.rs:42-55); values are GGML type ids.
    Q4_1 / Q5_1 are served natively here; the reference decodes them only on
    its dense path (gguf.rs:798-874)."""
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q4K = 12
    Q5K = 13
    Q6K = 14


_BLOCK = {QuantFormat.Q4_0: (32, 18), QuantFormat.Q5_0: (32, 22), QuantFormat.Q8_0: (32, 34),
          QuantFormat.Q4_1: (32, 20), QuantFormat.Q5_1: (32, 24),
          QuantFormat.Q4K: (256, 144), QuantFormat.Q5K: (256, 176), QuantFormat.Q6K: (256, 210)}


def block_values(fmt) -> int:
    return _BLOCK[QuantFormat(fmt)][0]


def block_bytes(fmt) -> int:
    return _BLOCK[QuantFormat(fmt)][1]


def tensor_byte_size(fmt, n: int, k: int) -> int:
    """gguf.rs:709-748 for an [n, k] weight; BadShape if k is not a block multiple."""
    qk, bb = _BLOCK[QuantFormat(fmt)]
    if n < 1 or k < 1 or k % qk:
        raise BadShape(f"{QuantFormat(fmt).name} weight", [n, k], [n, k], f"k must be a multiple of {qk}")
    return n * (k // qk) * bb


@dataclass
class QuantTensor:
    """combs_formats::QuantTensor (source.rs:58-66): packed GGUF bytes, HF shape [n_out, k]."""
    format: QuantFormat
    shape: list
    data: bytes


def _check(status: int, what: str, tensor: str = "", expected=(), got=()):
    if status == L.CQ_OK:
        return
    msg = L.last_error()
    if status == L.CQ_ERR_BAD_SHAPE:
        raise BadShape(tensor or what, expected, got, msg)
    raise ModelError(f"{what}: status {status}: {msg}")


def _torch():
    import torch
    return torch


def _stream_ptr(device=None) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


_XT = {"torch.float16": L.CQ_F16, "torch.float32": L.CQ_F32}


class QuantWeight:
    """A device-resident GGUF weight ([n_out, k], blocks along k), the
    QuantWeight / Q*Weight types of qmatmul.rs:195-1689, without the repack:
    the bytes are stored exactly as in the file."""

    def __init__(self, handle: int, fmt: QuantFormat, n_out: int, k: int, keepalive=None):
        self._h = ctypes.c_void_p(handle)
        self.format = QuantFormat(fmt)
        self._n_out, self._k = n_out, k
        self._keepalive = keepalive

    # -- construction --------------------------------------------------------
    @classmethod
    def from_gguf_bytes(cls, fmt, data, n_out: int, k: int, stream=None) -> "QuantWeight":
        """Q*Weight::from_gguf_bytes (e.g. qmatmul.rs:1318-1344): validate and
        upload the raw block stream; BadShape on a size mismatch or a k that
        is not a block multiple."""
        fmt = QuantFormat(fmt)
        buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, np.uint8)
        # shape rules first (no device work on a bad shape, qmatmul.rs:1326-1335)
        if buf.size != tensor_byte_size(fmt, n_out, k):
            raise BadShape(f"{fmt.name.lower()} weight", [n_out, k], [buf.size])
        out = ctypes.c_void_p()
        s = stream if stream is not None else _stream_ptr()
        st = L.lib().cq_weight_create(int(fmt), buf.ctypes.data, buf.size, n_out, k, s, ctypes.byref(out))
        _check(st, "cq_weight_create", f"{fmt.name.lower()} weight", [n_out, k], [buf.size])
        return cls(out.value, fmt, n_out, k)

    @classmethod
    def from_device(cls, fmt, tensor, n_out: int, k: int) -> "QuantWeight":
        """Wrap a uint8 CUDA tensor that already holds the block stream (no copy)."""
        fmt = QuantFormat(fmt)
        out = ctypes.c_void_p()
        nbytes = tensor.numel() * tensor.element_size()
        st = L.lib().cq_weight_wrap_device(int(fmt), tensor.data_ptr(), nbytes, n_out, k, ctypes.byref(out))
        _check(st, "cq_weight_wrap_device", f"{fmt.name.lower()} weight", [n_out, k], [nbytes])
        return cls(out.value, fmt, n_out, k, keepalive=tensor)

    @classmethod
    def from_quant_tensor(cls, fmt, data, n_out: int, k: int) -> "QuantWeight":
        """QuantWeight::from_quant_tensor (qmatmul.rs:1619-1635)."""
        return cls.from_gguf_bytes(fmt, data, n_out, k)

    def __del__(self):
        h = getattr(self, "_h", None)
        # (at interpreter exit the module globals may already be cleared)
        lib = getattr(L, "_lib", None) if L is not None else None
        if h is not None and h.value and lib is not None:
            lib.cq_weight_destroy(h)
            self._h = None

    # -- accessors -------------------------------------------------------------
    def n_out(self) -> int:
        return self._n_out

    def k(self) -> int:
        return self._k

    def vram_bytes(self) -> int:
        """Packed bytes in device memory (GGUF-native; the reference's repacked
        layout was 20/24/36/148/180/212 B per block, qmatmul.rs:242-1553)."""
        return L.lib().cq_weight_vram_bytes(self._h)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    # -- compute ---------------------------------------------------------------
    def _io(self, x, y):
        """Validates x [m, k] / y [m, n_out] device tensors; returns (m, xt, yt)."""
        if not (x.is_cuda and y.is_cuda) or x.device != y.device:
            raise ModelError("x and y must be device tensors on the weight's device")
        if x.dim() != 2 or x.shape[1] != self._k or not x.is_contiguous():
            raise BadShape(f"{self.format.name.lower()} matmul input", [-1, self._k], list(x.shape))
        m = x.shape[0]
        if y.shape != (m, self._n_out) or not y.is_contiguous():
            raise BadShape(f"{self.format.name.lower()} matmul output", [m, self._n_out], list(y.shape))
        xt = _XT.get(str(x.dtype))
        yt = _XT.get(str(y.dtype))
        if xt is None or yt is None:
            raise ModelError(f"unsupported dtypes x={x.dtype} y={y.dtype}")
        return m, xt, yt

    def matmul_into(self, x, y, path: int = L.CQ_PATH_AUTO, stream=None):
        """Launch y[m, n] = x[m, k] . W^T on the current (or given) stream.
        x: CUDA fp16/fp32 contiguous [m, k]; y: CUDA fp32/fp16 contiguous [m, n]."""
        m, xt, yt = self._io(x, y)
        s = stream if stream is not None else _stream_ptr(x.device)
        st = L.lib().cq_matmul_path(self._h, x.data_ptr(), xt, m, y.data_ptr(), yt, path, s)
        _check(st, "cq_matmul", f"{self.format.name.lower()} matmul input", [m, self._k], list(x.shape))
        return y

    def matmul_bias_into(self, x, bias, y, stream=None):
        """y = x . W^T + bias[n] with the bias add in the kernels' epilogue
        (Linear::forward's quantized branch, qlinear.rs:84-98).  bias: device
        fp32/fp16 [n_out], or None."""
        m, xt, yt = self._io(x, y)
        bp, bt = 0, L.CQ_F32
        if bias is not None:
            if not bias.is_cuda or bias.device != x.device or bias.numel() != self._n_out or not bias.is_contiguous():
                raise BadShape(f"{self.format.name.lower()} bias", [self._n_out], list(bias.shape))
            bt = _XT.get(str(bias.dtype))
            if bt is None:
                raise ModelError(f"unsupported bias dtype {bias.dtype}")
            bp = bias.data_ptr()
        s = stream if stream is not None else _stream_ptr(x.device)
        st = L.lib().cq_matmul_bias(self._h, x.data_ptr(), xt, m, bp, bt, y.data_ptr(), yt, s)
        _check(st, "cq_matmul_bias", f"{self.format.name.lower()} matmul input", [m, self._k], list(x.shape))
        return y

    def matmul_device(self, x, m: Optional[int] = None, out_dtype=None, path: int = L.CQ_PATH_AUTO):
        """QuantWeight::matmul_device (qmatmul.rs:1674-1688): device x [m, k]
        in, freshly allocated device y [m, n_out] out (fp32 unless out_dtype)."""
        torch = _torch()
        if m is not None:
            x = x.reshape(m, self._k)
        x = x.contiguous()
        y = torch.empty((x.shape[0], self._n_out), dtype=out_dtype or torch.float32, device=x.device)
        return self.matmul_into(x, y, path=path)

    def matmul_host(self, x, m: int) -> np.ndarray:
        """Q*Weight::matmul_host (qmatmul.rs:1407-1419): host f32 x in, host
        f32 y out; BadShape when len(x) != m*k."""
        torch = _torch()
        x = np.ascontiguousarray(x, np.float32).ravel()
        if m < 1 or x.size != m * self._k:
            raise BadShape(f"{self.format.name.lower()} matmul input", [m, self._k], [x.size])
        xd = torch.from_numpy(x.reshape(m, self._k)).cuda()
        y = self.matmul_device(xd)
        return y.cpu().numpy()


def _kernel_input(x):
    """x itself when the kernels take its dtype (fp16, fp32), else x in fp32."""
    if str(x.dtype) in _XT:
        return x
    if not x.dtype.is_floating_point:
        raise ModelError(f"unsupported activation dtype {x.dtype}")
    return x.float()


class QuantLinearOp:
    """trait QuantLinearOp (qlinear.rs:56-63) over a QuantWeight."""

    def __init__(self, weight: QuantWeight):
        self.w = weight

    def forward(self, x):
        """x [batch, seq, k] -> [batch, seq, n_out] in x's dtype (the
        reference's output follows the input dtype, qlinear.rs:126-143).
        fp16 and fp32 go to the kernels as they are; any other float dtype
        (bf16) is cast to fp32 around the launch and the result cast back,
        as the reference casts every non-f32 input (qlinear.rs:126-143)."""
        b, s, k = x.shape
        xk = _kernel_input(x)
        y = self.w.matmul_device(xk.reshape(b * s, k), out_dtype=xk.dtype)
        return y.reshape(b, s, self.w.n_out()).to(x.dtype)

    def forward_bias(self, x, bias):
        """forward(x) + bias broadcast over rows, one kernel (qlinear.rs:84-98)."""
        b, s, k = x.shape
        xk = _kernel_input(x)
        if bias is not None and str(bias.dtype) not in _XT:
            bias = bias.float()
        y = _torch().empty((b * s, self.w.n_out()), dtype=xk.dtype, device=x.device)
        self.w.matmul_bias_into(xk.reshape(b * s, k).contiguous(), None if bias is None else bias.contiguous(), y)
        return y.reshape(b, s, self.w.n_out()).to(x.dtype)

    def dims(self):
        return [self.w.n_out(), self.w.k()]

    def vram_bytes(self) -> int:
        return self.w.vram_bytes()


class Activation(enum.IntEnum):
    """combs_formats::Activation as applied by act.rs:20-30."""
    Silu = L.CQ_ACT_SILU
    GeluTanh = L.CQ_ACT_GELU_TANH
    Gelu = L.CQ_ACT_GELU


def gated_up(activation, gate: "QuantLinearOp", up: "QuantLinearOp", h):
    """`act::apply(activation, gate.forward(h)) * up.forward(h)`
    (llama.rs:301-303) as one library call: up's product goes to the output,
    gate's kernel epilogue applies the activation and the product in place.
    h [batch, seq, k] fp16/fp32 -> [batch, seq, n] in h's dtype."""
    torch = _torch()
    b, s, k = h.shape
    if gate.dims() != up.dims() or gate.dims()[1] != k:
        raise BadShape("gate/up", gate.dims(), up.dims())
    n = gate.dims()[0]
    x = _kernel_input(h).reshape(b * s, k).contiguous()
    y = torch.empty((b * s, n), dtype=x.dtype, device=h.device)
    gate.w._io(x, y)
    xt, yt = _XT[str(x.dtype)], _XT[str(y.dtype)]
    st = L.lib().cq_matmul_gate_up(gate.w.handle, up.w.handle, x.data_ptr(), xt, b * s, int(Activation(activation)),
                                   y.data_ptr(), yt, _stream_ptr(x.device))
    _check(st, "cq_matmul_gate_up", "gate/up input", [b * s, k], list(x.shape))
    return y.reshape(b, s, n).to(h.dtype)


def multi_forward(ops, h):
    """[op.forward(h) for op in ops] (the q / k / v projections of one input,
    llama.rs:261-263) as one library call (cq_matmul_multi): for decode a
    single launch streams every weight.  h [batch, seq, k] fp16/fp32 (other
    float dtypes through fp32) -> list of [batch, seq, n_i] in h's dtype."""
    torch = _torch()
    b, s, k = h.shape
    if not 1 <= len(ops) <= 4 or any(op.dims()[1] != k for op in ops):
        raise BadShape("multi input", [len(ops), k], [op.dims() for op in ops])
    x = _kernel_input(h).reshape(b * s, k).contiguous()
    ys = [torch.empty((b * s, op.dims()[0]), dtype=x.dtype, device=h.device) for op in ops]
    for op, y in zip(ops, ys):
        op.w._io(x, y)
    xt = _XT[str(x.dtype)]
    wa = (ctypes.c_void_p * len(ops))(*[op.w.handle.value for op in ops])
    ya = (ctypes.c_void_p * len(ops))(*[y.data_ptr() for y in ys])
    st = L.lib().cq_matmul_multi(len(ops), wa, x.data_ptr(), xt, b * s, ya, xt, _stream_ptr(x.device))
    _check(st, "cq_matmul_multi", "multi input", [b * s, k], list(x.shape))
    return [y.reshape(b, s, -1).to(h.dtype) for y in ys]


class Linear:
    """enum Linear { Dense(Tensor), Quant(Box<dyn QuantLinearOp>) }
    (qlinear.rs:67-99).  The bias is added outside the op."""

    def __init__(self, dense=None, quant: Optional[QuantLinearOp] = None):
        if (dense is None) == (quant is None):
            raise ValueError("exactly one of dense / quant")
        self.dense, self.quant = dense, quant

    @classmethod
    def Dense(cls, w):
        return cls(dense=w)

    @classmethod
    def Quant(cls, op: QuantLinearOp):
        return cls(quant=op)

    def dims(self):
        return list(self.dense.shape) if self.dense is not None else self.quant.dims()

    def forward(self, x, bias=None):
        if self.dense is not None:
            # fp32 accumulation, output in the activation dtype
            out = (x.float() @ self.dense.t().float()).to(x.dtype)
            if bias is not None:
                out = out + bias.to(out.dtype).reshape(1, 1, -1)
            return out
        # quantized: the bias add runs in the kernels' epilogue
        return self.quant.forward(x) if bias is None else self.quant.forward_bias(x, bias)


def try_quant_linear(source, name: str, device=None) -> Optional[QuantLinearOp]:
    """try_quant_linear (qlinear.rs:284-339): the fast path for `name`, or
    None so the caller keeps its dense fallback.

    - COMBS_NO_QUANT_KERNELS set (and not "0") -> None (:291)
    - source has no packed tensor for `name`  -> None
    - not rank 2                              -> None
    - kernel-incompatible shape (BadShape)    -> None (:318-325)
    - errors from the source propagate (Err in the reference)
    """
    v = os.environ.get("COMBS_NO_QUANT_KERNELS")
    if v is not None and v != "0":
        return None
    qt = source.open_tensor_quant(name)
    if qt is None:
        return None
    if len(qt.shape) != 2:
        return None
    n_out, k = qt.shape
    try:
        w = QuantWeight.from_quant_tensor(qt.format, qt.data, n_out, k)
    except BadShape:
        return None
    return QuantLinearOp(w)


def dequantize_gpu(fmt, data) -> np.ndarray:
    """dequantize_*_gpu (qmatmul.rs:171-190, 530-573, 1232-1305): upload a
    block stream, run the bit-exact dequant kernel, return host f32."""
    torch = _torch()
    fmt = QuantFormat(fmt)
    buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, np.uint8)
    qk, bb = _BLOCK[fmt]
    if buf.size == 0 or buf.size % bb:
        raise BadShape(f"{fmt.name.lower()} block stream", [bb], [buf.size])
    n = buf.size // bb * qk
    d = torch.from_numpy(buf.copy()).cuda()
    out = torch.empty(n, dtype=torch.float32, device=d.device)
    st = L.lib().cq_dequantize(int(fmt), d.data_ptr(), buf.size, n, out.data_ptr(), _stream_ptr(d.device))
    _check(st, "cq_dequantize", f"{fmt.name.lower()} block stream", [bb], [buf.size])
    return out.cpu().numpy()


def quantize(fmt, values: np.ndarray, threads: int = 0) -> bytes:
    """Quantise f32 rows [rows, k] into the GGUF block stream (host, ggml's
    reference quantisers; input generation only)."""
    fmt = QuantFormat(fmt)
    v = np.ascontiguousarray(values, np.float32)
    if v.ndim == 1:
        v = v.reshape(1, -1)
    rows, k = v.shape
    nbytes = tensor_byte_size(fmt, rows, k)
    out = np.empty(nbytes, np.uint8)
    st = L.lib().cq_quantize(int(fmt), v.ctypes.data, rows, k, out.ctypes.data, nbytes, threads)
    _check(st, "cq_quantize", f"{fmt.name.lower()} quantize", [rows, k], [v.size])
    return out.tobytes()

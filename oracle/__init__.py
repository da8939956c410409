"""CPU oracle for the GGUF dequant-matmul path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline).
The product library never imports it and has no CPU fallback.

Thin numpy wrapper over oracle/gguf_oracle.c (see that file's header for the
reference citations and for what pins each function).  The synthetic block
generators below restate the reference's own test fixtures
(engine/core/combs-models/src/qmatmul.rs:1698-1829, 1974-1993).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

# GGML type ids (GGUF on-disk enum).
Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 6, 7, 8, 12, 13, 14
FORMATS = {"Q4_0": Q4_0, "Q4_1": Q4_1, "Q5_0": Q5_0, "Q5_1": Q5_1, "Q8_0": Q8_0,
           "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build as _b
            _b.build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_block_values.argtypes = [ctypes.c_int]
        L.orc_block_bytes.argtypes = [ctypes.c_int]
        L.orc_tensor_bytes.argtypes = [ctypes.c_int, i64]
        L.orc_tensor_bytes.restype = i64
        L.orc_scale_min_k4.argtypes = [ctypes.c_int, P, P, P]
        L.orc_dequant.argtypes = [ctypes.c_int, P, i64, i64, P]
        L.orc_dequant_mt.argtypes = [ctypes.c_int, P, i64, i64, P, ctypes.c_int]
        L.orc_ref_matmul.argtypes = [P, P, i64, i64, i64, P]
        L.orc_fused_matmul.argtypes = [ctypes.c_int, P, P, i64, i64, i64, P]
        L.orc_dense_gemm.argtypes = [P, P, i64, i64, i64, P, ctypes.c_int]
        L.orc_lcg_bytes.argtypes = [P, i64, ctypes.c_uint32]
        L.orc_synth_q4_0.argtypes = [P, i64, P]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def block_values(fmt: int) -> int:
    return lib().orc_block_values(fmt)


def block_bytes(fmt: int) -> int:
    return lib().orc_block_bytes(fmt)


def tensor_bytes(fmt: int, n_elems: int) -> int:
    return lib().orc_tensor_bytes(fmt, n_elems)


def scale_min_k4(j: int, scales12: bytes):
    q = np.frombuffer(bytes(scales12), dtype=np.uint8).copy()
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().orc_scale_min_k4(j, _p(q), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def dequant(fmt: int, data, n: int, threads: int = 0) -> np.ndarray:
    """gguf.rs dequantize_* for the block stream `data` (bytes or uint8 array)."""
    buf = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray)) else data, dtype=np.uint8)
    out = np.empty(n, np.float32)
    if threads:
        rc = lib().orc_dequant_mt(fmt, _p(buf), buf.size, n, _p(out), threads)
    else:
        rc = lib().orc_dequant(fmt, _p(buf), buf.size, n, _p(out))
    if rc != 0:
        raise ValueError(f"oracle dequant failed rc={rc} fmt={fmt} nbytes={buf.size} n={n}")
    return out


def ref_matmul(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """qmatmul.rs:1713-1725: sequential f32 y = x.W^T; x [m,k], w [n,k]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_ref_matmul(_p(x), _p(w), m, k, n, _p(out))
    return out


def fused_matmul(fmt: int, data, x: np.ndarray, n: int, k: int) -> np.ndarray:
    """The reference fused kernels' arithmetic (qmatmul.rs) restated on CPU.
    Q4_1 / Q5_1 have no fused kernel in the reference: their path is the
    dense one, dequantise (gguf.rs:798-874) then the f32 matmul
    (ref_matmul)."""
    buf = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray)) else data, dtype=np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    if fmt in (Q4_1, Q5_1):
        return ref_matmul(x, dequant(fmt, buf, n * k).reshape(n, k))
    m = x.shape[0]
    out = np.empty((m, n), np.float32)
    if lib().orc_fused_matmul(fmt, _p(buf), _p(x), m, n, k, _p(out)) != 0:
        raise ValueError("unsupported format")
    return out


def dense_gemm(x: np.ndarray, w: np.ndarray, threads: int = 1) -> np.ndarray:
    """The reference CPU path's per-call dense f32 matmul (timed baseline)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_dense_gemm(_p(x), _p(w), m, n, k, _p(out), threads)
    return out


# ---- the steps either side of the op ---------------------------------------

ACT_SILU, ACT_GELU_TANH, ACT_GELU = 0, 1, 2


def activation(kind: int, v) -> np.ndarray:
    """The gated MLP activations of combs-models act.rs:20-30, in float64:
    SiLU = burn's silu, x * sigmoid(x); GeluTanh = gelu_tanh (act.rs:10-17),
    x/2 * (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); Gelu = burn's exact
    gelu, x/2 * (1 + erf(x / sqrt(2))).  Pinned by act.rs:41-52's known
    values (GeluTanh), silu(x) - silu(-x) = x and silu(0) = 0, and the
    standard normal CDF, gelu(x) = x * Phi(x) (Phi(1) = 0.8413447460685429)."""
    from scipy.special import erf
    v = np.asarray(v, np.float64)
    if kind == ACT_SILU:
        return v / (1.0 + np.exp(-v))
    if kind == ACT_GELU_TANH:
        c = 0.7978845608028654  # sqrt(2/pi), act.rs:13
        return 0.5 * v * (1.0 + np.tanh(c * (v + 0.044715 * v ** 3)))
    if kind == ACT_GELU:
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    raise ValueError(f"unknown activation {kind}")


def linear(fmt: int, data, x: np.ndarray, n: int, k: int, bias=None) -> np.ndarray:
    """Linear::forward's quantized branch (qlinear.rs:84-98): the op's
    y = x . W^T (fused_matmul, the reference kernels' arithmetic) then
    `out + b` broadcast over rows; float64 result."""
    y = fused_matmul(fmt, data, x, n, k).astype(np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64).reshape(1, -1)
    return y


def gated_up(kind: int, gate, up, x: np.ndarray, n: int, k: int) -> np.ndarray:
    """llama.rs:301-303: act(gate.forward(h)) * up.forward(h); gate and up
    are (fmt, data) pairs of the same [n, k] shape; float64 result."""
    g = fused_matmul(gate[0], gate[1], x, n, k).astype(np.float64)
    u = fused_matmul(up[0], up[1], x, n, k).astype(np.float64)
    return activation(kind, g) * u


# ---- the reference's synthetic fixtures -----------------------------------

def lcg_bytes(n: int, seed: int) -> bytes:
    """qmatmul.rs:1784-1792 (lcg_bytes)."""
    out = np.empty(n, np.uint8)
    lib().orc_lcg_bytes(_p(out), n, seed & 0xFFFFFFFF)
    return out.tobytes()


def _f16le(v: float) -> bytes:
    return np.array([v], dtype=np.float32).astype(np.float16).tobytes()


def synth_q4_0(n_blocks: int) -> bytes:
    """qmatmul.rs:1698-1710: scale f16(0.003*((b%11)+1)), one running LCG."""
    sc = np.array([np.float32(0.003) * np.float32(b + 1.0) for b in range(11)], np.float32).astype(np.float16).view(np.uint16)
    sc = np.ascontiguousarray(sc)
    out = np.empty(n_blocks * 18, np.uint8)
    lib().orc_synth_q4_0(_p(out), n_blocks, _p(sc))
    return out.tobytes()


def synth_q4_k(n_sb: int) -> bytes:
    """qmatmul.rs:1795-1805."""
    parts = []
    for b in range(n_sb):
        d = np.float32(0.002) * np.float32((b % 9) + 1.0)
        dmin = np.float32(0.001) * np.float32((b % 5) + 1.0)
        parts += [_f16le(d), _f16le(dmin), lcg_bytes(140, 0xC0FFEE ^ b)]
    return b"".join(parts)


def synth_q5_k(n_sb: int) -> bytes:
    """qmatmul.rs:1808-1818."""
    parts = []
    for b in range(n_sb):
        d = np.float32(0.003) * np.float32((b % 7) + 1.0)
        dmin = np.float32(0.001) * np.float32((b % 5) + 1.0)
        parts += [_f16le(d), _f16le(dmin), lcg_bytes(172, 0x5EED ^ b)]
    return b"".join(parts)


def synth_q6_k(n_sb: int) -> bytes:
    """qmatmul.rs:1821-1829 (d last)."""
    parts = []
    for b in range(n_sb):
        d = np.float32(0.002) * np.float32((b % 9) + 1.0)
        parts += [lcg_bytes(208, 0xBEE5 ^ b), _f16le(d)]
    return b"".join(parts)


def synth_q5_0(n_blocks: int) -> bytes:
    """qmatmul.rs:1974-1982."""
    parts = []
    for b in range(n_blocks):
        d = np.float32(0.003) * np.float32((b % 11) + 1.0)
        parts += [_f16le(d), lcg_bytes(20, 0x51D0 ^ b)]
    return b"".join(parts)


def synth_q8_0(n_blocks: int) -> bytes:
    """qmatmul.rs:1985-1993."""
    parts = []
    for b in range(n_blocks):
        d = np.float32(0.003) * np.float32((b % 11) + 1.0)
        parts += [_f16le(d), lcg_bytes(32, 0x80C0 ^ b)]
    return b"".join(parts)


def synth_q4_1(n_blocks: int) -> bytes:
    """Not a reference fixture (the reference has no Q4_1 kernel test): the
    synth_q5_0 construction with a min, d = 0.003*((b%11)+1), m = -8d, then
    16 LCG bytes."""
    parts = []
    for b in range(n_blocks):
        d = np.float32(0.003) * np.float32((b % 11) + 1.0)
        parts += [_f16le(d), _f16le(-8 * d), lcg_bytes(16, 0x41D1 ^ b)]
    return b"".join(parts)


def synth_q5_1(n_blocks: int) -> bytes:
    """As synth_q4_1 for Q5_1: d, m = -16d, then 20 LCG bytes (qh, qs)."""
    parts = []
    for b in range(n_blocks):
        d = np.float32(0.003) * np.float32((b % 11) + 1.0)
        parts += [_f16le(d), _f16le(-16 * d), lcg_bytes(20, 0x51D1 ^ b)]
    return b"".join(parts)


SYNTH = {Q4_0: synth_q4_0, Q5_0: synth_q5_0, Q8_0: synth_q8_0, Q4_1: synth_q4_1, Q5_1: synth_q5_1,
         Q4_K: synth_q4_k, Q5_K: synth_q5_k, Q6_K: synth_q6_k}


def x_pattern(m: int, k: int, a: int = 7, b: int = 13, c: float = 6.0, s: float = 8.0) -> np.ndarray:
    """Activation patterns of the reference tests: ((i*a % b) - c)/s
    (qmatmul.rs:1767 (7,13,6,8), :2118 (11,29,14,16), :2144 (13,31,15,16))."""
    i = np.arange(m * k, dtype=np.int64)
    return (((i * a) % b).astype(np.float32) - np.float32(c)) / np.float32(s)


def assert_close(got, expect, rel: float, what: str = ""):
    """qmatmul.rs:1831-1837: |g - e| <= rel * max(|e|, 1) elementwise."""
    got = np.asarray(got, np.float64).ravel()
    expect = np.asarray(expect, np.float64).ravel()
    assert got.shape == expect.shape, f"{what}: length {got.shape} vs {expect.shape}"
    tol = rel * np.maximum(np.abs(expect), 1.0)
    bad = np.nonzero(np.abs(got - expect) > tol)[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}[{i}]: got {got[i]!r}, expect {expect[i]!r} "
                             f"({bad.size} of {got.size} outside rel {rel})")

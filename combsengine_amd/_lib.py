"""ctypes binding of the C ABI in include/combs_qlinear.h.

The library is the in-tree lib/libcombs_qlinear.so built by build.py.  There is
no fallback: importing a function that needs the library when it is missing
raises, so a GPU run can never silently take another path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libcombs_qlinear.so")

# Every symbol include/combs_qlinear.h declares.
EXPORTS = (
    "cq_block_values", "cq_block_bytes", "cq_tensor_bytes", "cq_weight_create",
    "cq_weight_wrap_device", "cq_weight_destroy", "cq_weight_dims", "cq_weight_vram_bytes",
    "cq_weight_device_ptr", "cq_matmul", "cq_matmul_path", "cq_matmul_bias", "cq_matmul_gate_up", "cq_matmul_multi",
    "cq_dequantize", "cq_quantize", "cq_matmul_kernels", "cq_reload_options", "cq_matmul_noalloc",
    "cq_device_init",
    "cq_last_error", "cq_version",
)

CQ_OK, CQ_ERR_BAD_FORMAT, CQ_ERR_BAD_SHAPE, CQ_ERR_BAD_DTYPE, CQ_ERR_NULL, CQ_ERR_HIP, CQ_ERR_NO_DEVICE = range(7)
CQ_F32, CQ_F16 = 0, 1
CQ_PATH_AUTO, CQ_PATH_GEMV, CQ_PATH_GEMM = 0, 1, 2
CQ_ACT_SILU, CQ_ACT_GELU_TANH, CQ_ACT_GELU = 0, 1, 2

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    """Load the library (once).  Raises LibraryMissing if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(f"{LIB_PATH} not found: run `python -c 'import __graft_entry__ as g; g.build()'` "
                             "(or python combsengine_amd/build.py) first")
    L = ctypes.CDLL(LIB_PATH)
    P, i64, sz, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
    sig = {
        "cq_block_values": ([i32], i32),
        "cq_block_bytes": ([i32], i32),
        "cq_tensor_bytes": ([i32, i64, i64, ctypes.POINTER(sz)], i32),
        "cq_weight_create": ([i32, P, sz, i64, i64, P, ctypes.POINTER(P)], i32),
        "cq_weight_wrap_device": ([i32, P, sz, i64, i64, ctypes.POINTER(P)], i32),
        "cq_weight_destroy": ([P], None),
        "cq_weight_dims": ([P, ctypes.POINTER(i64), ctypes.POINTER(i64)], i32),
        "cq_weight_vram_bytes": ([P], sz),
        "cq_weight_device_ptr": ([P], P),
        "cq_matmul": ([P, P, i32, i64, P, i32, P], i32),
        "cq_matmul_path": ([P, P, i32, i64, P, i32, i32, P], i32),
        "cq_matmul_bias": ([P, P, i32, i64, P, i32, P, i32, P], i32),
        "cq_matmul_gate_up": ([P, P, P, i32, i64, i32, P, i32, P], i32),
        "cq_matmul_multi": ([i32, P, P, i32, i64, P, i32, P], i32),
        "cq_dequantize": ([i32, P, sz, i64, P, P], i32),
        "cq_quantize": ([i32, P, i64, i64, P, sz, i32], i32),
        "cq_matmul_kernels": ([P, i32, i64, i32, ctypes.c_char_p, sz], i32),
        "cq_reload_options": ([], None),
        "cq_matmul_noalloc": ([P, P, i32, i64, P, i32, P], i32),
        "cq_device_init": ([], i32),
        "cq_last_error": ([], ctypes.c_char_p),
        "cq_version": ([], ctypes.c_char_p),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def last_error() -> str:
    return lib().cq_last_error().decode(errors="replace")


def reload_options() -> None:
    """Re-read the COMBS_* tuning variables (the library reads them once)."""
    lib().cq_reload_options()


def kernels(weight, x_dtype: int, m: int, y_dtype: int) -> str:
    """Names of the kernels cq_matmul launches for this call shape."""
    buf = ctypes.create_string_buffer(512)
    st = lib().cq_matmul_kernels(weight.handle, x_dtype, m, y_dtype, buf, 512)
    if st != CQ_OK:
        raise RuntimeError(last_error())
    return buf.value.decode()


def path_name(weight, x, y) -> str:
    """kernels() for device tensors x [m, k] and y [m, n]."""
    xt = CQ_F16 if str(x.dtype) == "torch.float16" else CQ_F32
    yt = CQ_F16 if str(y.dtype) == "torch.float16" else CQ_F32
    return kernels(weight, xt, x.shape[0], yt)

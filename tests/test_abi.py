"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad shapes/formats on the host before any
device work (the reference's BadShape rules, qmatmul.rs:2050-2081,
2156-2173), reporting a message through cq_last_error."""
import ctypes
import os
import re

import numpy as np
import pytest

from combsengine_amd import _lib as L
from combsengine_amd import BadShape, QuantFormat, tensor_byte_size

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "combs_qlinear.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(cq_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_header_symbol():
    lib = L.lib()
    syms = header_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), s
    assert sorted(L.EXPORTS) == syms


def test_version():
    assert b"gfx950" in L.lib().cq_version()


@pytest.mark.parametrize("fmt,qk,bb", [(2, 32, 18), (6, 32, 22), (8, 32, 34), (12, 256, 144), (13, 256, 176), (14, 256, 210)])
def test_block_sizes(fmt, qk, bb):
    assert L.lib().cq_block_values(fmt) == qk
    assert L.lib().cq_block_bytes(fmt) == bb


def test_tensor_bytes_and_errors():
    out = ctypes.c_size_t()
    assert L.lib().cq_tensor_bytes(12, 14336, 4096, ctypes.byref(out)) == L.CQ_OK
    assert out.value == 33030144
    assert L.lib().cq_tensor_bytes(12, 1, 128, ctypes.byref(out)) == L.CQ_ERR_BAD_SHAPE
    assert "multiple of 256" in L.last_error()
    # Q4_1 (3) / Q5_1 (7): 20 / 24 bytes per 32 values (gguf.rs:733-735)
    assert L.lib().cq_tensor_bytes(3, 2, 64, ctypes.byref(out)) == L.CQ_OK and out.value == 80
    assert L.lib().cq_tensor_bytes(7, 1, 32, ctypes.byref(out)) == L.CQ_OK and out.value == 24
    # Q4_1's neighbours in the ggml enum are not block formats served here
    assert L.lib().cq_tensor_bytes(4, 1, 32, ctypes.byref(out)) == L.CQ_ERR_BAD_FORMAT
    assert L.lib().cq_block_values(4) == 0 and L.lib().cq_block_values(1) == 0


@pytest.mark.parametrize("fmt,nbytes,n,k", [
    (2, 17, 1, 32),          # truncated block stream
    (2, 36, 2, 31),          # k not a block multiple
    (2, 36, 2, 64),          # byte count disagrees with [n, k]
    (6, 44, 2, 31), (8, 66, 2, 64),
    (12, 144, 1, 128),       # K-quant k must be a superblock multiple
    (14, 210, 1, 128),
])
def test_weight_create_rejects_on_host(fmt, nbytes, n, k):
    buf = np.zeros(nbytes, np.uint8)
    h = ctypes.c_void_p()
    st = L.lib().cq_weight_create(fmt, buf.ctypes.data, nbytes, n, k, None, ctypes.byref(h))
    assert st == L.CQ_ERR_BAD_SHAPE
    assert h.value is None
    assert L.last_error()
    st = L.lib().cq_weight_wrap_device(fmt, buf.ctypes.data, nbytes, n, k, ctypes.byref(h))
    assert st == L.CQ_ERR_BAD_SHAPE


def test_null_arguments():
    h = ctypes.c_void_p()
    assert L.lib().cq_weight_create(12, None, 144, 1, 256, None, ctypes.byref(h)) == L.CQ_ERR_NULL
    assert L.lib().cq_matmul(None, None, 1, 1, None, 0, None) == L.CQ_ERR_NULL
    assert L.lib().cq_weight_vram_bytes(None) == 0


def test_python_tensor_byte_size():
    assert tensor_byte_size(QuantFormat.Q6K, 128256, 4096) == 430940160
    with pytest.raises(BadShape):
        tensor_byte_size(QuantFormat.Q4K, 1, 128)

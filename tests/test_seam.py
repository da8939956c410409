"""The quantized-linear seam (engine/core/combs-models/src/qlinear.rs):
dispatch rules on the CPU, Linear forward parity on the GPU
(qlinear.rs:341-475 compares a quant Linear with the dense Linear over the
dequantised weight, with bias: 1e-4 in f32, 1e-2 in f16)."""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import BadShape, Linear, QuantFormat, QuantLinearOp, QuantTensor, QuantWeight, try_quant_linear


class FakeSource:
    """ModelSource::open_tensor_quant stand-in (source.rs:35)."""

    def __init__(self, tensors):
        self.tensors = tensors
        self.calls = []

    def open_tensor_quant(self, name):
        self.calls.append(name)
        return self.tensors.get(name)


def test_no_quant_kernels_env(monkeypatch):
    monkeypatch.setenv("COMBS_NO_QUANT_KERNELS", "1")
    src = FakeSource({"w": QuantTensor(QuantFormat.Q4K, [1, 256], O.synth_q4_k(1))})
    assert try_quant_linear(src, "w") is None
    assert src.calls == []  # checked before touching the source (qlinear.rs:291)


def test_missing_and_non_2d_fall_back():
    src = FakeSource({"v": QuantTensor(QuantFormat.Q8_0, [32], O.synth_q8_0(1))})
    assert try_quant_linear(src, "absent") is None
    assert try_quant_linear(src, "v") is None


def test_bad_shape_falls_back_without_device():
    # k = 128 is not a K-quant superblock multiple: dense fallback, not an error
    src = FakeSource({"w": QuantTensor(QuantFormat.Q4K, [1, 128], O.synth_q4_k(1))})
    assert try_quant_linear(src, "w") is None
    with pytest.raises(BadShape):
        QuantWeight.from_gguf_bytes(QuantFormat.Q4_0, O.synth_q4_0(2), 2, 31)
    with pytest.raises(BadShape):
        QuantWeight.from_gguf_bytes(QuantFormat.Q4_0, O.synth_q4_0(2), 2, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [QuantFormat.Q4_0, QuantFormat.Q8_0, QuantFormat.Q4K, QuantFormat.Q6K])
def test_quant_linear_matches_dense(cuda, fmt):
    import torch
    n, k = 64, 512
    data = O.SYNTH[int(fmt)](n * k // O.block_values(int(fmt)))
    src = FakeSource({"model.layers.0.mlp.up_proj.weight": QuantTensor(fmt, [n, k], data)})
    op = try_quant_linear(src, "model.layers.0.mlp.up_proj.weight")
    assert isinstance(op, QuantLinearOp)
    assert op.dims() == [n, k] and op.vram_bytes() == len(data)
    wd = torch.from_numpy(O.dequant(int(fmt), data, n * k).reshape(n, k)).cuda()
    bias = torch.linspace(-1, 1, n, device="cuda")
    x = torch.from_numpy(O.x_pattern(2 * 3, k).reshape(2, 3, k)).cuda()
    quant, dense = Linear.Quant(op), Linear.Dense(wd)
    assert quant.dims() == dense.dims()
    q32, d32 = quant.forward(x, bias), dense.forward(x, bias)
    assert q32.shape == (2, 3, n) and q32.dtype == torch.float32
    O.assert_close(q32.cpu().numpy(), d32.cpu().numpy(), 1e-4 if fmt == QuantFormat.Q4_0 else 1e-3, "f32")
    q16, d16 = quant.forward(x.half(), bias), dense.forward(x.half(), bias)
    assert q16.dtype == torch.float16
    O.assert_close(q16.float().cpu().numpy(), d16.float().cpu().numpy(), 1e-2, "f16")
    # bf16 activations: cast to fp32 around the launch, result cast back
    # (the reference casts every non-f32 input, qlinear.rs:126-143)
    xb = x.bfloat16()
    qb = quant.forward(xb, bias)
    assert qb.dtype == torch.bfloat16 and qb.shape == (2, 3, n)
    db = dense.forward(xb.float(), bias).bfloat16()
    O.assert_close(qb.float().cpu().numpy(), db.float().cpu().numpy(), 1e-2, "bf16")
    assert op.forward(xb).dtype == torch.bfloat16

"""GPU parity of the fused output epilogues against the CPU oracle, through
the C ABI: the bias add of Linear::forward (qlinear.rs:84-98) and the gated
MLP product act(gate(h)) * up(h) (llama.rs:301-303, act.rs:20-30).

Every kernel path is covered: the single-row GEMV (m = 1), the MFMA GEMV
(m = 4), the prefill GEMM (m >= 64, with and without split K, whose reduction
applies the epilogue) and the fp32-activation GEMM.  Expected values come
from the oracle's fused matmul in float64; the bar is the matmul's own,
|g - e| <= rel * max(|e|, 1)."""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import Activation, Linear, QuantFormat, QuantLinearOp, QuantWeight, gated_up, quantize
from combsengine_amd import _lib as L

pytestmark = pytest.mark.gpu

FMTS = [QuantFormat.Q4_0, QuantFormat.Q5_0, QuantFormat.Q8_0, QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K]
KQ = [QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K]
ALL_FMTS = FMTS + [QuantFormat.Q4_1, QuantFormat.Q5_1]


def _weight(fmt, n, k, seed):
    rng = np.random.default_rng(seed)
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return data, QuantWeight.from_gguf_bytes(fmt, data, n, k)


def _x(m, k, seed):
    return np.random.default_rng(seed).normal(0, 1, (m, k)).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 4, 12, 64])
@pytest.mark.parametrize("bias_dt", ["f32", "f16"])
@pytest.mark.parametrize("y_dt", ["f32", "f16"])
def test_bias_epilogue(cuda, fmt, m, bias_dt, y_dt):
    import torch
    n, k = 300, 2048
    data, w = _weight(fmt, n, k, 10 + int(fmt))
    x = _x(m, k, m)
    b = np.random.default_rng(7).normal(0, 2, n).astype(np.float32)
    bt = torch.float32 if bias_dt == "f32" else torch.float16
    b = b.astype(np.float16).astype(np.float32) if bias_dt == "f16" else b
    if y_dt == "f16":
        # the reference's fp16 model: the op's output in fp16, then `+ b` in fp16
        # (qlinear.rs:84-98, 126-143); the bar carries the two fp16 roundings
        expect = O.fused_matmul(int(fmt), data, x, n, k).astype(np.float16).astype(np.float64) + b
    else:
        expect = O.linear(int(fmt), data, x, n, k, b)
    print(f"bias {fmt.name} m={m} bias={bias_dt} y={y_dt}", flush=True)
    yt = torch.float32 if y_dt == "f32" else torch.float16
    y = torch.empty((m, n), dtype=yt, device="cuda")
    w.matmul_bias_into(torch.from_numpy(x).cuda().half(), torch.from_numpy(b).cuda().to(bt), y)
    O.assert_close(y.float().cpu().numpy(), expect, 1e-4 if fmt == QuantFormat.Q4_0 and y_dt == "f32" else
                   1e-3 if y_dt == "f32" else 2e-3)


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("split", ["1", "3"])
def test_bias_epilogue_prefill_split_and_fp32_x(cuda, monkeypatch, fmt, split):
    """The split-K reduction applies the bias; fp32 activations take the
    fp32-x GEMM, whose epilogue is the same."""
    import torch
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", split)
    n, k, m = 200, 3072, 130
    data, w = _weight(fmt, n, k, 20 + int(fmt))
    x = _x(m, k, 3)
    b = np.random.default_rng(8).normal(0, 1, n).astype(np.float32)
    expect = O.linear(int(fmt), data, x, n, k, b)
    print(f"bias prefill {fmt.name} split={split}", flush=True)
    for xt in (torch.float16, torch.float32):
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        w.matmul_bias_into(torch.from_numpy(x).cuda().to(xt), torch.from_numpy(b).cuda(), y)
        O.assert_close(y.cpu().numpy(), expect, 1e-3, f"x {xt}")


def test_bias_none_equals_matmul(cuda):
    import torch
    data, w = _weight(QuantFormat.Q4K, 100, 1024, 5)
    x = torch.from_numpy(_x(3, 1024, 1)).cuda().half()
    a = torch.empty((3, 100), device="cuda")
    b = torch.empty((3, 100), device="cuda")
    w.matmul_into(x, a)
    w.matmul_bias_into(x, None, b)
    assert torch.equal(a, b)


PAIRS = [(QuantFormat.Q4K, QuantFormat.Q4K), (QuantFormat.Q4K, QuantFormat.Q6K), (QuantFormat.Q8_0, QuantFormat.Q5_0),
         (QuantFormat.Q4_1, QuantFormat.Q5_1)]


@pytest.mark.parametrize("gf,uf", PAIRS)
@pytest.mark.parametrize("act", [Activation.Silu, Activation.GeluTanh, Activation.Gelu])
@pytest.mark.parametrize("m", [1, 4, 12, 64, 130])
@pytest.mark.parametrize("y_dt", ["f32", "f16"])
def test_gate_up_epilogue(cuda, gf, uf, act, m, y_dt):
    """y = act(x.G^T) * (x.U^T).  With an fp16 output the library rounds the
    gate and up products to fp16 (as the reference's f16 model rounds every
    projection), so the expected value does too; the bar then carries the
    fp16 roundings (2^-11 relative each) on top of the matmul's 1e-3."""
    import torch
    n, k = 260, 2048
    gd, gw = _weight(gf, n, k, 30 + int(gf))
    ud, uw = _weight(uf, n, k, 40 + int(uf))
    x = _x(m, k, 50 + m)
    g = O.fused_matmul(int(gf), gd, x, n, k).astype(np.float64)
    u = O.fused_matmul(int(uf), ud, x, n, k).astype(np.float64)
    if y_dt == "f16":
        g, u = g.astype(np.float16).astype(np.float64), u.astype(np.float16).astype(np.float64)
    expect = O.activation(int(act), g) * u
    print(f"gate_up {gf.name}/{uf.name} {act.name} m={m} y={y_dt}", flush=True)
    h = torch.from_numpy(x).cuda().half().reshape(1, m, k)
    if y_dt == "f32":
        h = h.float()  # y follows h's dtype; fp32 h takes the fp32-x kernels
    y = gated_up(act, QuantLinearOp(gw), QuantLinearOp(uw), h)
    assert y.shape == (1, m, n) and y.dtype == h.dtype
    O.assert_close(y.float().cpu().numpy(), expect, 1e-3 if y_dt == "f32" else 2e-3)


@pytest.mark.parametrize("fmt", ALL_FMTS)
@pytest.mark.parametrize("n,k", [(300, 4096), (257, 256), (45, 1024), (97, 3584), (50, 768)])
@pytest.mark.parametrize("m", [2, 7, 16])
@pytest.mark.parametrize("act", [Activation.Silu, Activation.Gelu])
def test_gate_up_batched_one_launch(cuda, monkeypatch, fmt, n, k, m, act):
    """Batched decode of the gated gate / up pair (fp16 h, 2 <= m <= 16): one
    launch of the column kernel whose tiles hold 8 gate rows and the same 8
    up rows (ragged last tile: n not a multiple of 8), the product
    act(fp16(g)) * fp16(u) formed where the rows' sums are added; against the
    oracle and the two-launch path (COMBS_GATEUP_FUSED=0)."""
    import torch
    gd, gw = _weight(fmt, n, k, 70 + int(fmt))
    ud, uw = _weight(fmt, n, k, 80 + int(fmt))
    x = _x(m, k, 90 + m)
    g = O.fused_matmul(int(fmt), gd, x, n, k).astype(np.float16).astype(np.float64)
    u = O.fused_matmul(int(fmt), ud, x, n, k).astype(np.float16).astype(np.float64)
    expect = O.activation(int(act), g) * u
    print(f"gate_up batched {fmt.name} [{n}x{k}] m={m} {act.name}", flush=True)
    h = torch.from_numpy(x).cuda().half().reshape(1, m, k)
    y = gated_up(act, QuantLinearOp(gw), QuantLinearOp(uw), h)
    O.assert_close(y.float().cpu().numpy().reshape(m, n), expect, 2e-3)
    monkeypatch.setenv("COMBS_GATEUP_FUSED", "0")
    y2 = gated_up(act, QuantLinearOp(gw), QuantLinearOp(uw), h)
    O.assert_close(y.float().cpu().numpy(), y2.float().cpu().numpy(), 2e-3, "vs two launches")


@pytest.mark.parametrize("split", ["1", "4"])
def test_gate_up_prefill_split(cuda, monkeypatch, split):
    import torch
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", split)
    n, k, m = 300, 4096, 200
    gd, gw = _weight(QuantFormat.Q4K, n, k, 61)
    ud, uw = _weight(QuantFormat.Q4K, n, k, 62)
    x = _x(m, k, 63)
    expect = O.gated_up(O.ACT_SILU, (int(QuantFormat.Q4K), gd), (int(QuantFormat.Q4K), ud), x, n, k)
    print(f"gate_up prefill split={split}", flush=True)
    y = torch.empty((m, n), device="cuda")
    st = L.lib().cq_matmul_gate_up(gw.handle, uw.handle, torch.from_numpy(x).cuda().half().data_ptr(), L.CQ_F16, m,
                                   L.CQ_ACT_SILU, y.data_ptr(), L.CQ_F32, 0)
    assert st == L.CQ_OK, L.last_error()
    torch.cuda.synchronize()
    O.assert_close(y.cpu().numpy(), expect, 1e-3)


def test_linear_forward_bias_fused(cuda):
    """Linear::forward with a bias (qlinear.rs:84-98) on the quantized branch
    takes the fused epilogue and matches the dense branch's definition."""
    import torch
    n, k = 128, 1024
    data, w = _weight(QuantFormat.Q6K, n, k, 70)
    x = _x(6, k, 71)
    b = np.random.default_rng(72).normal(0, 1, n).astype(np.float32)
    lin = Linear.Quant(QuantLinearOp(w))
    out = lin.forward(torch.from_numpy(x).cuda().float().reshape(2, 3, k), torch.from_numpy(b).cuda())
    assert out.shape == (2, 3, n)
    O.assert_close(out.cpu().numpy().reshape(6, n), O.linear(int(QuantFormat.Q6K), data, x, n, k, b), 1e-3)


def test_gate_up_rejects_mismatched_shapes(cuda):
    import torch
    _, a = _weight(QuantFormat.Q4K, 64, 512, 1)
    _, b = _weight(QuantFormat.Q4K, 32, 512, 2)
    x = torch.zeros((1, 512), dtype=torch.float16, device="cuda")
    y = torch.zeros((1, 64), device="cuda")
    st = L.lib().cq_matmul_gate_up(a.handle, b.handle, x.data_ptr(), L.CQ_F16, 1, L.CQ_ACT_SILU, y.data_ptr(),
                                   L.CQ_F32, 0)
    assert st == L.CQ_ERR_BAD_SHAPE and "differ" in L.last_error()
    st = L.lib().cq_matmul_gate_up(a.handle, a.handle, x.data_ptr(), L.CQ_F16, 1, 7, y.data_ptr(), L.CQ_F32, 0)
    assert st == L.CQ_ERR_BAD_SHAPE


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("g2", ["0", "2"])
@pytest.mark.parametrize("n,k", [(140000, 256), (3000, 512), (700, 4096), (300, 5120), (301, 18944)])
def test_epilogue_single_row_kernels(cuda, monkeypatch, fmt, g2, n, k):
    """m = 1 epilogues of both single-row kernels: the streaming kernel
    (COMBS_GEMV2=2) preloads each wave's first 64 rows' bias / gate values and
    loads the rest at store time (n = 140000 puts ~68 rows on a wave), with R
    rows per step (k = 256, 512) or several steps per row (k = 5120); the
    whole-superblock kernel (=0) loads them at store time; k = 18944 runs
    the half-row wave-pair kernel (cq_gemv1k) either way."""
    import torch
    monkeypatch.setenv("COMBS_GEMV2", g2)
    data, w = _weight(fmt, n, k, 80 + int(fmt))
    x = _x(1, k, 81)
    b = np.random.default_rng(82).normal(0, 1, n).astype(np.float32)
    print(f"single-row epilogue {fmt.name} gemv2={g2} n={n} k={k}", flush=True)
    y = torch.empty((1, n), device="cuda")
    w.matmul_bias_into(torch.from_numpy(x).cuda().half(), torch.from_numpy(b).cuda(), y)
    O.assert_close(y.cpu().numpy(), O.linear(int(fmt), data, x, n, k, b), 1e-3, "bias")
    # gate(x) * silu: the same weight as gate and up
    g = gated_up(Activation.Silu, QuantLinearOp(w), QuantLinearOp(w), torch.from_numpy(x).cuda().float().reshape(1, 1, k)
                 .half())
    yy = O.fused_matmul(int(fmt), data, x, n, k).astype(np.float64)
    y16 = yy.astype(np.float16).astype(np.float64)
    expect = O.activation(O.ACT_SILU, y16) * y16
    O.assert_close(g.float().cpu().numpy().reshape(1, n), expect, 2e-3, "gate_up")




@pytest.mark.parametrize("fmt", ALL_FMTS)
@pytest.mark.parametrize("n,k", [(300, 4096), (257, 256), (130, 8192), (45, 1024), (97, 3584), (50, 768),
                                 (33, 5120), (40, 16384)])
@pytest.mark.parametrize("fused", ["1", "0"])
@pytest.mark.parametrize("y_dt", ["f32", "f16"])
@pytest.mark.parametrize("spread", ["1", "0"])
def test_gate_up_single_row_one_launch(cuda, monkeypatch, fmt, n, k, fused, y_dt, spread):
    """m = 1, fp16 x, gate and up of one format: the one-launch kernel (both
    weights against one activation staging, floor(R/2) gate and up rows per
    task, ragged last task; K = 768: 21-row tasks with a lane row left over,
    K = 3584 / 5120: row sums over the whole wave) for K/256 up to 32 where
    the weights suit the span loads; K = 16384 (64 units, one row per task)
    and COMBS_GATEUP_FUSED=0 take the two-launch path.  With fp16 y both
    paths round the gate and up products to fp16 before the activation and
    the product, as the reference's fp16 model rounds each projection."""
    import torch
    monkeypatch.setenv("COMBS_GATEUP_FUSED", fused)
    monkeypatch.setenv("COMBS_GEMV1_SPREAD", spread)  # tasks wave-major over the grid, or packed
    gd, gw = _weight(fmt, n, k, 90 + int(fmt))
    ud, uw = _weight(fmt, n, k, 95 + int(fmt))
    x = _x(1, k, 96)
    g = O.fused_matmul(int(fmt), gd, x, n, k).astype(np.float64)
    u = O.fused_matmul(int(fmt), ud, x, n, k).astype(np.float64)
    if y_dt == "f16":
        g, u = g.astype(np.float16).astype(np.float64), u.astype(np.float16).astype(np.float64)
    expect = O.activation(O.ACT_GELU_TANH, g) * u
    print(f"gate_up m=1 {fmt.name} n={n} k={k} fused={fused} y={y_dt}", flush=True)
    h = torch.from_numpy(x).cuda().half().reshape(1, 1, k)
    yt = torch.float32 if y_dt == "f32" else torch.float16
    y = torch.empty((1, n), dtype=yt, device="cuda")
    st = L.lib().cq_matmul_gate_up(gw.handle, uw.handle, h.data_ptr(), L.CQ_F16, 1, L.CQ_ACT_GELU_TANH, y.data_ptr(),
                                   L.CQ_F32 if y_dt == "f32" else L.CQ_F16, 0)
    assert st == L.CQ_OK, L.last_error()
    torch.cuda.synchronize()
    O.assert_close(y.float().cpu().numpy(), expect, 1e-3 if y_dt == "f32" else 2e-3)


@pytest.mark.parametrize("fmt", [QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K, QuantFormat.Q4_0,
                                 QuantFormat.Q8_0, QuantFormat.Q5_0])
@pytest.mark.parametrize("ns,k", [((4096, 1024, 1024), 4096), ((512, 128, 128, 64), 1024), ((300, 36), 2304),
                                  ((96,), 16384), ((3584, 512, 512), 3584)])
@pytest.mark.parametrize("m", [1, 3, 9, 16])
def test_matmul_multi(cuda, monkeypatch, fmt, ns, k, m):
    """Several projections of one input (q / k / v, llama.rs:261-263): one
    launch for decode where every weight's rows fill whole tasks (fp16-register
    formats) at m = 1, one launch of the batched column kernel over every
    weight's tiles at 2 <= m <= 16 (rows of at most 16 columns: ragged tiles
    at segment ends, up to 4 weights), else one call per weight; each output
    against the oracle, and equal to the separate launches
    (COMBS_MULTI_FUSED=0) to the same bar."""
    import torch
    from combsengine_amd import multi_forward
    ws = [_weight(fmt, n, k, 60 + i + int(fmt)) for i, n in enumerate(ns)]
    x = _x(m, k, 61)
    h = torch.from_numpy(x).cuda().half().reshape(1, m, k)
    ops = [QuantLinearOp(w) for _, w in ws]
    print(f"multi {fmt.name} ns={ns} k={k} m={m} kernels={L.kernels(ws[0][1], L.CQ_F16, m, L.CQ_F16)}", flush=True)
    ys = multi_forward(ops, h)
    monkeypatch.setenv("COMBS_MULTI_FUSED", "0")
    ys_sep = multi_forward(ops, h)
    for (data, w), n, y, ysep in zip(ws, ns, ys, ys_sep):
        assert y.shape == (1, m, n) and y.dtype == torch.float16
        expect = O.fused_matmul(int(fmt), data, x, n, k)
        O.assert_close(y.float().cpu().numpy().reshape(m, n), expect, 2e-3, f"n={n}")
        O.assert_close(y.float().cpu().numpy(), ysep.float().cpu().numpy(), 2e-3, f"n={n} vs separate")

"""Tiling invariants and many-task launches (GPU, through the C ABI).

The reference checks that its tiled and untiled kernels agree bit for bit
(qmatmul.rs:2083-2154): both accumulate each output in the same order.  The
kernels here have the same property wherever only the work distribution
changes, so these tests require bit-identical outputs across:
  * cq_gemv1's grid size and task placement (COMBS_GEMV1_GRID,
    COMBS_GEMV1_SPREAD): a row's sum does not depend on which wave runs it;
  * cq_gemm2's tile shape (COMBS_GEMM2_NT, COMBS_GEMM2_MT);
  * cq_gemvd's row tiles per workgroup (COMBS_GVD_NT) at a fixed wave count;
  * cq_gemvq's workgroup count (COMBS_GEMVQ_GROUPS): which workgroup runs a
    tile, and where the reduction chunks fall, changes no sum.
Grids of one to three workgroups also give every wave of cq_gemv1 dozens of
tasks, so its two-slice task loop runs through every branch, for each
format, with no epilogue, a bias epilogue and the one-launch gated gate/up;
all are checked against the oracle too.
"""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat as F
from combsengine_amd import QuantWeight, dequantize_gpu, quantize
from combsengine_amd import _lib as L

pytestmark = pytest.mark.gpu

ALL = [F.Q4_0, F.Q5_0, F.Q8_0, F.Q4K, F.Q5K, F.Q6K, F.Q4_1, F.Q5_1]
KQ = [F.Q4K, F.Q5K, F.Q6K]


def _weight(fmt, n, k, seed):
    data = quantize(fmt, np.random.default_rng(seed).normal(0, 0.02, (n, k)).astype(np.float32))
    return data, QuantWeight.from_gguf_bytes(fmt, data, n, k)


def _x(m, k, seed):
    return np.random.default_rng(seed).normal(0, 1, (m, k)).astype(np.float16).astype(np.float32)


def _bits(t):
    return t.float().cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("fmt", ALL)
@pytest.mark.parametrize("n,k", [(4096, 4096), (1003, 2048), (700, 16384)])
def test_gemv1_many_tasks_per_wave(cuda, monkeypatch, fmt, n, k):
    """m = 1 on 1, 2 and 3 workgroups (tasks packed, so each wave runs up to
    ~130 tasks) and on the default grid: oracle parity for y, y + bias and
    the gated gate/up, and bit-identical results across the grids."""
    import torch
    data, w = _weight(fmt, n, k, 700 + int(fmt) + k)
    udata, uw = _weight(fmt, n, k, 800 + int(fmt) + k)
    x = _x(1, k, 5)
    b = np.random.default_rng(6).normal(0, 1, n).astype(np.float32)
    y_ref = O.fused_matmul(int(fmt), data, x, n, k).astype(np.float64)
    u_ref = O.fused_matmul(int(fmt), udata, x, n, k).astype(np.float64)
    xd = torch.from_numpy(x).cuda().half()
    bd = torch.from_numpy(b).cuda()
    s = torch.cuda.current_stream().cuda_stream
    runs = {}
    # one arithmetic path throughout (the int8-activation kernels that small
    # Q4_0 / Q8_0 weights take by default differ in the last bits): the
    # fp16-register kernels where they serve the format
    monkeypatch.setenv("COMBS_GEMV1_I8", "0")
    monkeypatch.setenv("COMBS_GEMVR", "0")  # cq_gemv1 on every grid
    monkeypatch.setenv("COMBS_GEMV2", "-1")
    for grid in ("1", "2", "3", "default"):
        if grid == "default":
            monkeypatch.delenv("COMBS_GEMV1_GRID", raising=False)
            monkeypatch.setenv("COMBS_GEMV1_SPREAD", "1")
        else:
            monkeypatch.setenv("COMBS_GEMV1_GRID", grid)
            monkeypatch.setenv("COMBS_GEMV1_SPREAD", "0")
        y = torch.empty((1, n), device="cuda")
        kern = L.path_name(w, xd, y)
        print(f"{fmt.name} n={n} k={k} grid={grid} kernel={kern}", flush=True)
        w.matmul_into(xd, y)
        yb = torch.empty((1, n), device="cuda")
        w.matmul_bias_into(xd, bd, yb)
        yg = torch.empty((1, n), device="cuda")
        st = L.lib().cq_matmul_gate_up(w.handle, uw.handle, xd.data_ptr(), L.CQ_F16, 1, L.CQ_ACT_SILU,
                                       yg.data_ptr(), L.CQ_F32, s)
        assert st == L.CQ_OK, L.last_error()
        torch.cuda.synchronize()
        O.assert_close(y.cpu().numpy(), y_ref, 1e-3, f"y grid={grid}")
        O.assert_close(yb.cpu().numpy(), y_ref + b, 1e-3, f"bias grid={grid}")
        O.assert_close(yg.cpu().numpy(), O.activation(O.ACT_SILU, y_ref) * u_ref, 1e-3, f"gated grid={grid}")
        runs[grid] = (_bits(y), _bits(yb), _bits(yg))
    for grid, r in runs.items():
        for a, c in zip(r, runs["1"]):
            assert np.array_equal(a, c), f"grid {grid} differs from grid 1"


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("m", [130, 300])
def test_gemm2_tile_shapes_bit_identical(cuda, monkeypatch, fmt, m):
    """Every (NT, MT) tile shape of the prefill GEMM gives the same bits."""
    import torch
    n, k = 520, 2048
    data, w = _weight(fmt, n, k, 900 + int(fmt))
    x = torch.from_numpy(_x(m, k, 9)).cuda().half()
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", "1")
    outs = {}
    for nt, mt in (("1", "4"), ("1", "8"), ("1", "16"), ("2", "8"), ("2", "16")):
        monkeypatch.setenv("COMBS_GEMM2_NT", nt)
        monkeypatch.setenv("COMBS_GEMM2_MT", mt)
        y = torch.empty((m, n), device="cuda")
        w.matmul_into(x, y, path=L.CQ_PATH_GEMM)
        torch.cuda.synchronize()
        outs[(nt, mt)] = _bits(y)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    O.assert_close(outs[("1", "8")].view(np.float32), x.float().cpu().numpy().astype(np.float64) @ wd.T.astype(
        np.float64), 1e-3, "gemm2")
    for key, v in outs.items():
        assert np.array_equal(v, outs[("1", "8")]), f"tile {key} differs from (1, 8)"


@pytest.mark.parametrize("fmt", [F.Q4_0, F.Q5_0, F.Q8_0, F.Q4_1, F.Q5_1])
@pytest.mark.parametrize("m", [17, 64, 130])
def test_gemml_tile_shapes_bit_identical(cuda, monkeypatch, fmt, m):
    """Legacy-format prefill: 64- and 128-row activation tiles and one or two
    weight tiles per wave give the same bits (the K split held fixed)."""
    import torch
    n, k = 520, 2048
    data, w = _weight(fmt, n, k, 910 + int(fmt))
    x = torch.from_numpy(_x(m, k, 12)).cuda().half()
    monkeypatch.setenv("COMBS_GEMML_SPLIT", "2")
    outs = {}
    for mt, nt in (("4", "1"), ("8", "1"), ("8", "2")):
        monkeypatch.setenv("COMBS_GEMML_MT", mt)
        monkeypatch.setenv("COMBS_GEMML_NT", nt)
        y = torch.empty((m, n), device="cuda")
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        outs[(mt, nt)] = _bits(y)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    O.assert_close(outs[("8", "1")].view(np.float32), x.float().cpu().numpy().astype(np.float64) @ wd.T.astype(
        np.float64), 1e-3, "gemml")
    for key, v in outs.items():
        assert np.array_equal(v, outs[("8", "1")]), f"tile {key} differs from (8, 1)"


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("nw", ["2", "4"])
def test_gemvd_row_tiles_bit_identical(cuda, monkeypatch, fmt, nw):
    """Batched decode: 1, 2 or 4 row tiles per workgroup at a fixed wave
    count give the same bits."""
    import torch
    n, k, m = 600, 4096, 9
    data, w = _weight(fmt, n, k, 950 + int(fmt))
    x = torch.from_numpy(_x(m, k, 10)).cuda().half()
    monkeypatch.setenv("COMBS_GEMVQ", "0")  # cq_gemvd_*
    monkeypatch.setenv("COMBS_GEMVS", "0")
    monkeypatch.setenv("COMBS_GVD_WAVES", nw)
    outs = {}
    for nt in ("1", "2", "4"):
        monkeypatch.setenv("COMBS_GVD_NT", nt)
        y = torch.empty((m, n), device="cuda")
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        outs[nt] = _bits(y)
    for nt, v in outs.items():
        assert np.array_equal(v, outs["1"]), f"NT={nt} differs from NT=1"


@pytest.mark.parametrize("fmt", ALL)
@pytest.mark.parametrize("m", [3, 16])
@pytest.mark.parametrize("msum", ["0", "2"])
def test_gemvq_groups_bit_identical(cuda, monkeypatch, fmt, m, msum):
    """Batched decode through the column kernel: 1, 5, 64 workgroups and the
    default grid give the same bits, for each way of forming the Q4_K / Q5_K
    min term (8 MFMAs against the mins, or one against the column's
    sub-block sums: COMBS_GEMVQ_MSUM=0 / 2; by default the grid picks)."""
    import torch
    monkeypatch.setenv("COMBS_GEMVQ_MSUM", msum)
    n, k = 1300, 3584
    data, w = _weight(fmt, n, k, 960 + int(fmt))
    x = torch.from_numpy(_x(m, k, 11)).cuda().half()
    outs = {}
    for gr in ("0", "1", "5", "64"):
        monkeypatch.setenv("COMBS_GEMVQ_GROUPS", gr)
        assert L.path_name(w, x, torch.empty((m, n), device="cuda")).startswith("cq_gemvq_")
        y = torch.empty((m, n), device="cuda")
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        outs[gr] = _bits(y)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    O.assert_close(outs["0"].view(np.float32), _x(m, k, 11).astype(np.float64) @ wd.T.astype(np.float64),
                   1e-3, "gemvq")
    for gr, v in outs.items():
        assert np.array_equal(v, outs["0"]), f"{gr} workgroups differ from the default grid"


def test_dequant_rounding_blocks_bit_exact(cuda):
    """The oracle-pinning blocks (random non-power-of-two d, dmin, scales,
    signed zeros) through the GPU dequant: bit-identical to the oracle."""
    import importlib.util
    import os
    spec = importlib.util.spec_from_file_location(
        "rounding", os.path.join(os.path.dirname(__file__), "test_oracle_rounding.py"))
    R = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(R)
    rng = np.random.default_rng(77)
    blocks = {F.Q4K: R._kq_blocks(rng, O.Q4_K), F.Q5K: R._kq_blocks(rng, O.Q5_K), F.Q6K: R._q6_blocks(rng),
              F.Q4_1: R._q51_blocks(rng, O.Q4_1), F.Q5_1: R._q51_blocks(rng, O.Q5_1)}
    for fmt, blk in blocks.items():
        got = dequantize_gpu(fmt, blk.tobytes())
        want = O.dequant(int(fmt), blk.tobytes(), got.size)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), fmt.name


@pytest.mark.parametrize("fmt", [F.Q4K, F.Q5K])
@pytest.mark.parametrize("m", [2, 9, 16])
@pytest.mark.parametrize("n,k", [(1300, 3584), (520, 4096), (300, 14336)])
def test_gemvq_min_term_sums_close(cuda, monkeypatch, fmt, m, n, k):
    """The batched decode's two ways of forming the Q4_K / Q5_K min term —
    eight MFMAs of the activations against the mins, or one against the
    column's sub-block sums (sum / 64 split into fp16 hi + lo) — differ
    only by the sums' rounding (about 22 bits): the outputs agree to 1e-5 of
    their scale, far inside the 1e-3 the oracle comparison allows."""
    import torch
    data, w = _weight(fmt, n, k, 990 + int(fmt) + m)
    x = torch.from_numpy(_x(m, k, 12 + m)).cuda().half()
    outs = {}
    for ms in ("0", "2"):
        monkeypatch.setenv("COMBS_GEMVQ_MSUM", ms)
        y = torch.empty((m, n), device="cuda")
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        outs[ms] = y.cpu().numpy().astype(np.float64)
    scale = max(np.abs(outs["0"]).max(), 1.0)
    assert np.abs(outs["0"] - outs["2"]).max() <= 1e-5 * scale
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    O.assert_close(outs["2"], _x(m, k, 12 + m).astype(np.float64) @ wd.T.astype(np.float64), 1e-3, "sums")

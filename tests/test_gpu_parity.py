"""GPU parity of the gfx950 kernels against the CPU oracle, through the C ABI.

Mirrors the reference's own GPU tests (engine/core/combs-models/src/qmatmul.rs
:1727-2174): bit-exact dequant, fused matmul vs ref_matmul(dequant) within
|g - e| <= rel * max(|e|, 1) (rel 1e-4 for Q4_0, 1e-3 otherwise), at the
reference's shapes, x patterns and synthetic block streams, plus ragged and
multi-tile shapes, fp32/fp16 activations and outputs, and quantised N(0, 0.02)
weights with N(0, 1) activations."""
import os

import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat, QuantWeight, dequantize_gpu, quantize
from combsengine_amd import _lib as L

pytestmark = pytest.mark.gpu

FMTS = [QuantFormat.Q4_0, QuantFormat.Q5_0, QuantFormat.Q8_0, QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K,
        QuantFormat.Q4_1, QuantFormat.Q5_1]
LEGACY = {QuantFormat.Q4_0, QuantFormat.Q5_0, QuantFormat.Q8_0, QuantFormat.Q4_1, QuantFormat.Q5_1}


def rel_of(fmt):
    return 1e-4 if fmt == QuantFormat.Q4_0 else 1e-3


def synth(fmt, n, k):
    return O.SYNTH[int(fmt)](n * k // O.block_values(int(fmt)))


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact_synth(cuda, fmt):
    n_blocks = 33 if fmt in LEGACY else 9  # qmatmul.rs:1733, 1845: not a multiple of anything
    data = O.SYNTH[int(fmt)](n_blocks)
    n = n_blocks * O.block_values(int(fmt))
    print(f"dequant {fmt.name} blocks={n_blocks}", flush=True)
    got = dequantize_gpu(fmt, data)
    want = O.dequant(int(fmt), data, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact_quantized(cuda, fmt):
    x = np.random.default_rng(int(fmt)).normal(0, 0.02, (37, 1024)).astype(np.float32)
    data = quantize(fmt, x)
    got = dequantize_gpu(fmt, data)
    want = O.dequant(int(fmt), data, x.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_known_answers(cuda):
    import json
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))
    for name, case in gold.items():
        got = dequantize_gpu(case["format"], bytes.fromhex(case["hex"]))
        assert np.array_equal(got, np.array(case["expect"], np.float32)), name


def _run(w, x_np, x_dtype, y_dtype, path=L.CQ_PATH_AUTO):
    import torch
    x = torch.from_numpy(x_np).to("cuda").to(x_dtype)
    y = torch.empty((x.shape[0], w.n_out()), dtype=y_dtype, device="cuda")
    w.matmul_into(x, y, path=path)
    return y.float().cpu().numpy()


@pytest.mark.parametrize("fmt", FMTS)
def test_matmul_reference_shapes(cuda, fmt):
    """qmatmul.rs:1751-1781 / 1893-1971 / 2019-2048: (67,128) legacy,
    (35,512) K-quants, m in {1, 3}, x = ((i*7 % 13) - 6)/8."""
    import torch
    n, k = (67, 128) if fmt in LEGACY else (35, 512)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    assert w.vram_bytes() == len(data)
    for m in (1, 3):
        x = O.x_pattern(m, k).reshape(m, k)
        expect = O.ref_matmul(x, wd)
        for xt in (torch.float32, torch.float16):
            print(f"{fmt.name} n={n} k={k} m={m} x={xt}", flush=True)
            O.assert_close(_run(w, x, xt, torch.float32), expect, rel_of(fmt), f"{fmt.name} m={m} x={xt}")
        O.assert_close(w.matmul_host(x, m).reshape(m, n), expect, rel_of(fmt), "matmul_host")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 40])
def test_matmul_ragged_tiles(cuda, fmt, m):
    """Ragged row tiles (n % 16 != 0), several K units per wave, m across
    activation tiles; fp32 x (hi+lo split) and fp16 output."""
    import torch
    n, k = (300, 320) if fmt in LEGACY else (300, 1536)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 11, 29, 14.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    print(f"{fmt.name} n={n} k={k} m={m}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32), expect, 1e-3, "f16 x")
    O.assert_close(_run(w, x, torch.float32, torch.float16), expect, 1e-3, "f16 y")


@pytest.mark.parametrize("fmt", FMTS)
def test_matmul_quantized_gaussian(cuda, fmt):
    """N(0, 0.02) weights quantised with the GGUF quantiser, N(0, 1)
    activations, fp16 and fp32 (split) activations."""
    import torch
    rng = np.random.default_rng(100 + int(fmt))
    n, k, m = 200, 2048, 4
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x32 = rng.normal(0, 1, (m, k)).astype(np.float32)
    x16 = x32.astype(np.float16).astype(np.float32)
    print(f"gaussian {fmt.name}", flush=True)
    O.assert_close(_run(w, x16, torch.float16, torch.float32), O.ref_matmul(x16, wd), 1e-3, "x f16")
    O.assert_close(_run(w, x32, torch.float32, torch.float32), O.ref_matmul(x32, wd), 1e-3, "x f32")


@pytest.mark.parametrize("fmt", FMTS)
def test_matmul_deterministic(cuda, fmt):
    import torch
    n, k = (300, 320) if fmt in LEGACY else (300, 1536)
    w = QuantWeight.from_gguf_bytes(fmt, synth(fmt, n, k), n, k)
    x = O.x_pattern(3, k).reshape(3, k)
    a = _run(w, x, torch.float16, torch.float32)
    b = _run(w, x, torch.float16, torch.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_waves_override_consistent(cuda, monkeypatch):
    """Different K splits across waves only reorder fp32 sums."""
    import torch
    fmt, n, k = QuantFormat.Q4K, 64, 4096
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(1, k).reshape(1, k)
    expect = O.ref_matmul(x, wd)
    for nw in ("1", "3", "5", "8"):
        monkeypatch.setenv("COMBS_GEMV_WAVES", nw)
        O.assert_close(_run(w, x, torch.float16, torch.float32), expect, 1e-3, f"nw={nw}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n,k,m", [(4100, 512, 1), (70, 7168, 2), (8200, 2048, 3)])
def test_gemv_large_and_ragged(cuda, fmt, n, k, m):
    """Many row tiles, many K units per wave, ragged tiles."""
    import torch
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 13, 31, 15.0, 16.0).reshape(m, k)
    print(f"{fmt.name} n={n} k={k} m={m}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32), O.ref_matmul(x, wd), 1e-3, "gemv")


KQ = [QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n,k", [(300, 4096), (35, 512), (97, 3584), (50, 5120), (70, 14336), (130, 16384), (1, 256),
                                 (2053, 1024), (3000, 768), (9, 4352)])
@pytest.mark.parametrize("kernel", ["gemv2", "gemv1", "gemv1reg", "gemv1i8", "gemv1packed", "mfma", "gemvr"])
def test_gemv_single_row(cuda, monkeypatch, fmt, n, k, kernel):
    """m = 1 fp16 decode through each single-row kernel: the streaming
    quarter-superblock kernel (gemv2, K-quants: steps of 16 superblocks, R =
    16/units rows per step for units 1/2/4/8, several steps per row above 16,
    ragged row ranges per wave), the whole-superblock kernel (gemv1: wave
    tasks of 64/units rows, units from 1 to 64; by default small weights of
    Q4_0 / Q8_0 with more tasks than workgroups take its int8 path, gemv1reg
    forces the fp16-register path, gemv1i8 the int8 path for Q4_K / Q4_0 /
    Q8_0; small weights spread their tasks wave-major over the grid,
    gemv1packed packs them workgroup-major) and the 16-row MFMA kernel; fp32
    and fp16 outputs.  (COMBS_GEMV2=-1 keeps the small Q4_K weights, which
    take gemv2 by default, on the kernel named.)"""
    import torch
    if kernel == "gemv2" and fmt in LEGACY:
        pytest.skip("gemv2 serves the K-quants")
    if kernel == "gemvr" and fmt != QuantFormat.Q4K:
        pytest.skip("the row-split kernel serves Q4_K")
    monkeypatch.setenv("COMBS_GEMVR", "2" if kernel == "gemvr" else "0")
    monkeypatch.setenv("COMBS_GEMV1", "0" if kernel == "mfma" else "1")
    monkeypatch.setenv("COMBS_GEMV2", "2" if kernel == "gemv2" else "-1")
    monkeypatch.setenv("COMBS_GEMV1_I8", {"gemv1reg": "0", "gemv1i8": "2"}.get(kernel, "1"))
    monkeypatch.setenv("COMBS_GEMV1_SPREAD", "0" if kernel == "gemv1packed" else "1")
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(1, k, 13, 31, 15.0, 16.0).reshape(1, k)
    expect = O.ref_matmul(x, wd)
    print(f"{kernel} {fmt.name} n={n} k={k}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32), expect, rel_of(fmt), "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("m", [1, 17, 64, 100, 130, 300])
@pytest.mark.parametrize("kernel", ["1", "2:1:8", "2:2:8", "2:1:16", "2:2:16"])
def test_gemm_parity(cuda, monkeypatch, fmt, m, kernel):
    """Prefill dequant-GEMM (forced for small m too) vs the oracle, fp16/fp32
    activations, fp32/fp16 outputs, ragged m and n; every kernel and tile
    shape (kernel:NT:MT)."""
    import torch
    kern, nt, mt = (kernel.split(":") + ["0", "0"])[:3]
    monkeypatch.setenv("COMBS_GEMM_KERNEL", kern)
    monkeypatch.setenv("COMBS_GEMM2_NT", nt)
    monkeypatch.setenv("COMBS_GEMM2_MT", mt)
    n, k = 300, 1024
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 11, 29, 14.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    print(f"gemm kernel={kernel} {fmt.name} m={m}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32, path=L.CQ_PATH_GEMM), expect, 1e-3, "x16 y32")
    O.assert_close(_run(w, x, torch.float32, torch.float16, path=L.CQ_PATH_GEMM), expect, 1e-3, "x32 y16")


SCALE_OFF = {QuantFormat.Q4K: (0, 144), QuantFormat.Q5K: (0, 176), QuantFormat.Q6K: (208, 210)}


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("nt", ["1", "2"])
@pytest.mark.parametrize("mt", ["8", "16"])
@pytest.mark.parametrize("split", ["1", "3"])
def test_gemm_scale_edge_cases(cuda, monkeypatch, fmt, nt, mt, split):
    """Superblocks whose d is zero (min term only), subnormal, or 2^12 times
    larger than their neighbours: the large-tile kernel carries its
    accumulator in units of the running d and must still match the oracle."""
    import torch
    monkeypatch.setenv("COMBS_GEMM2_NT", nt)
    monkeypatch.setenv("COMBS_GEMM2_MT", mt)
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", split)
    off, bb = SCALE_OFF[fmt]
    n, k, m = 200, 2048, 150
    data = np.frombuffer(synth(fmt, n, k), dtype=np.uint8).copy()
    blocks = data.reshape(-1, bb)
    d = blocks[:, off:off + 2].copy().view(np.float16).reshape(-1)
    rng = np.random.default_rng(5)
    pick = rng.integers(0, 6, d.size)
    d[pick == 0] = 0.0
    d[pick == 1] = np.float16(3e-7)                      # subnormal
    d[pick == 2] = (d[pick == 2].astype(np.float32) * 4096).clip(-6e4, 6e4).astype(np.float16)
    blocks[:, off:off + 2] = d.view(np.uint8).reshape(-1, 2)
    data = data.tobytes()
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 7, 23, 12.0, 16.0).reshape(m, k)
    print(f"scale edges {fmt.name} nt={nt} mt={mt}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32, path=L.CQ_PATH_GEMM), O.ref_matmul(x, wd), 1e-3, "gemm")


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("split", ["2", "3", "4"])
@pytest.mark.parametrize("m", [17, 130])
def test_gemm_split_k(cuda, monkeypatch, fmt, split, m):
    """K split over workgroup slices (10 superblocks: 3 slices of 4, 4, 2)
    with fp32 partials and a reduction kernel, fp32 and fp16 outputs."""
    import torch
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", split)
    n, k = 200, 2560
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 11, 29, 14.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    print(f"split-K {fmt.name} split={split} m={m}", flush=True)
    O.assert_close(_run(w, x, torch.float16, torch.float32, path=L.CQ_PATH_GEMM), expect, 1e-3, "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16, path=L.CQ_PATH_GEMM), expect, 1e-3, "y16")


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("n,k,m", [(512, 7168, 64), (512, 3584, 512)])
def test_gemm_split_k_auto_down_projection(cuda, fmt, n, k, m):
    """Shapes with few weight rows take the automatic split (512 x 3584 at
    m = 512: four slices of 4, 4, 4, 2 superblocks); checked against float64
    torch on the GPU dequant."""
    import torch
    rng = np.random.default_rng(11 + int(fmt))
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd = torch.from_numpy(dequantize_gpu(fmt, data).reshape(n, k)).cuda().double()
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).cuda()
    y = w.matmul_device(x, out_dtype=torch.float32)
    O.assert_close(y.cpu().numpy(), (x.double() @ wd.t()).cpu().numpy(), 1e-3, "auto split")


@pytest.mark.parametrize("fmt", KQ)
def test_gemm_gaussian_prefill_shape(cuda, fmt):
    """Quantised N(0, 0.02) weights, N(0, 1) fp16 activations, prefill m=128,
    checked against a float64 torch matmul of the (bit-exact) GPU dequant."""
    import torch
    rng = np.random.default_rng(7 + int(fmt))
    n, k, m = 1024, 4096, 128
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd = torch.from_numpy(dequantize_gpu(fmt, data).reshape(n, k)).cuda().double()
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).cuda()
    y = w.matmul_device(x, out_dtype=torch.float32)
    ref = (x.double() @ wd.t()).cpu().numpy()
    O.assert_close(y.cpu().numpy(), ref, 1e-3, "gemm m=128")


def test_graph_capture_replays(cuda, monkeypatch):
    """cq_matmul launches captured into a HIP graph replay correctly, with
    eager work and synchronisations between replays (no memset nodes: the
    library records none).  The K split is pinned to one slice here (the
    captured split is test_graph_capture_prefill_split's).
    The graph holds single-row decode of a small weight (tasks spread over
    the grid), batched decode (m = 8), prefill (m = 64) and single-row
    decode of a 74-superblock Q6_K row (the row-half kernel)."""
    import torch
    monkeypatch.setenv("COMBS_GEMM2_SPLIT", "1")
    monkeypatch.setenv("COMBS_GEMVS", "0")  # batched decode (k = 4096) runs cq_gemvq_*, eager and captured
    fmt, n, k = QuantFormat.Q4K, 512, 4096
    rng = np.random.default_rng(3)
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    n2, k2 = 200, 18944
    w2 = QuantWeight.from_gguf_bytes(QuantFormat.Q6K, quantize(QuantFormat.Q6K, rng.normal(
        0, 0.02, (n2, k2)).astype(np.float32)), n2, k2)
    cases = []  # (weight, x, y)
    for wt, kk, nn, m, dt in ((w, k, n, 1, torch.float32), (w, k, n, 8, torch.float32), (w, k, n, 64, torch.float16),
                              (w2, k2, n2, 1, torch.float32)):
        cases.append((wt, torch.from_numpy(rng.normal(0, 1, (m, kk)).astype(np.float16)).cuda(),
                      torch.empty((m, nn), dtype=dt, device="cuda")))
    for wt, x, y in cases:
        wt.matmul_into(x, y)
    torch.cuda.synchronize()
    refs = [y.clone() for _, _, y in cases]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for wt, x, y in cases:
                wt.matmul_into(x, y)
    torch.cuda.current_stream().wait_stream(s)
    xp = cases[2][1]
    for rep in range(4):
        for _, _, y in cases:
            y.fill_(float("nan"))
        _ = (xp.float() @ xp.float().t()).sum()  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (_, _, y) in enumerate(cases):
            assert torch.equal(y, refs[i]), (rep, i)


@pytest.mark.parametrize("fmt,n,k,m", [(QuantFormat.Q6K, 512, 3584, 512), (QuantFormat.Q4K, 512, 3584, 130),
                                        (QuantFormat.Q5K, 300, 4096, 40), (QuantFormat.Q4K, 1024, 4096, 256),
                                        (QuantFormat.Q8_0, 1024, 4096, 100), (QuantFormat.Q5_1, 512, 3584, 40)])
def test_graph_capture_prefill_split(cuda, fmt, n, k, m):
    """Prefill captured into a HIP graph with the default K split (the
    K-quants' cq_gemm2_* and the 32-value formats' cq_gemml_*): the
    captured launch takes its activation sums and split partials from the
    device's fixed scratch buffer (no allocation in the graph) and must give
    the eager launch's bits (same kernels and slices, eager scratch allocated
    stream-ordered) on every replay, with eager prefill and a no-allocation
    call (which overwrites the fixed buffer) between the replays."""
    import torch
    rng = np.random.default_rng(40 + int(fmt) + m)
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).cuda()
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    kern = L.kernels(w, L.CQ_F16, m, L.CQ_F16)
    print(f"captured prefill {fmt.name} [{n}x{k}] m={m} kernels={kern}", flush=True)
    assert "splitk" in kern, "the shape is meant to take a K split"
    w.matmul_into(x, y)
    torch.cuda.synchronize()
    ref = y.clone()
    O.assert_close(ref.float().cpu().numpy(), x.double().cpu().numpy() @ wd.astype(np.float64).T, 1e-3, "eager")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            w.matmul_into(x, y)
    torch.cuda.current_stream().wait_stream(s)
    x2 = torch.from_numpy(rng.normal(0, 1, (m // 2 + 1, k)).astype(np.float16)).cuda()
    y2 = torch.empty((x2.shape[0], n), dtype=torch.float16, device="cuda")
    for rep in range(4):
        y.fill_(float("nan"))
        w.matmul_into(x2, y2)  # eager prefill between replays
        st = L.lib().cq_matmul_noalloc(w.handle, x2.data_ptr(), L.CQ_F16, x2.shape[0], y2.data_ptr(), L.CQ_F16,
                                       torch.cuda.current_stream().cuda_stream)
        assert st == L.CQ_OK, L.last_error()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), rep


@pytest.mark.parametrize("fmt,n,k,m", [(QuantFormat.Q4K, 4096, 14336, 16), (QuantFormat.Q6K, 300, 18944, 5),
                                        (QuantFormat.Q5K, 1000, 8192, 9), (QuantFormat.Q8_0, 700, 14336, 12),
                                        (QuantFormat.Q4_1, 300, 8192, 3)])
def test_graph_capture_batched_slices(cuda, fmt, n, k, m):
    """Batched decode of rows longer than 16 superblocks captured into a HIP
    graph: the captured column kernel takes its slice partials from the
    device's fixed scratch (no allocation in the graph) and must give the
    eager launch's bits (partials from the stream-ordered pool) on every
    replay, with eager batched decode and a no-allocation call (which
    overwrites the fixed buffer) between the replays."""
    import torch
    rng = np.random.default_rng(60 + int(fmt) + m)
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).cuda()
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    kern = L.kernels(w, L.CQ_F16, m, L.CQ_F32)
    print(f"captured batched {fmt.name} [{n}x{k}] m={m} kernels={kern}", flush=True)
    assert kern.startswith("cq_gemvq_") and "splitk" in kern
    w.matmul_into(x, y)
    torch.cuda.synchronize()
    ref = y.clone()
    O.assert_close(ref.cpu().numpy(), x.double().cpu().numpy() @ wd.astype(np.float64).T, 1e-3, "eager")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            w.matmul_into(x, y)
    torch.cuda.current_stream().wait_stream(s)
    x2 = torch.from_numpy(rng.normal(0, 1, (m - 1 if m > 2 else 2, k)).astype(np.float16)).cuda()
    y2 = torch.empty((x2.shape[0], n), dtype=torch.float32, device="cuda")
    for rep in range(4):
        y.fill_(float("nan"))
        w.matmul_into(x2, y2)  # eager batched decode between replays
        st = L.lib().cq_matmul_noalloc(w.handle, x2.data_ptr(), L.CQ_F16, x2.shape[0], y2.data_ptr(), L.CQ_F32,
                                       torch.cuda.current_stream().cuda_stream)
        assert st == L.CQ_OK, L.last_error()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), rep


def test_batched_slices_two_streams(cuda):
    """The batched decode's slice partials live in a per-device scratch kept
    across calls: calls alternating between two streams with no host
    synchronisation (each waits for the other stream's last use), growing
    the scratch midway (a wider weight, then m = 16), give every output the
    bits of the same call made alone."""
    import torch
    rng = np.random.default_rng(71)
    ws = []
    for n, k in ((500, 8192), (3000, 14336)):
        data = quantize(QuantFormat.Q4K, rng.normal(0, 0.02, (n, k)).astype(np.float32))
        ws.append(QuantWeight.from_gguf_bytes(QuantFormat.Q4K, data, n, k))
    calls = []  # (weight, x, y)
    for i in range(12):
        w = ws[0] if i < 6 else ws[1]
        m = 4 if i < 9 else 16
        calls.append((w, torch.from_numpy(rng.normal(0, 1, (m, w.k())).astype(np.float16)).cuda(),
                      torch.empty((m, w.n_out()), device="cuda")))
    assert "splitk" in L.kernels(ws[1], L.CQ_F16, 16, L.CQ_F32)
    refs = []
    for w, x, y in calls:
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        refs.append(y.clone())
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for _, _, y in calls:
        y.fill_(float("nan"))
    torch.cuda.synchronize()
    for i, (w, x, y) in enumerate(calls):
        with torch.cuda.stream(streams[i % 2]):
            w.matmul_into(x, y)
    torch.cuda.synchronize()
    for i, (_, _, y) in enumerate(calls):
        assert torch.equal(y, refs[i]), i


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("nt", ["1", "2", "4"])
@pytest.mark.parametrize("nw", ["1", "3", "8"])
@pytest.mark.parametrize("n,k,m", [(300, 4096, 2), (35, 512, 16), (97, 3584, 7), (70, 14336, 4), (33, 256, 16),
                                   (500, 1792, 9)])
def test_gemv_batched_direct(cuda, monkeypatch, fmt, nt, nw, n, k, m):
    """Batched decode (2 <= m <= 16, fp16 x) through the direct-activation
    kernel (cq_gemvd_*): NT row tiles per workgroup (ragged last tile), waves splitting
    the superblocks (more waves than superblocks, uneven shares, tails
    shorter than the load pipeline), m not a multiple of 4; checked against
    the oracle and bit-for-bit stable over repeated launches."""
    import torch
    monkeypatch.setenv("COMBS_GEMVQ", "0")  # cq_gemvd_*, not the column kernel
    monkeypatch.setenv("COMBS_GEMVS", "0")  # nor the LDS-shared one
    monkeypatch.setenv("COMBS_GVD_NT", nt)
    monkeypatch.setenv("COMBS_GVD_WAVES", nw)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 13, 31, 15.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    print(f"gemvd {fmt.name} nt={nt} nw={nw} n={n} k={k} m={m}", flush=True)
    a = _run(w, x, torch.float16, torch.float32)
    O.assert_close(a, expect, 1e-3, "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")
    assert np.array_equal(a.view(np.uint32), _run(w, x, torch.float16, torch.float32).view(np.uint32))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("groups", ["0", "1", "3", "7"])
@pytest.mark.parametrize("n,k,m", [(300, 4096, 2), (35, 512, 16), (97, 3584, 7), (33, 256, 16), (500, 1792, 9),
                                   (1000, 2048, 16), (129, 3840, 3), (4100, 4096, 13), (70, 1280, 15),
                                   (70, 14336, 4), (300, 18944, 9), (33, 4352, 16), (129, 8192, 3)])
def test_gemv_batched_columns(cuda, monkeypatch, fmt, groups, n, k, m):
    """Batched decode (2 <= m <= 16, fp16 x) through the column kernel
    (cq_gemvq_*), every format: one wave per column of 256 values (a
    superblock, or 8 blocks of a 32-value format; 1 to 16 columns), rows of
    more than 16 columns cut into slices (4 x 14, 5 x 15 with an idle wave in
    the last, 2 x 9 with one idle, 2 x 16) whose partials are summed in
    order, ragged last tile, tile ranges split over the default grid or 1, 3 or 7
    workgroups (runs of many tiles: the two-slot ring wraps, reduction
    chunks are full and partial), odd m, activation transits of one and of
    two phases (m > 12, or > 14 for Q4_K / Q5_K), Q6_K rows at every even
    byte offset of their 16-byte pieces (odd superblock counts); fp32 and
    fp16 y and the bias epilogue, against the oracle and bit-for-bit stable
    over repeated launches.  A weight whose size is not a multiple of 16
    bytes takes the next kernel (the DMA reads whole pieces): cq_gemvd_* for
    the K-quants, the 16-row MFMA GEMV for the others."""
    import torch
    monkeypatch.setenv("COMBS_GEMVQ_GROUPS", groups)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 13, 31, 15.0, 16.0).reshape(m, k)
    # above 4096 values the synthetic rows cancel far enough that the
    # oracle's sequential fp32 sum is itself ~1e-3 off: float64 of its
    # (bit-exact) dequant there (Q6_K [300 x 18944]: fp32 1.95363, float64
    # 1.95614 at [2, 212])
    expect = O.ref_matmul(x, wd) if k <= 4096 else x.astype(np.float64) @ wd.astype(np.float64).T
    xd = torch.from_numpy(x).cuda().half()
    kern = L.path_name(w, xd, torch.empty((m, n), device="cuda"))
    print(f"gemvq {fmt.name} groups={groups} n={n} k={k} m={m} kernels={kern}", flush=True)
    fallback = "cq_gemvd_" if fmt in KQ else "cq_gemv_"
    assert kern.startswith("cq_gemvq_" if len(data) % 16 == 0 else fallback)
    a = _run(w, x, torch.float16, torch.float32)
    O.assert_close(a, expect, rel_of(fmt) if k <= 4096 else 1e-3, "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")
    assert np.array_equal(a.view(np.uint32), _run(w, x, torch.float16, torch.float32).view(np.uint32))
    b = np.linspace(-1, 1, n).astype(np.float32)
    yb = torch.empty((m, n), device="cuda")
    w.matmul_bias_into(xd, torch.from_numpy(b).cuda(), yb)
    O.assert_close(yb.cpu().numpy(), expect.astype(np.float64) + b, 1e-3, "bias")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n,k", [(300, 4096), (97, 1536), (70, 14336)])
@pytest.mark.parametrize("m", [2, 4, 9, 16, 17, 40])
def test_f32_activations_split(cuda, monkeypatch, fmt, n, k, m):
    """fp32 activations at m >= 2 through the split path (x = hi + lo fp16
    rows, one pass of the fp16 kernels over 2m rows, the halves added by the
    split-K reduction; rows in blocks of 8 up to m = 16): against float64 of
    the oracle's dequant at the fp32-x bar, against the fp32-x kernels
    (COMBS_F32_SPLIT=0) and bit-for-bit stable over repeats; the dry run
    names the split kernels where the split is taken (K-quants from m = 4,
    the 32-value formats from m = 2)."""
    import torch
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    rng = np.random.default_rng(90 + m)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    expect = x.astype(np.float64) @ wd.astype(np.float64).T
    kern = L.kernels(w, L.CQ_F32, m, L.CQ_F32)
    print(f"f32 split {fmt.name} [{n}x{k}] m={m} kernels={kern}", flush=True)
    assert kern.startswith("cq_split_f32") == (m >= 4 or fmt not in KQ), kern
    a = _run(w, x, torch.float32, torch.float32)
    O.assert_close(a, expect, rel_of(fmt), "split")
    assert np.array_equal(a.view(np.uint32), _run(w, x, torch.float32, torch.float32).view(np.uint32))
    O.assert_close(_run(w, x, torch.float32, torch.float16), expect, 1e-3, "split y16")
    monkeypatch.setenv("COMBS_F32_SPLIT", "0")
    assert not L.kernels(w, L.CQ_F32, m, L.CQ_F32).startswith("cq_split_f32")
    O.assert_close(a, _run(w, x, torch.float32, torch.float32), 2 * rel_of(fmt), "vs the fp32-x kernels")


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("m", [4, 16])
def test_gemv_batched_gaussian_column_shape(cuda, fmt, m):
    """Llama-3-8B gate / up [14336 x 4096] at batch 4 / 16 through the column
    kernel: N(0, 0.02) quantised weights, N(0, 1) fp16 activations, against
    the oracle, a float64 torch matmul and the direct-activation kernel."""
    import torch
    rng = np.random.default_rng(310 + int(fmt) + m)
    n, k = 14336, 4096
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = rng.normal(0, 1, (m, k)).astype(np.float16).astype(np.float32)
    xd = torch.from_numpy(x).cuda().half()
    kern = L.path_name(w, xd, torch.empty((m, n), device="cuda"))
    print(f"gemvq gaussian {fmt.name} m={m} kernels={kern}", flush=True)
    assert kern.startswith("cq_gemvq_")
    got = _run(w, x, torch.float16, torch.float32)
    O.assert_close(got, O.ref_matmul(x, wd), 1e-3, "oracle")
    f64 = (torch.from_numpy(x).double() @ torch.from_numpy(wd).double().T).numpy()
    O.assert_close(got, f64, 1e-3, "f64")
    os.environ["COMBS_GEMVQ"] = "0"
    L.reload_options()
    try:
        O.assert_close(got, _run(w, x, torch.float16, torch.float32), 1e-3, "cq_gemvd")
    finally:
        os.environ.pop("COMBS_GEMVQ")
        L.reload_options()


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("m", [4, 16])
def test_gemv_batched_gaussian_llama_shape(cuda, fmt, m):
    """BASELINE config 3 shape [4096 x 14336] at batch 4 / 16: N(0, 0.02)
    quantised weights, N(0, 1) fp16 activations, against the oracle, a
    float64 torch matmul and, after the column kernel (four slices), the
    direct-activation kernel and the 16-row LDS-staged MFMA kernel."""
    import torch
    rng = np.random.default_rng(300 + int(fmt) + m)
    n, k = 4096, 14336
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = rng.normal(0, 1, (m, k)).astype(np.float16).astype(np.float32)
    print(f"gemvd gaussian {fmt.name} m={m}", flush=True)
    got = _run(w, x, torch.float16, torch.float32)
    O.assert_close(got, O.ref_matmul(x, wd), 1e-3, "oracle")
    f64 = (torch.from_numpy(x).double() @ torch.from_numpy(wd).double().T).numpy()
    O.assert_close(got, f64, 1e-3, "f64")
    assert L.kernels(w, L.CQ_F16, m, L.CQ_F32).startswith("cq_gemvq_")
    knobs = ("COMBS_GEMVQ", "COMBS_GEMVS", "COMBS_GEMVD")  # then direct-activation, then the 16-row MFMA GEMV
    try:
        for knob in knobs:
            os.environ[knob] = "0"
            L.reload_options()
            old = _run(w, x, torch.float16, torch.float32)
            O.assert_close(got, old, 1e-3, f"with {knob}=0")
    finally:
        for knob in knobs:
            os.environ.pop(knob, None)
        L.reload_options()


@pytest.mark.parametrize("fmt", [QuantFormat.Q4K, QuantFormat.Q5K, QuantFormat.Q6K, QuantFormat.Q4_0, QuantFormat.Q8_0])
@pytest.mark.parametrize("n,k", [(300, 18944), (67, 16640), (40, 33024), (3, 18944), (37, 27136), (513, 32768),
                                 (1029, 17152)])
@pytest.mark.parametrize("kernel", ["gemv1k", "mfma", "gemvr"])
def test_gemv_single_row_long_k(cuda, monkeypatch, fmt, n, k, kernel):
    """m = 1 with K above the single-row kernels' 16384 (a Qwen2.5-7B down
    projection is 18944 wide): rows of 65 to 128 units (106 for Q6_K) on the
    half-row wave-pair kernel (Q4_K / Q5_K / Q6_K / Q4_0: odd unit counts,
    Q6_K half rows at every even byte offset, row counts that leave a pair
    idle), the rest and COMBS_GEMV1K=0 on the 16-row MFMA GEMV; fp32 and
    fp16 y, checked against the oracle and for bit-identical repeats."""
    import torch
    if kernel == "gemvr" and (fmt != QuantFormat.Q4K or k > 32768):
        pytest.skip("the row-split kernel serves Q4_K up to K = 32768")
    monkeypatch.setenv("COMBS_GEMV1K", "1" if kernel == "gemv1k" else "0")
    monkeypatch.setenv("COMBS_GEMVR", "2" if kernel == "gemvr" else "0")
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(1, k, 13, 31, 15.0, 16.0).reshape(1, k)
    print(f"long-k {fmt.name} n={n} k={k}", flush=True)
    # float64 of the oracle's (bit-exact) dequant: at K = 32768 the synthetic
    # rows cancel to ~1e-5 of their absolute sum, where a sequential fp32 sum
    # is itself ~1e-3 off
    expect = x.astype(np.float64) @ wd.astype(np.float64).T
    a = _run(w, x, torch.float16, torch.float32)
    O.assert_close(a, expect, rel_of(fmt), "y32")
    assert np.array_equal(a.view(np.uint32), _run(w, x, torch.float16, torch.float32).view(np.uint32))
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("split", ["0", "1", "3"])
@pytest.mark.parametrize("n,k,m", [(300, 4096, 2), (35, 512, 16), (97, 3584, 7), (70, 14336, 4), (33, 256, 16),
                                   (500, 1792, 9), (1000, 2048, 16), (129, 4608, 3)])
def test_gemv_batched_shared(cuda, monkeypatch, fmt, split, n, k, m):
    """Batched decode (2 <= m <= 16, fp16 x) through the LDS-shared kernel
    (cq_gemvs_*): 128-row workgroups (ragged last group and tile), slices of
    the superblocks over the grid (automatic, one, three: ragged last slice,
    slices shorter than the 4-slot ring), fp32 and fp16 y, the bias epilogue
    on both the direct and the split path; against the oracle and bit-for-bit
    stable over repeated launches."""
    import torch
    monkeypatch.setenv("COMBS_GEMVQ", "0")  # not the column kernel, which comes first
    monkeypatch.setenv("COMBS_GEMVS", "2")
    monkeypatch.setenv("COMBS_GEMVS_SPLIT", split)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 13, 31, 15.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    xd = torch.from_numpy(x).cuda().half()
    kern = L.path_name(w, xd, torch.empty((m, n), device="cuda"))
    print(f"gemvs {fmt.name} split={split} n={n} k={k} m={m} kernels={kern}", flush=True)
    # (the LDS DMA reads whole 16-byte pieces: a weight whose size is not a
    # multiple of 16 bytes takes cq_gemvd_*)
    assert kern.startswith("cq_gemvs_" if len(data) % 16 == 0 else "cq_gemvd_")
    a = _run(w, x, torch.float16, torch.float32)
    O.assert_close(a, expect, 1e-3, "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")
    assert np.array_equal(a.view(np.uint32), _run(w, x, torch.float16, torch.float32).view(np.uint32))
    b = np.linspace(-1, 1, n).astype(np.float32)
    yb = torch.empty((m, n), device="cuda")
    w.matmul_bias_into(xd, torch.from_numpy(b).cuda(), yb)
    O.assert_close(yb.cpu().numpy(), expect.astype(np.float64) + b, 1e-3, "bias")


@pytest.mark.parametrize("fmt", sorted(LEGACY))
@pytest.mark.parametrize("mt,nt", [("8", "1"), ("8", "2"), ("4", "1")])
@pytest.mark.parametrize("split", ["0", "1", "3"])
@pytest.mark.parametrize("n,k,m", [(300, 320, 17), (130, 4096, 64), (1000, 1056, 130), (70, 2048, 300)])
def test_gemm_legacy_formats(cuda, monkeypatch, fmt, mt, nt, split, n, k, m):
    """Prefill GEMM for the 32-value formats (cq_gemml_*): 128- or 64-row
    activation tiles (ragged m), 16-row weight tiles (ragged n), steps of four blocks
    with a partial last step (k = 320, 1056), one or two weight tiles per
    wave, the steps split over the grid (automatic, one, three slices: the
    last shorter, or holding only the partial step) with the slices'
    partials summed by cq_splitk_reduce_*; fp32 and fp16 y and the bias
    epilogue, against the oracle."""
    import torch
    monkeypatch.setenv("COMBS_GEMML_MT", mt)
    monkeypatch.setenv("COMBS_GEMML_NT", nt)
    monkeypatch.setenv("COMBS_GEMML_SPLIT", split)
    data = synth(fmt, n, k)
    wd = O.dequant(int(fmt), data, n * k).reshape(n, k)
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    x = O.x_pattern(m, k, 11, 29, 14.0, 16.0).reshape(m, k)
    expect = O.ref_matmul(x, wd)
    xd = torch.from_numpy(x).cuda().half()
    kern = L.path_name(w, xd, torch.empty((m, n), device="cuda"))
    print(f"gemml {fmt.name} mt={mt} nt={nt} n={n} k={k} m={m} kernels={kern}", flush=True)
    assert kern.startswith(f"cq_gemml_{fmt.name.lower()}_n{nt}" + ("_m4" if mt == "4" else "_y"))
    O.assert_close(_run(w, x, torch.float16, torch.float32), expect, 1e-3, "y32")
    O.assert_close(_run(w, x, torch.float16, torch.float16), expect, 1e-3, "y16")
    b = np.linspace(-2, 2, n).astype(np.float32)
    yb = torch.empty((m, n), device="cuda")
    w.matmul_bias_into(xd, torch.from_numpy(b).cuda(), yb)
    O.assert_close(yb.cpu().numpy(), expect.astype(np.float64) + b, 1e-3, "bias")

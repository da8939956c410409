"""GPU parity at every BASELINE configuration's full workload.

Each case quantises N(0, 0.02) weights of the configuration's exact shape
(seeded torch generator on the GPU, then the GGUF quantiser on the host), runs
the library's default dispatch (cq_matmul, no tuning overrides) on N(0, 1)
fp16 activations, and checks:

  * the GPU dequant of the whole weight is bit-identical to the oracle's
    (gguf.rs:755-999 restated in oracle/gguf_oracle.c);
  * every output element against a float64 matmul of the oracle's dequant
    (BASELINE measurement rule: |y - y_ref| <= 1e-3 * max(|y_ref|, 1));
  * a seeded subset of weight rows (first and last 16-row tile included)
    against the oracle's ref_matmul, the reference test oracle
    (qmatmul.rs:1713-1725), on up to four activation rows.

This mirrors the reference's GPU-vs-ref_matmul tests (qmatmul.rs:1893-1971)
at the shapes the benchmark times, so every number bench.py reports has
correctness evidence at its own launch geometry.
"""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat as F
from combsengine_amd import QuantWeight, dequantize_gpu, quantize
from combsengine_amd import _lib as L

pytestmark = pytest.mark.gpu

TOL = 1e-3

# (case id, format, n, k, activation rows, y dtype name)
CASES = []
for _f in (F.Q4_0, F.Q8_0):  # config 2: Llama-3-8B attention / MLP shapes, batch 1
    for _n, _k in ((4096, 4096), (14336, 4096), (4096, 14336)):
        CASES.append((f"c2-{_f.name}-{_n}x{_k}", _f, _n, _k, (1,), "f32"))
for _f in (F.Q4K, F.Q5K):  # config 3: K-quant projections at batch 1 / 4 / 16
    for _n, _k in ((14336, 4096), (4096, 14336)):
        CASES.append((f"c3-{_f.name}-{_n}x{_k}", _f, _n, _k, (1, 4, 16), "f32"))
CASES.append(("c3-Q6K-lm_head-128256x4096", F.Q6K, 128256, 4096, (1, 4, 16), "f32"))
# config 4: chunked prefill, fp16 out
CASES.append(("c4-Q4K-14336x4096", F.Q4K, 14336, 4096, (128, 512, 2048), "f16"))
CASES.append(("c4-Q6K-4096x14336", F.Q6K, 4096, 14336, (128, 512, 2048), "f16"))
# prefill of the legacy formats at the config-2 MLP shape (the reference's
# tiled Q8_0 kernel, qmatmul.rs:481-527), fp16 out
for _f in (F.Q8_0, F.Q4_0):
    CASES.append((f"c2p-{_f.name}-14336x4096", _f, 14336, 4096, (128, 512), "f16"))
# config 5: one Qwen2.5-7B decoder layer (V and down in Q6_K)
for _name, _f, _n, _k in (("q", F.Q4K, 3584, 3584), ("k", F.Q4K, 512, 3584), ("v", F.Q6K, 512, 3584),
                          ("o", F.Q4K, 3584, 3584), ("gate", F.Q4K, 18944, 3584), ("up", F.Q4K, 18944, 3584),
                          ("down", F.Q6K, 3584, 18944)):
    CASES.append((f"c5-{_name}-{_f.name}-{_n}x{_k}", _f, _n, _k, (1, 8, 16, 512), "f32|f16"))


def _seed(case_id: str) -> int:
    return sum((i + 1) * ord(c) for i, c in enumerate(case_id)) % 100003


def _weights(fmt, n, k, seed):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02).cpu().numpy()
    return quantize(fmt, w)


def _oracle_dequant(fmt, data, n, k):
    return O.dequant(int(fmt), data, n * k, threads=16).reshape(n, k)


def _rows_subset(n, seed, count=32):
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(n, size=min(count, n), replace=False).tolist())
    pick |= set(range(min(16, n))) | set(range(max(0, n - 16), n))
    return np.array(sorted(pick))


def _check_case(cid, fmt, n, k, ms, ydt):
    import torch
    seed = _seed(cid)
    print(f"[{cid}] seed={seed} quantise {fmt.name} [{n}x{k}]", flush=True)
    data = _weights(fmt, n, k, seed)
    wd = _oracle_dequant(fmt, data, n, k)
    got = dequantize_gpu(fmt, data).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), wd.view(np.uint32)), f"{cid}: dequant not bit-exact"
    del got
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd_dev = torch.from_numpy(wd).cuda().double()
    rows = _rows_subset(n, seed)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    for m in ms:
        yt = torch.float16 if (ydt == "f16" or (ydt == "f32|f16" and m > 16)) else torch.float32
        x = torch.randn((m, k), generator=g, device="cuda", dtype=torch.float32).half()
        y = torch.empty((m, n), dtype=yt, device="cuda")
        print(f"[{cid}] m={m} y={yt} path={L.path_name(w, x, y)}", flush=True)
        w.matmul_into(x, y)
        torch.cuda.synchronize()
        ref = (x.double() @ wd_dev.t()).cpu().numpy()
        yh = y.float().cpu().numpy()
        O.assert_close(yh, ref, TOL, f"{cid} m={m} vs float64")
        xr = x[: min(m, 4)].float().cpu().numpy()
        O.assert_close(yh[: xr.shape[0]][:, rows], O.ref_matmul(xr, wd[rows]), TOL, f"{cid} m={m} vs ref_matmul")
    del w, wd_dev


@pytest.mark.parametrize("cid,fmt,n,k,ms,ydt", CASES, ids=[c[0] for c in CASES])
def test_config_workload(cuda, cid, fmt, n, k, ms, ydt):
    _check_case(cid, fmt, n, k, ms, ydt)


@pytest.mark.parametrize("n,k", [(14336, 4096), (18944, 3584)])
@pytest.mark.parametrize("ydt", ["f32", "f16"])
def test_config_gated_gate_up(cuda, n, k, ydt):
    """The one-launch gated gate/up at the Llama-3-8B and Qwen2.5-7B MLP
    shapes (batch 1, fp16 x): silu(x.Wg^T) * (x.Wu^T) against float64 over
    the oracle dequant (llama.rs:301-303)."""
    import torch
    seed = 7 * n + k
    print(f"gated gate/up [{n}x{k}] y={ydt} seed={seed}", flush=True)
    dg, du = _weights(F.Q4K, n, k, seed), _weights(F.Q4K, n, k, seed + 1)
    wg, wu = QuantWeight.from_gguf_bytes(F.Q4K, dg, n, k), QuantWeight.from_gguf_bytes(F.Q4K, du, n, k)
    g = torch.Generator(device="cuda").manual_seed(seed + 2)
    x = torch.randn((1, k), generator=g, device="cuda").half()
    yt = torch.float16 if ydt == "f16" else torch.float32
    y = torch.empty((1, n), dtype=yt, device="cuda")
    st = L.lib().cq_matmul_gate_up(wg.handle, wu.handle, x.data_ptr(), L.CQ_F16, 1, L.CQ_ACT_SILU, y.data_ptr(),
                                   L.CQ_F16 if ydt == "f16" else L.CQ_F32, torch.cuda.current_stream().cuda_stream)
    assert st == L.CQ_OK, L.last_error()
    xd = x.double().cpu().numpy()
    gd = xd @ _oracle_dequant(F.Q4K, dg, n, k).astype(np.float64).T
    ud = xd @ _oracle_dequant(F.Q4K, du, n, k).astype(np.float64).T
    if ydt == "f16":  # the reference's f16 model rounds each projection's output (qlinear.rs:126-143)
        gd, ud = gd.astype(np.float16).astype(np.float64), ud.astype(np.float16).astype(np.float64)
    O.assert_close(y.float().cpu().numpy(), O.activation(O.ACT_SILU, gd) * ud, 2e-3 if ydt == "f16" else TOL,
                   "gated")

"""cq_matmul_noalloc (the entry point that allocates nothing) against
cq_matmul, through the C ABI, on prefill shapes whose kernels use scratch:
the Q4_K / Q5_K activation sub-block sums and split-K partials (a
down-projection shape with few rows and long K), then Q6_K (partials only).
Two calls in a row on each weight, the second with fewer activation rows, so
the second reuses the scratch the first left behind.  Checked bit for bit
against cq_matmul (same kernels and K split) and against float64 over the
oracle's dequant (|y - y_ref| <= 1e-3 * max(|y_ref|, 1)); the decode path
(no scratch at m = 1 and for rows of at most 16 superblocks; for longer
rows the batched decode's slice partials, m = 16 then 5, 9 then 3) is
checked too, and a prefill whose activation sums exceed the scratch is
rejected with CQ_ERR_BAD_SHAPE."""
import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat as F
from combsengine_amd import QuantWeight, quantize
from combsengine_amd import _lib as L

pytestmark = pytest.mark.gpu


def _call(fn, w, x, y):
    import torch
    st = fn(w.handle, x.data_ptr(), L.CQ_F16, x.shape[0], y.data_ptr(), L.CQ_F16 if y.dtype == torch.float16
            else L.CQ_F32, torch.cuda.current_stream().cuda_stream)
    assert st == L.CQ_OK, L.last_error()


@pytest.mark.parametrize("fmt,n,k,ms", [(F.Q4K, 512, 3584, (512, 130)), (F.Q5K, 1000, 2048, (300, 40)),
                                        (F.Q6K, 512, 3584, (512, 64)), (F.Q4K, 300, 4096, (1, 9)),
                                        (F.Q6K, 700, 14336, (16, 5)), (F.Q4K, 300, 18944, (9, 3))])
def test_noalloc_matches_matmul(cuda, fmt, n, k, ms):
    import torch
    assert L.lib().cq_device_init() == L.CQ_OK, L.last_error()
    rng = np.random.default_rng(21 + int(fmt))
    data = quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    w = QuantWeight.from_gguf_bytes(fmt, data, n, k)
    wd = torch.from_numpy(O.dequant(int(fmt), data, n * k).reshape(n, k)).cuda().double()
    for m in ms:  # second call smaller: the scratch keeps the first call's contents
        x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).cuda()
        print(f"noalloc {fmt.name} [{n}x{k}] m={m} kernels={L.kernels(w, L.CQ_F16, m, L.CQ_F32)}", flush=True)
        y0 = torch.empty((m, n), device="cuda")
        y1 = torch.full((m, n), float("nan"), device="cuda")
        _call(L.lib().cq_matmul, w, x, y0)
        _call(L.lib().cq_matmul_noalloc, w, x, y1)
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), f"m={m}: noalloc differs from cq_matmul"
        O.assert_close(y1.cpu().numpy(), (x.double() @ wd.t()).cpu().numpy(), 1e-3, f"m={m} vs float64")


def test_noalloc_rejects_oversized_sums(cuda):
    import torch
    n, k, m = 16, 65536, 4200  # Q4_K sums: 4200 * 256 * 32 bytes > 32 MiB
    data = quantize(F.Q4K, np.zeros((n, k), np.float32))
    w = QuantWeight.from_gguf_bytes(F.Q4K, data, n, k)
    x = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    y = torch.empty((m, n), device="cuda")
    st = L.lib().cq_matmul_noalloc(w.handle, x.data_ptr(), L.CQ_F16, m, y.data_ptr(), L.CQ_F32,
                                   torch.cuda.current_stream().cuda_stream)
    assert st == L.CQ_ERR_BAD_SHAPE and "scratch" in L.last_error()

"""Benchmark of the fused GGUF dequant-matmul on one MI355X.

Headline (BASELINE.json metric "Q4_K decode GEMV HBM GB/s (% of peak)"):
one step = one decode token's Q4_K projections at Llama-3-8B shapes, batch 1:
a [14336 x 4096] (gate/up) and a [4096 x 14336] (down) GEMV, the two K-quant
projection shapes of BASELINE config 3; x fp16 N(0, 1), y fp32.  Weights are
N(0, 0.02) quantised to Q4_K from a seed and replicated into a pool of
>= 1.25 GiB of distinct device buffers that the steps rotate through, so each
launch streams its weight from HBM rather than the 256 MB Infinity Cache.

The K timed steps are captured once into a HIP graph (torch.cuda.CUDAGraph
over the library's hipModuleLaunchKernel calls) and replayed, so the number
measures the kernels back to back rather than Python's launch overhead.

value = algorithmic bytes (GGUF-native weight bytes + x + y) of K steps
        / device time of the K steps (HIP events around the graph replay).

Also reported: the roofline of the dominant kernel (cq_gemv1_q4_k_yf32, the
single-row decode GEMV)
from graphs of single-shape launches, prefill dequant-GEMM TFLOP/s (config 4,
the faster of eager launches, which may split K, and a captured graph),
lm_head Q6_K and batch 4/16, and the reference CPU path (dequantise once,
dense f32 GEMV per call) timed on this host as cpu_baseline.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
HEADLINE_KERNEL = "cq_gemv1_q4_k_yf32"  # what cq_matmul launches for m = 1, fp16 x, Q4_K
FP16_PEAK_TFLOPS = 2500.0


def algo_bytes(wbytes, m, k, n, xbytes=2, ybytes=4):
    return wbytes + m * k * xbytes + m * n * ybytes


def make_pool(fmt, n, k, pool_bytes, seed, count=None):
    """One seeded quantised weight, replicated into distinct device buffers
    (`count` of them, or as many as fit in `pool_bytes`)."""
    import numpy as np
    import torch
    from combsengine_amd import QuantWeight, quantize
    rng = np.random.default_rng(seed)
    data = np.frombuffer(quantize(fmt, rng.normal(0, 0.02, (n, k)).astype(np.float32)), np.uint8)
    base = torch.from_numpy(data.copy()).cuda()
    count = count or max(1, int(pool_bytes // data.size))
    pool = [QuantWeight.from_device(fmt, base if i == 0 else base.clone(), n, k) for i in range(count)]
    return pool, data


def graph_time_us(launch, count, reps=3):
    """Capture `count` launches (launch(i)) in one HIP graph; return the
    device time per launch (us), best of `reps` replays."""
    import torch
    launch(0)  # make sure the library and modules are loaded outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(count):
                launch(i)
    torch.cuda.current_stream().wait_stream(s)
    g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        t = a.elapsed_time(b) * 1e3 / count
        best = t if best is None else min(best, t)
    return best, g


def eager_time_us(launch, count, reps=3):
    """Device time per launch (us) of `count` eager launches on the current
    stream (HIP events around them), best of `reps`.  Used for the prefill
    GEMMs: each launch runs 30-600 us, so host launch overhead is hidden,
    and the eager path may split K (captured launches do not)."""
    import torch
    launch(0)
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(count):
            launch(i)
        b.record()
        torch.cuda.synchronize()
        t = a.elapsed_time(b) * 1e3 / count
        best = t if best is None else min(best, t)
    return best


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return {}


def cpu_baseline(seconds=6.0):
    """Reference CPU path (dequantise at load, dense f32 GEMV per call) on the
    headline gate shape, 1 thread (matrixmultiply without threading) and all
    cores; reported in the same GB/s metric as the GPU."""
    import numpy as np
    import oracle as O
    from combsengine_amd import QuantFormat, quantize
    n, k = 14336, 4096
    rng = np.random.default_rng(7)
    data = np.frombuffer(quantize(QuantFormat.Q4K, rng.normal(0, 0.02, (n, k)).astype(np.float32)), np.uint8)
    t0 = time.perf_counter()
    w = O.dequant(O.Q4_K, data, n * k, threads=1).reshape(n, k)
    t_deq = time.perf_counter() - t0
    x = rng.normal(0, 1, (1, k)).astype(np.float16).astype(np.float32)
    res = {}
    for threads in (1, os.cpu_count() or 1):
        calls, t0 = 0, time.perf_counter()
        while True:
            O.dense_gemm(x, w, threads)
            calls += 1
            el = time.perf_counter() - t0
            if el > seconds / 2:
                break
        res[threads] = (calls, el)
    per = algo_bytes(data.size, 1, k, n)
    c1, e1 = res[1]
    call_max = max(res)
    cm, em = res[call_max]
    return {
        "value": round(per * c1 / e1 / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"Q4_K [{n}x{k}] m=1: dequantise once ({t_deq:.2f} s, 1 thread), then {c1} dense f32 GEMV "
                  f"calls in {e1:.1f} s on 1 thread (oracle restatement of llama.rs:81-97 -> sgemm)",
        "all_cores": {"value": round(per * cm / em / 1e9, 3), "cores": call_max, "calls": cm},
        "dequant_s": round(t_deq, 3), "ms_per_call_1t": round(e1 / c1 * 1e3, 3),
    }


def secondary(dev):
    """Prefill dequant-GEMM (config 4: the faster of eager launches through
    fast_launcher, which may split K, and a captured graph, which does not), lm_head Q6_K and batch
    4/16 GEMV (captured graphs)."""
    import numpy as np
    import torch
    from combsengine_amd import QuantFormat
    out = {}
    rng = np.random.default_rng(9)
    # prefill: M in {128, 512, 2048} x Q4_K [14336 x 4096] and Q6_K [4096 x 14336], fp16 out
    for fmt, n, k in ((QuantFormat.Q4K, 14336, 4096), (QuantFormat.Q6K, 4096, 14336)):
        pool, data = make_pool(fmt, n, k, 0.3 * (1 << 30), seed=300 + int(fmt))
        for m in (128, 512, 2048):
            x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16)).to(dev)
            y = torch.empty((m, n), dtype=torch.float16, device=dev)
            launch = lambda i: pool[i % len(pool)].matmul_into(x, y)  # noqa: E731
            cnt = 40 if m < 2048 else 16
            # eager: the library call with its arguments resolved once (no
            # Python-side checks per launch), as in the config 2/3/5 bursts
            us_e = eager_time_us(fast_launcher(pool, x, y), cnt)
            us_g, _ = graph_time_us(launch, cnt)
            us = min(us_e, us_g)
            fl = 2.0 * m * n * k
            out[f"prefill_{fmt.name}_{n}x{k}_m{m}"] = {"us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                                                      "frac_fp16_peak": round(fl / us / 1e6 / FP16_PEAK_TFLOPS, 4),
                                                      "us_eager": round(us_e, 2), "us_graph": round(us_g, 2)}
        del pool
    # lm_head Q6_K [128256 x 4096] (431 MB: larger than the Infinity Cache)
    pool, data = make_pool(QuantFormat.Q6K, 128256, 4096, 2 * 431e6, seed=77)
    x = torch.from_numpy(rng.normal(0, 1, (1, 4096)).astype(np.float16)).to(dev)
    y = torch.empty((1, 128256), dtype=torch.float32, device=dev)
    us, _ = graph_time_us(lambda i: pool[i % len(pool)].matmul_into(x, y), 8)
    b = algo_bytes(data.size, 1, 4096, 128256)
    out["lm_head_q6_k_m1"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1)}
    del pool
    # gated MLP input at batch 1 (llama.rs:301-303): silu(x.Wg^T) * (x.Wu^T),
    # one launch over both weights, and the two-launch path for comparison
    from combsengine_amd import _lib as L
    gpool, gdata = make_pool(QuantFormat.Q4K, 14336, 4096, 0.6 * (1 << 30), seed=1100)
    upool, _ = make_pool(QuantFormat.Q4K, 14336, 4096, 0.6 * (1 << 30), seed=1101)
    x = torch.from_numpy(rng.normal(0, 1, (1, 4096)).astype(np.float16)).to(dev)
    y = torch.empty((1, 14336), dtype=torch.float16, device=dev)

    def gate_up(i):
        j = i % len(gpool)
        st = L.lib().cq_matmul_gate_up(gpool[j].handle, upool[j].handle, x.data_ptr(), L.CQ_F16, 1, L.CQ_ACT_SILU,
                                       y.data_ptr(), L.CQ_F16, torch.cuda.current_stream().cuda_stream)
        assert st == L.CQ_OK, L.last_error()

    b = 2 * gdata.size + 4096 * 2 + 14336 * 2
    res = {}
    for mode in ("1", "0"):
        os.environ["COMBS_GATEUP_FUSED"] = mode
        L.reload_options()
        us, _ = graph_time_us(gate_up, 2 * len(gpool))
        res["one_launch" if mode == "1" else "two_launches"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1)}
    os.environ.pop("COMBS_GATEUP_FUSED")
    L.reload_options()
    out["gate_up_silu_q4_k_14336x4096_m1"] = res
    del gpool, upool
    # decode batch 4 / 16 on the gate shape
    pool, data = make_pool(QuantFormat.Q4K, 14336, 4096, 0.6 * (1 << 30), seed=1000)
    for m in (4, 16):
        x = torch.from_numpy(rng.normal(0, 1, (m, 4096)).astype(np.float16)).to(dev)
        y = torch.empty((m, 14336), dtype=torch.float32, device=dev)
        us, _ = graph_time_us(lambda i: pool[i % len(pool)].matmul_into(x, y), 2 * len(pool))
        b = algo_bytes(data.size, m, 4096, 14336)
        out[f"q4_k_14336x4096_m{m}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1)}
    return out


def fast_launcher(pool, x, y):
    """launch(i): cq_matmul on pool[i % len(pool)] with the arguments resolved
    once (a ctypes call per launch, no Python-side checks), so that eager
    bursts stay device-bound."""
    import torch
    from combsengine_amd import _lib as L
    fn = L.lib().cq_matmul_path
    xt = L.CQ_F16 if x.dtype == torch.float16 else L.CQ_F32
    yt = L.CQ_F16 if y.dtype == torch.float16 else L.CQ_F32
    hs = [w.handle for w in pool]
    xp, yp, m = x.data_ptr(), y.data_ptr(), x.shape[0]
    s = torch.cuda.current_stream().cuda_stream
    P = len(hs)

    def launch(i):
        st = fn(hs[i % P], xp, xt, m, yp, yt, L.CQ_PATH_AUTO, s)
        if st != L.CQ_OK:
            raise RuntimeError(L.last_error())
    return launch


def configs_2_3_5(dev):
    """BASELINE configs 2, 3 and 5 as eager bursts of launches (HIP events
    around 2 x pool-size launches on the current stream, best of 3), each
    launch streaming a distinct weight buffer from a pool larger than the
    Infinity Cache.  Reported per shape: device us per launch and
    algorithmic GB/s (weight + x + y bytes)."""
    import numpy as np
    import torch
    from combsengine_amd import QuantFormat
    rng = np.random.default_rng(11)
    out = {}

    def one(fmt, n, k, m, pool_gib, seed, key, ydt=torch.float32):
        pool, data = make_pool(fmt, n, k, pool_gib * (1 << 30), seed=seed)
        res = {}
        for mm in m:
            x = torch.from_numpy(rng.normal(0, 1, (mm, k)).astype(np.float16)).to(dev)
            y = torch.empty((mm, n), dtype=ydt, device=dev)
            us = eager_time_us(fast_launcher(pool, x, y), max(2 * len(pool), 40))
            b = algo_bytes(data.size, mm, k, n, ybytes=2 if ydt == torch.float16 else 4)
            res[f"m{mm}"] = {"us": round(us, 2), "GBps": round(b / us / 1e3, 1)}
        out[key] = res
        del pool
        return res

    # config 2: Q4_0 / Q8_0 at the Llama-3-8B attention and MLP shapes, batch 1
    for fmt in (QuantFormat.Q4_0, QuantFormat.Q8_0):
        for n, k in ((4096, 4096), (14336, 4096), (4096, 14336)):
            one(fmt, n, k, (1,), 0.6, 2000 + n + k, f"config2_{fmt.name}_{n}x{k}")
    # config 3: Q4_K / Q5_K projections at batch 1, 4, 16; Q6_K lm_head
    for fmt in (QuantFormat.Q4K, QuantFormat.Q5K):
        for n, k in ((14336, 4096), (4096, 14336)):
            one(fmt, n, k, (1, 4, 16), 0.6, 3000 + n + k, f"config3_{fmt.name}_{n}x{k}")
    one(QuantFormat.Q6K, 128256, 4096, (1, 4, 16), 0.85, 3100, "config3_Q6K_lm_head_128256x4096")
    # config 5: one Qwen2.5-7B layer's seven projections (hidden 3584,
    # intermediate 18944, 4 KV heads x 128); V and down in Q6_K
    layer = [("q", QuantFormat.Q4K, 3584, 3584), ("k", QuantFormat.Q4K, 512, 3584), ("v", QuantFormat.Q6K, 512, 3584),
             ("o", QuantFormat.Q4K, 3584, 3584), ("gate", QuantFormat.Q4K, 18944, 3584),
             ("up", QuantFormat.Q4K, 18944, 3584), ("down", QuantFormat.Q6K, 3584, 18944)]
    sweep = {}
    wbytes = 0
    tot = {1: 0.0, 8: 0.0, 16: 0.0, 512: 0.0}
    for name, fmt, n, k in layer:
        pool, data = make_pool(fmt, n, k, 0.4 * (1 << 30), seed=5000 + n + k)
        wbytes += data.size
        per = {}
        for mm in tot:
            x = torch.from_numpy(rng.normal(0, 1, (mm, k)).astype(np.float16)).to(dev)
            y = torch.empty((mm, n), dtype=torch.float16 if mm > 16 else torch.float32, device=dev)
            us = eager_time_us(fast_launcher(pool, x, y), max(2 * len(pool), 40))
            per[f"m{mm}"] = round(us, 2)
            tot[mm] += us
        sweep[name] = per
        del pool
    out["config5_qwen2.5_7b_layer"] = {
        "weight_bytes": wbytes, "us_per_projection": sweep,
        "layer": {f"m{mm}": {"us": round(t, 2), "weight_GBps": round(wbytes / t / 1e3, 1),
                             **({"TFLOPs": round(2.0 * mm * sum(n * k for _, _, n, k in layer) / t / 1e6, 1)}
                                if mm > 16 else {})}
                  for mm, t in tot.items()}}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--pool-gib", type=float, default=1.25)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the BASELINE configs 2 / 3 / 5 sweep")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding of the quantized linear "
                          "layer is design-only (output-row split, see DESIGN.md)", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch
    from combsengine_amd import QuantFormat

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    fmt = QuantFormat.Q4K
    shapes = [(14336, 4096), (4096, 14336)]
    pools, sizes = [], []
    for si, (n, k) in enumerate(shapes):
        p, data = make_pool(fmt, n, k, args.pool_gib * (1 << 30) / len(shapes), seed=1000 + si)
        pools.append(p)
        sizes.append(data.size)
    P = min(len(p) for p in pools)
    rng = np.random.default_rng(5)
    xs = [torch.from_numpy(rng.normal(0, 1, (1, k)).astype(np.float16)).to(dev) for (_, k) in shapes]
    ys = [torch.empty((1, n), dtype=torch.float32, device=dev) for (n, _) in shapes]

    def step(i):
        e = i % P
        for s in range(len(shapes)):
            pools[s][e].matmul_into(xs[s], ys[s])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the K timed steps, captured once and replayed (timing brackets the replay)
    t_cap = time.perf_counter()
    us_per_step, graph = graph_time_us(step, args.steps, reps=1)
    wall = time.perf_counter() - t_cap
    ms_total = us_per_step * args.steps / 1e3
    step_bytes = sum(algo_bytes(sz, 1, k, n) for sz, (n, k) in zip(sizes, shapes))
    value = step_bytes * args.steps / (ms_total / 1e3) / 1e9

    # Dominant kernel: launches of one shape back to back in a graph.
    launch, tot_b, tot_us = {}, 0.0, 0.0
    traffic = load_traffic().get(HEADLINE_KERNEL, {})
    for s, (n, k) in enumerate(shapes):
        us, _ = graph_time_us(lambda i, s=s: pools[s][i % P].matmul_into(xs[s], ys[s]), 4 * P)
        b = algo_bytes(sizes[s], 1, k, n)
        launch[f"{n}x{k}"] = {"us": round(us, 3), "GBps": round(b / us / 1e3, 1),
                              "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
        tot_b += b
        tot_us += us
    achieved = tot_b / tot_us / 1e3
    t_bytes = [traffic.get(f"{n}x{k}") for (n, k) in shapes]
    traffic_val = round(sum(t_bytes) / len(t_bytes)) if all(t_bytes) else None

    extra = {} if args.no_extra else secondary(dev)
    if not args.no_extra and not args.no_configs:
        extra["configs"] = configs_2_3_5(dev)
    prefill = {k: v for k, v in extra.items() if k.startswith("prefill_")}
    best_prefill = max((v["TFLOPs"] for v in prefill.values()), default=None)

    line = {
        "metric": "Q4_K decode GEMV HBM GB/s (% of peak); prefill dequant-GEMM TFLOP/s",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_total / args.steps, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k", "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV, Llama-3-8B shapes [14336x4096]+[4096x14336], batch 1, x f16, "
                               f"y f32; weight pool {P} x {len(shapes)} buffers ({P * sum(sizes) / 2**30:.2f} GiB)",
                   "global_batch": 1, "parallelism": "none (1 GPU)"},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": HEADLINE_KERNEL, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_val,
                     "algorithmic_bytes_per_launch": round(tot_b / len(shapes)), "launches": launch},
        "prefill_TFLOPs_best": best_prefill,
        "wall_s_capture_and_replay": round(wall, 3),
        "secondary": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the MX quantize/pack + block-scaled GEMM path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]

Headline (the JSON line's `value`): config 2 of the benchmark
configurations, the int4d weight-only linear at decode shape — x fp32
[16, 8192] ~ N(0,1), W [8192 (out), 8192 (in)] ~ 0.02 N(0,1) with 0.1%
outliers x20, stored as
quantize(W.t()) int4d block 128 — one step = one mx_linear forward (one
fused kernel).  `value` = algorithmic bytes per step (packed weights 32 MiB +
scales 2 MiB + x + y = 36,700,160 B) / time per step, in GB/s.  The
kernel reads the tiled copy of the packed weight (same 32 MiB) and the
block-major scales that each layer makes once, on its first forward, before
the timed region.

Timing: W warm-up steps, then K steps captured into one HIP graph, untimed
warm replays of it (at least 3, for at least 50 ms), then one replay
between two HIP events recorded on the stream the kernels run on (torch's
current stream), synchronize on both sides; inputs are resident in HBM.
ms_per_step = elapsed / K.  Step i runs layer i % 12 of twelve identical
quantized layers (12 x 34 MiB of weights and scales, more than the
256 MiB last-level cache), so every step streams its weights from HBM rather
than from the previous step's cache lines.

`cpu_baseline`: the CPU oracle (oracle/mx_oracle.py, the reference's CPU
path restated with the same torch ops) on the full config-2 workload, 2
warm-ups then the median of 5, on this host's cores.

`extras`: configs 1, 3, 4 and 5 measured the same way, each with its
roofline fraction (HBM 8.0 TB/s, dense int8 MFMA 5.0 POP/s, dense f16 MFMA
2.5 PFLOP/s), config 2 with bfloat16 activations, config 1 with its two
quantizes, mx_linear beyond the decode shape, and the CPU oracle on bounded
samples of configs 1, 3, 4 and 5.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
F16_PEAK_TFLOPS = 2500.0
PROFILES = os.path.join(ROOT, "profiles")


def gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


EAGER = False  # --eager: launch the steps directly (no graph), for counter collection


def graph_time(step, steps: int, warmup: int, repeats: int = 1) -> float:
    """Seconds per step: `steps` calls of step() captured in one graph,
    replayed between events on the current stream (the median over
    `repeats` timed replays)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    # warm-up on the stream the graph is captured on, so that per-stream
    # workspaces exist before the capture
    with torch.cuda.stream(s):
        for _ in range(max(warmup, 1)):
            step()
    torch.cuda.synchronize()
    if EAGER:
        st = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(steps):
            step()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / steps
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(steps):
                step()
    torch.cuda.current_stream().wait_stream(s)
    # untimed warm replays for at least 50 ms of wall time (3 at least): the
    # first replays of a run are slower while the GPU clock settles (config 2:
    # 13.3 us per step in the first replay, 12.7 from the eighth on)
    t0 = time.perf_counter()
    n_warm = 0
    while n_warm < 3 or (time.perf_counter() - t0 < 0.05 and n_warm < 100):
        g.replay()
        torch.cuda.synchronize()
        n_warm += 1
    st = torch.cuda.current_stream()
    times = []
    for _ in range(max(repeats, 1)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / 1e3 / steps)
    del g
    times.sort()
    return times[len(times) // 2]


def load_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if any."""
    p = os.path.join(PROFILES, f"{name}.traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("traffic_bytes")


# ---------------------------------------------------------------- config 2
def config2_inputs():
    K = N = 8192
    x = torch.randn(16, K, generator=gen(2))
    W = 0.02 * torch.randn(N, K, generator=gen(3))
    W[torch.rand(N, K, generator=gen(4)) < 1e-3] *= 20
    return x, W


N_LAYERS = 12  # distinct weight copies cycled through by the timed steps


def bench_linear(args, qa):
    dev = torch.device("cuda:0")
    x_cpu, W_cpu = config2_inputs()
    K = N = 8192
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W_cpu)
    lin = lin.to(dev)
    layers = [qa.mx_linear.from_linear(lin, qa.get_mx_dtype("int4d"), 128) for _ in range(N_LAYERS)]
    m = layers[0]
    x = x_cpu.to(dev)
    y = m(x)
    for layer in layers:  # each layer makes its block-major scale and tiled weight copies once, outside the timed graph
        layer(x)
    torch.cuda.synchronize()
    it = [0]

    def step():
        layers[it[0] % N_LAYERS](x)
        it[0] += 1

    sec = graph_time(step, args.steps, args.warmup)
    algo_bytes = K * N // 2 + (K * N // 128) * 4 + 16 * K * 4 + 16 * N * 4
    gbs = algo_bytes / sec / 1e9
    res = {"sec": sec, "algo_bytes": algo_bytes, "gbs": gbs, "y": y.cpu(),
           "w_packed": m._mx_weight._mx_packed.cpu(), "w_scales": m._mx_weight._mx_scales.cpu(),
           "x": x_cpu}
    # the same step with config 2's bfloat16 activations (x.float() is exact)
    xb = x.bfloat16()
    it[0] = 0

    def step_bf16():
        layers[it[0] % N_LAYERS](xb)
        it[0] += 1

    sec_b = graph_time(step_bf16, args.steps, args.warmup)
    algo_b = K * N // 2 + (K * N // 128) * 4 + 16 * K * 2 + 16 * N * 4
    res["bf16"] = {"us": round(sec_b * 1e6, 3), "GBs": round(algo_b / sec_b / 1e9, 1),
                   "frac": round(algo_b / sec_b / 1e9 / HBM_PEAK_GBS, 4), "bytes": algo_b}
    return res


def cpu_baseline_linear(res):
    from oracle import mx_oracle as orc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    x, wp, ws = res["x"], res["w_packed"], res["w_scales"]

    def run():
        return orc.linear_forward(x, wp, ws, "int4d", 8192, 8192, 128)

    for _ in range(2):
        y_ref = run()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        y_ref = run()
        ts.append(time.perf_counter() - t0)
    sec = statistics.median(ts)
    err = (res["y"] - y_ref).abs().max().item() / y_ref.abs().max().item()
    return {"value": round(res["algo_bytes"] / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "full config-2 workload (x[16,8192] @ dequant(int4d W[8192,8192])), "
                      "median of 5 after 2 warm-ups",
            "sec_per_step": round(sec, 4)}, err


# ---------------------------------------------------------------- extras
def bench_quant_sweep(qa, reps):
    dev = torch.device("cuda:0")
    n = 1 << 28
    g = gen(7, "cuda")
    x = torch.randn(n, generator=g, device=dev)
    mask = torch.rand(n, generator=gen(8, "cuda"), device=dev) < 1e-3
    x[mask] *= 50
    del mask
    x = x.view(1 << 21, 128)
    out = {}
    for name in ("int8d", "int4d", "int2d", "int1d", "float4d", "float8d", "int4dh"):
        dt = qa.get_mx_dtype(name)
        bits = dt.bits
        algo = n * 4 + n * bits // 8 + (n // 128) * 4
        seed = 1534857261 if dt.is_hadamard else None
        packed, scales, _ = qa.ops.quantize(x, dt, 128, seed=seed)
        tq = graph_time(lambda: qa.ops.quantize(x, dt, 128, seed=seed), reps, 1)
        td = graph_time(lambda: qa.ops._dequant(packed, scales, dt, n, 128, orig_shape=(1 << 21, 128),
                                                seed=seed), reps, 1)
        out[name] = {"quantize_us": round(tq * 1e6, 2), "quantize_GBs": round(algo / tq / 1e9, 1),
                     "quantize_frac": round(algo / tq / 1e9 / HBM_PEAK_GBS, 4),
                     "dequantize_us": round(td * 1e6, 2), "dequantize_GBs": round(algo / td / 1e9, 1),
                     "dequantize_frac": round(algo / td / 1e9 / HBM_PEAK_GBS, 4)}
        del packed, scales
        torch.cuda.empty_cache()
    return out


def bench_gemm(qa, M, K, N, reps, dtype="int8d"):
    """Packed block-scaled GEMM A @ B (mxtorch.py:5497-5573) of two seeded
    randn operands quantized with `dtype` block 128: fp32 C out, and the
    packed int16d output the reference's matmul returns."""
    dev = torch.device("cuda:0")
    A = torch.randn(M, K, generator=gen(5, "cuda"), device=dev)
    B = torch.randn(K, N, generator=gen(6, "cuda"), device=dev)
    dt = qa.get_mx_dtype(dtype)
    pa, sa, _ = qa.ops.quantize(A, dt, 128)
    pb, sb, _ = qa.ops.quantize(B, dt, 128)
    del A, B
    bits = dt.bits
    # the median of 5 replays: back-to-back 8192^3 GEMMs move the clock by +-10% from launch to launch
    t_c = graph_time(lambda: qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, bits, 128, 16, want_packed=False,
                                                  want_c=True), reps, 1, repeats=5)
    # the packed output of qa @ qb: int16d for int8 operands, int8d for int4 (mxtorch.py:1393-1418)
    ob = qa.matmul_output_dtype(dt, dt).bits
    t_p = graph_time(lambda: qa.ops.qscale_gemm(pa, sa, pb, sb, M, K, N, bits, 128, ob), reps, 1, repeats=5)
    ops = 2.0 * M * K * N
    return {"shape": [M, K, N], "fp32_out_us": round(t_c * 1e6, 2), "fp32_out_TOPS": round(ops / t_c / 1e12, 2),
            "fp32_out_frac_int8_peak": round(ops / t_c / 1e12 / INT8_PEAK_TOPS, 4),
            f"packed_int{ob}d_out_us": round(t_p * 1e6, 2), "packed_TOPS": round(ops / t_p / 1e12, 2)}


def bench_config1_full(qa, reps):
    """Config 1 end to end: quantize the fp32 512x512 A and B (int8d block
    128), then the packed GEMM A_q @ B_q with the reference's int16d output
    (mxtorch.py:1684-1763, 5497-5573): three launches of quantize + the GEMM
    kernels per step."""
    dev = torch.device("cuda:0")
    A = torch.randn(512, 512, generator=gen(0)).to(dev)
    B = torch.randn(512, 512, generator=gen(1)).to(dev)
    dt = qa.get_mx_dtype("int8d")

    def step():
        qa.mx_tensor.quantize(A, dt, 128) @ qa.mx_tensor.quantize(B, dt, 128)

    t = graph_time(step, reps, 2, repeats=3)
    ops = 2.0 * 512 ** 3
    return {"us": round(t * 1e6, 2), "TOPS": round(ops / t / 1e12, 3),
            "note": "quantize A and B + packed GEMM + int16d requantization per step"}


def bench_linear_mfma(qa, reps):
    """mx_linear beyond the decode shape (mxtorch.py:7454-7473): x fp32 [M,
    8192] @ dequant(W [8192, 8192] stored as quantize(W.t())), M = 512 and
    8192, int4d, int8d, int2d, int1d, float4d and float8d weights.  The kernel issues two f16 MFMAs per
    product (x*s as hi + lo against the exact codes), so the f16 MFMA work is
    twice 2*M*K*N; frac_f16_peak is that work over 2.5 PFLOP/s dense f16."""
    dev = torch.device("cuda:0")
    K = N = 8192
    _, W_cpu = config2_inputs()
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W_cpu)
    lin = lin.to(dev)
    out = {}
    for name in ("int4d", "int8d", "int2d", "int1d", "float4d", "float8d"):
        m = qa.mx_linear.from_linear(lin, qa.get_mx_dtype(name), 128)
        for M in (512, 8192):
            x = torch.randn(M, K, generator=gen(20 + M, "cuda"), device=dev)
            with torch.no_grad():
                m(x)
                t = graph_time(lambda: m(x), reps if M <= 512 else max(2, reps // 4), 1, repeats=3)
            flops = 2.0 * M * K * N
            out[f"{name}_{M}x{K}x{N}"] = {"us": round(t * 1e6, 2), "TFLOPS": round(flops / t / 1e12, 1),
                                          "f16_mfma_TFLOPS": round(2 * flops / t / 1e12, 1),
                                          "frac_f16_peak": round(2 * flops / t / 1e12 / F16_PEAK_TFLOPS, 4)}
            del x
        if name in ("int8d", "int2d", "int1d", "float4d", "float8d"):
            # decode batch (16 rows): the decode kernels (float4d on its tiled copy), HBM-bound
            x = torch.randn(16, K, generator=gen(36, "cuda"), device=dev)
            with torch.no_grad():
                m(x)
                t = graph_time(lambda: m(x), reps * 5, 1, repeats=3)
            bits = qa.get_mx_dtype(name).bits
            # codes, block scales, x, y (as config 2)
            nbytes = K * N * bits // 8 + (K * N // 128) * 4 + 16 * K * 4 + 16 * N * 4
            out[f"{name}_decode_16x8192x8192"] = {"us": round(t * 1e6, 2), "GBs": round(nbytes / t / 1e9, 1),
                                                  "frac_hbm": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                                                  "bytes": nbytes}
            del x
        del m
        torch.cuda.empty_cache()
    return out


# The reference's published rows (README.md:590-595, 599-603, 618-624; RX
# 7900 XTX, its Triton path), in ms
README_QUANT_MS = {("int4d", 512): 0.05, ("int4d", 1024): 0.07, ("int8d", 512): 0.05, ("int8d", 1024): 0.06,
                   ("float4d", 512): 0.24, ("float4d", 1024): 0.30, ("float8d", 512): 0.18, ("float8d", 1024): 0.23}
README_GEMM_MS = {256: 0.073, 512: 0.085, 1024: 0.190}
README_LINEAR_MS = {(512, 512): {"int8d": 0.82, "int4d": 1.75}, (1024, 512): {"int8d": 0.83, "int4d": 1.89},
                    (2048, 1024): {"int8d": 0.82, "int4d": 2.16}}


def bench_readme_rows(qa):
    """The reference's own published benchmark rows, timed the way its
    benchmark times them (mxtorch_test.py:3474-3496, 3523-3580, 3616-3628):
    3 eager warm-up calls, then 20 eager calls each bracketed by a pair of
    events and a synchronize, and the mean in ms.  Rows: quantize 512^2 and
    1024^2 (block 128) for int4d / int8d / float4d / float8d; the int8d GEMM
    _dispatch_qgemm of 256^3, 512^3, 1024^3 operands quantized with block 64;
    mx_linear at batch 32 for 512->512, 1024->512, 2048->1024 (int8d and
    int4d weights, block 128).  Each row carries the published RX 7900 XTX
    time and published / ours."""
    from qtpytorch_amd.tensor import _dispatch_qgemm

    dev = torch.device("cuda:0")

    def ev_mean(fn, warmup=3, runs=20):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(runs):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return statistics.mean(ts)

    def row(ms, pub):
        return {"ms": round(ms, 4), "published_ms": pub, "published_over_ours": round(pub / ms, 1)}

    out = {"method": "eager calls, event pair per call, mean of 20 after 3 warm-ups (the reference's _bench)"}
    q = {}
    for n in (512, 1024):
        x = torch.randn(n, n, generator=gen(300 + n, "cuda"), device=dev)
        for name in ("int4d", "int8d", "float4d", "float8d"):
            dt = qa.get_mx_dtype(name)
            q[f"{name}_{n}x{n}"] = row(ev_mean(lambda: qa.mx_tensor.quantize(x, dt, 128)), README_QUANT_MS[(name, n)])
    out["quantize"] = q
    g = {}
    for n in (256, 512, 1024):
        a = qa.mx_tensor.quantize(torch.randn(n, n, generator=gen(310 + n, "cuda"), device=dev),
                                  qa.get_mx_dtype("int8d"), 64)
        b = qa.mx_tensor.quantize(torch.randn(n, n, generator=gen(320 + n, "cuda"), device=dev),
                                  qa.get_mx_dtype("int8d"), 64)
        g[f"int8d_{n}^3_block64"] = row(ev_mean(lambda: _dispatch_qgemm(a, b)), README_GEMM_MS[n])
    out["qgemm"] = g
    lin_rows = {}
    for (k, n), pubs in README_LINEAR_MS.items():
        lin = torch.nn.Linear(k, n, device=dev)
        x = torch.randn(32, k, generator=gen(330 + k, "cuda"), device=dev)
        for name, pub in pubs.items():
            m = qa.mx_linear.from_linear(lin, qa.get_mx_dtype(name), 128)
            with torch.no_grad():
                lin_rows[f"{name}_{k}->{n}_batch32"] = row(ev_mean(lambda: m(x)), pub)
    out["mx_linear"] = lin_rows
    return out


def cpu_baselines_extra():
    """The CPU oracle (the reference's CPU path restated) on bounded
    samples of configs 1, 3, 4 and 5, 2 warm-ups then the median of 5, on
    this host's cores; each entry states its sample."""
    from oracle import mx_oracle as orc

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def timed(f, runs=5):
        for _ in range(2):
            f()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            f()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    out = {}
    A = torch.randn(512, 512, generator=gen(0))
    B = torch.randn(512, 512, generator=gen(1))

    def c1():
        pa, sa, na = orc.quantize(A, "int8d", 128)
        pb, sb, nb = orc.quantize(B, "int8d", 128)
        orc.dispatch_qgemm(pa, sa, "int8d", (512, 512), na, pb, sb, "int8d", (512, 512), nb, 128)

    t = timed(c1)
    out["config1"] = {"value": round(2 * 512 ** 3 / t / 1e12, 5), "unit": "TOPS", "cores": cores, "kind": "port",
                      "sample": "full config 1: quantize A, B (int8d) + _dispatch_qgemm 512^3", "sec": round(t, 5)}
    # config 3: the first 512 rows of A against all of B (the product's rows are independent)
    Mr, K, N = 512, 8192, 8192
    a = torch.randint(-127, 128, (Mr * K,), generator=gen(5), dtype=torch.int32)
    b = torch.randint(-127, 128, (K * N,), generator=gen(6), dtype=torch.int32)
    sa = torch.rand(Mr * K // 128, generator=gen(7)) * 0.02
    sb = torch.rand(K * N // 128, generator=gen(8)) * 0.02
    t = timed(lambda: orc.qscale_matmul(a, sa, b, sb, Mr, K, N, 8, 128, 16, return_c=True), runs=3)
    out["config3"] = {"value": round(2.0 * Mr * K * N / t / 1e12, 5), "unit": "TOPS", "cores": cores,
                      "kind": "port", "sample": "512 of the 8192 rows of the 8192^3 _qscale_matmul "
                                                "(64 K-block mm + epilogue + int16 requant), median of 3",
                      "sec": round(t, 4)}
    del a, b
    # config 4: 2^24 elements of the seeded fp32 tensor, quantize then dequantize
    n = 1 << 24
    x = torch.randn(n, generator=gen(7))
    x[torch.rand(n, generator=gen(8)) < 1e-3] *= 50
    x = x.view(-1, 128)
    c4 = {}
    for name in ("int8d", "int4d", "float4d"):
        bits = 8 if name.endswith("8d") else 4
        algo = n * 4 + n * bits // 8 + (n // 128) * 4
        tq = timed(lambda: orc.quantize(x, name, 128))
        pk, sc, _ = orc.quantize(x, name, 128)
        td = timed(lambda: orc.dequant(pk, sc, name, n, 128))
        c4[name] = {"quantize_GBs": round(algo / tq / 1e9, 3), "dequantize_GBs": round(algo / td / 1e9, 3)}
    out["config4"] = {"value": c4["int4d"]["quantize_GBs"], "unit": "GB/s", "cores": cores, "kind": "port",
                      "sample": "2^24 of the 2^28 elements (int4d quantize is `value`)", "dtypes": c4}
    # config 5: 2^17 rows of 128 fp16 (2^24 elements) of K, int8dv and int4d
    kx = torch.randn(1 << 17, 128, generator=gen(9)).half()
    c5 = {}
    for name in ("int8dv", "int4d"):
        bits = 8 if name.startswith("int8") else 4
        nq = kx.numel()
        tq = timed(lambda: orc.quantize(kx, name, 128))
        pk, sc, _ = orc.quantize(kx, name, 128)
        td = timed(lambda: orc.dequant(pk, sc, name, nq, 128))
        c5[name] = {"quantize_GBs": round((nq * 2 + nq * bits // 8 + nq // 128 * 4) / tq / 1e9, 3),
                    "dequantize_GBs": round((nq * 4 + nq * bits // 8 + nq // 128 * 4) / td / 1e9, 3)}
    out["config5"] = {"value": c5["int8dv"]["quantize_GBs"], "unit": "GB/s", "cores": cores, "kind": "port",
                      "sample": "2^17 rows x 128 of the fp16 K tensor (int8dv quantize is `value`)", "dtypes": c5}
    return out


def bench_kv(qa, reps):
    dev = torch.device("cuda:0")
    shape = (8, 32, 4096, 128)
    out = {}
    k = torch.randn(*shape, generator=gen(9, "cuda"), device=dev).half()
    v = torch.randn(*shape, generator=gen(10, "cuda"), device=dev).half()
    rows_k, rows_v = k.view(-1, 128), v.view(-1, 128)
    n = rows_k.numel()
    for name in ("int8dv", "int4d"):
        dt = qa.get_mx_dtype(name)
        q_algo = 2 * (n * 2 + n * dt.bits // 8 + (n // 128) * 4)
        d_algo = 2 * (n * 4 + n * dt.bits // 8 + (n // 128) * 4)
        pk, sk, _ = qa.ops.quantize(rows_k, dt, 128)
        pv, sv, _ = qa.ops.quantize(rows_v, dt, 128)

        def q():
            qa.ops.quantize(rows_k, dt, 128)
            qa.ops.quantize(rows_v, dt, 128)

        def d():
            qa.ops._dequant(pk, sk, dt, n, 128)
            qa.ops._dequant(pv, sv, dt, n, 128)

        tq = graph_time(q, reps, 1)
        td = graph_time(d, reps, 1)
        out[name] = {"quantize_us": round(tq * 1e6, 2), "quantize_GBs": round(q_algo / tq / 1e9, 1),
                     "quantize_frac": round(q_algo / tq / 1e9 / HBM_PEAK_GBS, 4),
                     "dequantize_us": round(td * 1e6, 2), "dequantize_GBs": round(d_algo / td / 1e9, 1),
                     "dequantize_frac": round(d_algo / td / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def bench_elementwise(qa, reps):
    """Quantized element-wise add / mul (mxtorch.py:5321-5497) on 2^28
    elements, block 128: packed codes and scales in, packed codes and scales
    out (one launch)."""
    dev = torch.device("cuda:0")
    n = 1 << 28
    out = {}
    x = torch.randn(n, generator=gen(13, "cuda"), device=dev)
    y = torch.randn(n, generator=gen(14, "cuda"), device=dev) * 0.3
    for name in ("int8d", "int4d"):
        dt = qa.get_mx_dtype(name)
        A = qa.mx_tensor.quantize(x, dt, 128)
        B = qa.mx_tensor.quantize(y, dt, 128)
        nb = n // 128
        for op in ("add", "mul"):
            ob = dt.bits if op == "add" else qa.dtypes.qmul_output_dtype(dt).bits
            algo = n * (2 * dt.bits + ob) // 8 + 3 * nb * 4
            f = (lambda: A + B) if op == "add" else (lambda: A * B)
            t = graph_time(f, reps, 1, repeats=3)
            out[f"{name}_{op}"] = {"us": round(t * 1e6, 2), "GBs": round(algo / t / 1e9, 1),
                                   "frac": round(algo / t / 1e9 / HBM_PEAK_GBS, 4), "bytes": algo}
        del A, B
    return out


def bench_kv_stream(qa, steps):
    """kv_cache_quantizer streaming at config 5's shape: per-step append of
    K, V [8, 32, 1, 128] fp16 (one fused launch into the ring), then get()
    over 4096 steps (one gather launch per tensor)."""
    dev = torch.device("cuda:0")
    B, H, D, T = 8, 32, 128, 4096
    rows = B * H
    out = {}
    ks = torch.randn(steps, B, H, 1, D, generator=gen(11, "cuda"), device=dev).half()
    vs = torch.randn(steps, B, H, 1, D, generator=gen(12, "cuda"), device=dev).half()
    for name in ("int8dv", "int4d"):
        dt = qa.get_mx_dtype(name)
        cache = qa.kv_cache_quantizer(n_heads=H, head_dim=D, dtype=name, max_seq_len=T)
        # fill the ring to T steps (eager), so that appends below evict and get() sees T steps
        for t in range(T):
            cache.append_kv(ks[t % steps], vs[t % steps])
        i = [0]

        def step():
            cache.append_kv(ks[i[0] % steps], vs[i[0] % steps])
            i[0] += 1

        t_app = graph_time(step, steps, 2)
        t_get = graph_time(lambda: cache.get(), 3, 1, repeats=3)
        n = rows * T * D
        code_b = n * dt.bits // 8
        get_algo = 2 * (code_b + rows * T * 4 + n * 4) + rows * T * 4  # codes, scales, out (K and V) + V zero points
        app_algo = 2 * (rows * D * 2 + rows * D * dt.bits // 8 + rows * 4) + rows * 4
        out[name] = {"append_us_per_step": round(t_app * 1e6, 3), "append_bytes": app_algo,
                     "get_us": round(t_get * 1e6, 2), "get_GBs": round(get_algo / t_get / 1e9, 1),
                     "get_frac": round(get_algo / t_get / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def bench_dynamic(qa, steps, reps):
    """The int8 x int8 / dynamic-activation row (mxtorch.py:2665-2731,
    3910-3960, 8870-8968):
      * mx_dynamic_linear forward at config 2's decode shape: x fp32 [16, 8192]
        @ dequant(W int4d stored [8192 out][8192 in], block 128 along in).T,
        12 rotated layers as for the headline; HBM-bound, same algorithmic
        bytes as config 2;
      * fused_int8_linear with per-token int8 activations [8192, 8192] and int8d
        weights [8192, 8192] block 128: 2*8192^3 int8 ops on MFMA;
      * dynamic_quantize per token of fp32 [8192, 8192] to int8: 4 B read +
        1 B written per element + 4 B per row;
      * the same tensor per channel and per tensor: two passes (the absmax,
        then the codes), bytes counted as one read of x + the codes + the
        scales, so 0.5 is the ceiling of a two-read kernel pair."""
    dev = torch.device("cuda:0")
    out = {}
    x_cpu, W_cpu = config2_inputs()
    K = N = 8192
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(W_cpu)
    lin = lin.to(dev)
    layers = [qa.mx_dynamic_linear.from_linear(lin, "int4d", "int8d") for _ in range(N_LAYERS)]
    del lin
    x = x_cpu.to(dev)
    it = [0]

    def step():
        layers[it[0] % N_LAYERS](x)
        it[0] += 1

    t = graph_time(step, steps, 5)
    algo = K * N // 2 + (K * N // 128) * 4 + 16 * K * 4 + 16 * N * 4
    out["dynamic_linear_int4d_decode_16x8192x8192"] = {
        "us": round(t * 1e6, 2), "GBs": round(algo / t / 1e9, 1), "frac": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
        "bytes": algo}
    del layers
    torch.cuda.empty_cache()

    M = 8192
    xa = torch.randn(M, K, generator=gen(15, "cuda"), device=dev)
    wa = torch.randn(N, K, generator=gen(16, "cuda"), device=dev) * 0.02
    xq = qa.dynamic_quantize(xa, "int8d", "per_token")
    wq = qa.mx_tensor.quantize(wa, qa.get_mx_dtype("int8d"), 128)
    t = graph_time(lambda: qa.fused_int8_linear(xq, wq), reps, 1, repeats=5)
    ops = 2.0 * M * K * N
    out["fused_int8_linear_per_token_8192"] = {"us": round(t * 1e6, 2), "TOPS": round(ops / t / 1e12, 2),
                                               "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4)}
    del wa, wq, xq
    torch.cuda.empty_cache()
    t = graph_time(lambda: qa.dynamic_quantize(xa, "int8d", "per_token"), reps, 1, repeats=3)
    algo = M * K * 5 + M * 4
    out["dynamic_quantize_per_token_8192x8192"] = {
        "us": round(t * 1e6, 2), "GBs": round(algo / t / 1e9, 1), "frac": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
        "bytes": algo}
    for gran, ns in (("per_channel", K), ("per_tensor", 1)):
        t = graph_time(lambda: qa.dynamic_quantize(xa, "int8d", gran), reps, 1, repeats=3)
        algo = M * K * 5 + ns * 4
        out[f"dynamic_quantize_{gran}_8192x8192"] = {
            "us": round(t * 1e6, 2), "GBs": round(algo / t / 1e9, 1),
            "frac": round(algo / t / 1e9 / HBM_PEAK_GBS, 4), "bytes": algo}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of extras: quant,gemm,gemm4,kv,kvstream,elementwise,small,mfma,dynamic,readme,cpu")
    ap.add_argument("--eager", action="store_true", help="no graph capture (for rocprofv3 --pmc runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 512 MiB device copy (the reference kernel for HBM counter scaling)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every box in this build has one MI355X, and the path shards "
              "without collectives (see the design notes); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        a = torch.empty(1 << 27, device="cuda:0").fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": a.numel() * 4, "copy_bytes_written": b.numel() * 4}))
        return
    import qtpytorch_amd as qa

    res = bench_linear(args, qa)
    line = {
        "metric": "packed GEMM TOPS (int8d/int4d) + quantize GB/s; % of MI355X roofline",
        "value": round(res["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["sec"] * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (int4 codes; x*s as f16 hi+lo on f16 MFMA, f32 accumulate)",
        "data": "synthetic (seeded randn; weights 0.02*randn with 0.1% outliers x20)",
        "config": {"workload": "int4d weight-only linear, decode: x fp32 [16,8192] @ dequant(W int4d [8192,8192] "
                               "block 128), one mx_linear forward per step",
                   "M": 16, "K": 8192, "N": 8192, "block": 128, "weight_dtype": "int4d", "x_dtype": "float32"},
        "roofline": {"bound": "hbm", "achieved": round(res["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(res["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("linear_int4d_decode_16x8192x8192")},
    }
    if not args.no_cpu:
        cb, err = cpu_baseline_linear(res)
        line["cpu_baseline"] = cb
        line["max_rel_err_vs_oracle"] = err
    else:
        line["cpu_baseline"] = None
    if not args.no_extras:
        only = set(filter(None, args.only.split(",")))
        extras = {}
        extras["config2_bf16_x"] = res["bf16"]
        if not only or "small" in only:
            extras["config1_int8d_gemm_512"] = bench_gemm(qa, 512, 512, 512, 50)
            extras["config1_with_quantize_512"] = bench_config1_full(qa, 50)
        if not only or "mfma" in only:
            extras["mx_linear_mfma"] = bench_linear_mfma(qa, 20)
        if not only or "gemm" in only:
            extras["config3_int8d_gemm_8192"] = bench_gemm(qa, 8192, 8192, 8192, 3)
        if not only or "gemm4" in only:
            extras["int4d_gemm_8192"] = bench_gemm(qa, 8192, 8192, 8192, 3, "int4d")
        if not only or "quant" in only:
            extras["config4_quant_sweep_2e28"] = bench_quant_sweep(qa, 5)
        if not only or "kv" in only:
            extras["config5_kv_8x32x4096x128_fp16"] = bench_kv(qa, 5)
        if not only or "elementwise" in only:
            extras["elementwise_2e28_block128"] = bench_elementwise(qa, 5)
        if not only or "kvstream" in only:
            extras["kv_ring_stream_8x32x128_T4096"] = bench_kv_stream(qa, 64)
        if not only or "dynamic" in only:
            extras["dynamic_int8"] = bench_dynamic(qa, 120, 5)
        if not only or "readme" in only:
            extras["reference_published_rows"] = bench_readme_rows(qa)
        if not args.no_cpu and (not only or "cpu" in only):
            extras["cpu_baselines"] = cpu_baselines_extra()
        line["extras"] = extras
    print(json.dumps(line))


if __name__ == "__main__":
    main()

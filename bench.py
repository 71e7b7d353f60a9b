#!/usr/bin/env python3
"""Benchmark of the MI355X backend on BASELINE.json's headline metric.

Default workload: bf16 dense GEMM C = A @ B with
fp32 accumulation and bf16 output, M = N = K = 8192, A row-major [M,K], B
column-major (stored [N,K]), A,B ~ Normal(0,1)/sqrt(K) from seeds 1 and 2,
generated on the GPU. A "step" is one pyc_hip_gemm_dispatch launch over the
resident operands. Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--workload NAME]

The default line also carries one nested block per other BASELINE config,
each with its own roofline, HBM traffic and CPU baselines (min(cores, 32)
threads and one thread): "attention" (config 3, causal [8,32,2048,128] bf16),
"engine_cfg1" (config 1 through pyc_compile_model/pyc_run_model with
device-resident tensors, with the reference bench driver's fields under
"engine": execution path, profile, latency), "conv" (config 4, NHWC
32x56x56x256 -> 256, 3x3, +bias +ReLU) and "decode_chain" (config 5, the
8-layer fp8-weight chain as hipGraph replays). --no-extras leaves them out.

Other workloads (--workload) measure the remaining BASELINE configs for the
record; they are not the bench line the driver reads by default. Every line
carries "latency_ms" (mean/p50/p95/min/max of the per-launch device times, or
of the pyc_run_model wall times for the engine) and "settle": before the
warmup steps each workload runs back to back for --settle-ms (default 400 ms)
so the timed steps see the clock the card holds under sustained load, not an
idle card's ramp.

The cpu_baseline leg times the reference's own CPU executor (the C11 engine
built from the reference sources into oracle/_ref/libpyc_ref.so, through
pyc_compile_model/pyc_run_model) on a bounded row sample of the same GEMM, or
the oracle's restatement when that library is absent.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "bf16 GEMM/attention TFLOP/s + % MFMA peak at 1 MI355X; speedup vs CPU executor"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 MFMA (published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- timing helpers


def settle(torch, launch, ms: float) -> dict:
    """Run the launch back to back for `ms` of wall time before the warmup
    steps. An idle card's engine clock ramps up over the first tens to
    hundreds of milliseconds of load; without this the few warmup steps a
    short run asks for would be timed at a clock the card does not hold under
    sustained load. Untimed; reported as "settle"."""
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            launch()
        torch.cuda.synchronize()
        n += 8
    return {"ms": (time.perf_counter() - t0) * 1e3, "launches": n}


_LAST_SETTLE: dict = {}


def time_launches(torch, launch, steps: int, warmup: int, settle_ms: float = 0.0):
    """Settle the clock, warm up, then time `steps` launches back to back,
    bracketed by synchronize, with one HIP event before the first launch and
    one after the last, both recorded on the stream the launches run on.
    Returns (wall ms per step, device ms per launch, per-launch ms). The device
    ms per launch is that event span over `steps`: back to back, the command
    processor readies each dispatch while the previous kernel runs, so this is
    the kernel's own duration plus the dispatch gap. Events between the
    launches would add their own gap to every step (about 5 us on this stack,
    4 % of a 120 us kernel), so the per-launch times (reported as latency_ms)
    come from a second, untimed pass with an event pair around each launch."""
    stream = torch.cuda.current_stream()
    _LAST_SETTLE.clear()
    if settle_ms > 0:
        _LAST_SETTLE.update(settle(torch, launch, settle_ms))
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    e_first, e_last = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e_first.record(stream)
    for _ in range(steps):
        launch()
    e_last.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    span = e_first.elapsed_time(e_last) / steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record(stream)
        launch()
        e1.record(stream)
    torch.cuda.synchronize()
    per = [e0.elapsed_time(e1) for e0, e1 in evs]
    _LAST_LATENCY.clear()
    _LAST_LATENCY.update(latency_stats(per))
    return wall_ms / steps, span, per


# per-launch device-time statistics of the last timed loop (reported as
# latency_ms, the reference bench driver's field)
_LAST_LATENCY: dict = {}


def latency_stats(ms) -> dict:
    a = np.asarray(ms, dtype=np.float64)
    return {"mean": float(a.mean()), "p50": float(np.percentile(a, 50)), "p95": float(np.percentile(a, 95)),
            "min": float(a.min()), "max": float(a.max())}


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), committed under profiles/."""
    p = os.path.join(ROOT, "profiles", f"{name}.traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


# ---------------------------------------------------------------- CPU baseline


def _host_cores() -> int:
    """Cores this process may run on (the GPU box pins a CPU share)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _host_info() -> dict:
    """The CPU the cpu_baseline legs ran on: model name, logical CPUs of the
    machine and the ones this process may use."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "cores_available": _host_cores()}


def cpu_baseline_gemm(a_rows_f32: np.ndarray, b_kn_f32: np.ndarray, full_flops: float, sample_desc: str,
                      threads: int | None = None):
    """Time the reference CPU executor on a[rows] @ b (fp32) and scale to the
    metric's unit (TFLOP/s on the full workload's FLOP count; the per-row cost
    is constant so throughput extrapolates linearly). threads: the executor's
    PYC_NUM_THREADS (default min(cores, 32), the reference's cap; 1 is the
    reference default)."""
    rows, k = a_rows_f32.shape
    n = b_kn_f32.shape[1]
    flops = 2.0 * rows * k * n
    threads = threads or min(_host_cores(), 32)
    try:
        from tests import refengine
        use_ref = refengine.available()
    except Exception:  # noqa: BLE001
        use_ref = False
    out = None
    if use_ref:
        os.environ["PYC_NUM_THREADS"] = str(threads)
        model = refengine.matmul_model(rows, k, n)
        try:
            model.run([a_rows_f32, b_kn_f32], [(rows, n)])  # warm (page-in)
            t0 = time.perf_counter()
            st, (out,), _ = model.run([a_rows_f32, b_kn_f32], [(rows, n)])
            dt = time.perf_counter() - t0
        finally:
            model.close()
            os.environ.pop("PYC_NUM_THREADS", None)
        assert st == 0
        kind = "reference"
    else:
        import oracle
        t0 = time.perf_counter()
        out = oracle.matmul_f32(a_rows_f32, b_kn_f32, threads)
        dt = time.perf_counter() - t0
        kind = "port"
    tflops = flops / dt / 1e12
    return {
        "value": tflops,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{sample_desc}; {flops / 1e9:.1f} GFLOP in {dt:.2f} s, extrapolated linearly "
                  f"(full job {full_flops / 1e12:.3f} TFLOP -> {full_flops / flops * dt:.0f} s)",
    }, out


# ---------------------------------------------------------------- workloads


def wl_gemm_bf16(torch, args):
    import pyc_amd
    M = N = K = 8192
    g1 = torch.Generator(device="cuda").manual_seed(1)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    A = (torch.randn((M, K), generator=g1, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    B = (torch.randn((N, K), generator=g2, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    Cd = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    sym = args.symbol or "hip_gemm_bf16_nt"
    launch = lambda: pyc_amd.gemm(sym, A, B, Cd, M, N, K)  # noqa: E731
    ms_step, ms_kernel, _ = time_launches(torch, launch, args.steps, args.warmup, args.settle_ms)
    flops = 2.0 * M * N * K
    value = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (ms_kernel * 1e-3) / 1e12
    res = {
        "value": value, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": {"workload": "gemm_bf16_nt_8192x8192x8192", "kernel": sym, "M": M, "N": N, "K": K,
                   "layout": "A row-major [M,K], B column-major [N,K], C row-major bf16",
                   "accumulate": "fp32", "seeds": [1, 2], "init": "Normal(0,1)/sqrt(K)"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic("gemm_bf16_nt_8192"),
                     "kernel_ms": ms_kernel, "algorithmic_flop_per_launch": flops,
                     "algorithmic_bytes_per_launch": 3 * M * N * 2},
    }
    if not args.no_cpu:
        import oracle
        rows = np.arange(0, M, M // args.cpu_rows)[: args.cpu_rows]
        ridx = torch.from_numpy(rows).cuda()
        a_rows = A[ridx].float().cpu().numpy()
        b_kn = np.ascontiguousarray(B.float().cpu().numpy().T)
        cpu, out = cpu_baseline_gemm(a_rows, b_kn, flops,
                                     f"{len(rows)} of {M} rows of the 8192^3 GEMM, fp32 executor on the "
                                     "exactly decoded bf16 operands")
        res["cpu_baseline"] = cpu
        got = Cd[ridx].float().cpu().numpy()
        res["parity_sample_max_rel_err"] = float(np.abs(got - out).max() / np.abs(out).max())
        res["speedup_vs_cpu"] = value / cpu["value"]
        # the reference executor's default (PYC_NUM_THREADS unset): one thread
        n1 = max(1, args.cpu_rows // 16)
        cpu1, _ = cpu_baseline_gemm(a_rows[:n1], b_kn, flops,
                                    f"{n1} of {M} rows of the 8192^3 GEMM, fp32 executor, 1 thread", threads=1)
        res["cpu_baseline_1thread"] = cpu1
        del oracle
    return res


def wl_gemm_bf16_nn(torch, args):
    """Config 2's GEMM with B stored row-major [K,N]: the layout of the IR's
    MATMUL and of the reference's default bf16 symbol
    cutlass_gemm_tensorcore_bf16 (reference gemm/kernel.cu:175-187), on the
    persistent kernel's [K,N] form."""
    import pyc_amd
    M = N = K = 8192
    g1 = torch.Generator(device="cuda").manual_seed(1)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    A = (torch.randn((M, K), generator=g1, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    B = (torch.randn((K, N), generator=g2, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    Cd = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    sym = args.symbol or "cutlass_gemm_tensorcore_bf16"
    launch = lambda: pyc_amd.gemm(sym, A, B, Cd, M, N, K)  # noqa: E731
    ms_step, ms_kernel, _ = time_launches(torch, launch, args.steps, args.warmup, args.settle_ms)
    flops = 2.0 * M * N * K
    return {
        "value": flops / (ms_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": {"workload": "gemm_bf16_nn_8192x8192x8192", "kernel": sym, "M": M, "N": N, "K": K,
                   "layout": "A row-major [M,K], B row-major [K,N], C row-major bf16"},
        "roofline": {"bound": "mfma", "achieved": flops / (ms_kernel * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (ms_kernel * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic("gemm_bf16_nn_8192"), "kernel_ms": ms_kernel},
    }


def wl_gemm_f32_cfg1(torch, args):
    import pyc_amd
    M = N = K = 1024
    r = np.random.default_rng(0)
    x = r.uniform(-1, 1, (M, K)).astype(np.float32)
    w = r.uniform(-1, 1, (K, N)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    X, W, Bv = (torch.from_numpy(t).cuda() for t in (x, w, b))
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    epi = pyc_amd.abi.EPI_BIAS | pyc_amd.abi.EPI_RELU
    launch = lambda: pyc_amd.gemm("hip_gemm_f32_nn_64x64", X, W, Y, M, N, K, bias=Bv, epilogue=epi)  # noqa: E731
    ms_step, ms_kernel, _ = time_launches(torch, launch, args.steps, args.warmup, args.settle_ms)
    flops = 2.0 * M * N * K + 2.0 * M * N
    value = flops / (ms_step * 1e-3) / 1e12
    res = {
        "value": value, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "f32",
        "config": {"workload": "gemm_f32_bias_relu_1024", "M": M, "N": N, "K": K},
        "roofline": {"bound": "mfma", "achieved": flops / (ms_kernel * 1e-3) / 1e12, "peak": PEAK_F32_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (ms_kernel * 1e-3) / 1e12 / PEAK_F32_TFLOPS,
                     "traffic": load_traffic("gemm_f32_cfg1"), "kernel_ms": ms_kernel},
    }
    if not args.no_cpu:
        cpu, out = cpu_baseline_gemm(x, w, flops, "full config-1 GEMM (bias+ReLU not timed)")
        res["cpu_baseline"] = cpu
    return res


def hbm_copy_gbs(torch, nbytes: int = 1 << 31, reps: int = 10) -> dict:
    """Measured HBM bandwidth on this box: a device-to-device copy of `nbytes`
    (torch's copy kernel), timed over `reps` back-to-back copies by HIP events
    after three untimed ones; bytes read plus bytes written over the time. The
    published 8 TB/s stays the roofline's `peak`. torch's copy kernel reaches
    about 5 TB/s here, below what a streaming kernel reaches (the library's
    elementwise kernels move 6.3 TB/s), so this is a floor of the achievable
    rate, reported for reference, not a denominator."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return {"value": 2.0 * nbytes / (ms * 1e-3) / 1e9, "unit": "GB/s",
            "how": f"device-to-device copy of {nbytes >> 20} MiB (torch), read + write bytes, {reps} copies"}


def wl_decode_chain(torch, args):
    """Config 5: 8 x [x(32x4096) -> W_up(4096x11008, fp8) -> ReLU -> W_down(11008x4096, fp8)],
    the 16 GEMM steps run as one persistent launch, captured in a hipGraph and replayed."""
    import pyc_amd
    L, M, D, F = 8, 32, 4096, 11008
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((M, D), generator=g, device="cuda").to(torch.bfloat16)
    layers = []
    for l in range(L):
        gl = torch.Generator(device="cuda").manual_seed(10 + l)
        w_up = torch.randn((D, F), generator=gl, device="cuda") * np.sqrt(2.0 / D)
        w_dn = torch.randn((F, D), generator=gl, device="cuda") * np.sqrt(2.0 / F)
        pack = []
        for w in (w_up, w_dn):  # per-output-column scale, stored [N,K] e4m3fn
            s = (w.abs().amax(0) / 448.0).clamp_min(1e-30)
            q = (w / s).t().contiguous().to(torch.float8_e4m3fn).view(torch.uint8)
            pack += [q, s.float().contiguous()]
        layers.append(pack)
        del w_up, w_dn
    y = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    chain_layers = []
    for qu, su, qd, sd in layers:
        chain_layers += [(qu, su, True), (qd, sd, False)]

    # the whole chain is one launch (pyc_hip_w8a16_chain_dispatch), captured once
    pyc_amd.w8a16_chain_reserve(M, chain_layers)
    pyc_amd.w8a16_chain(x, chain_layers, y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        graph.capture_begin()
        pyc_amd.w8a16_chain(x, chain_layers, y, stream=s.cuda_stream)
        graph.capture_end()
    torch.cuda.synchronize()
    ms_step, ms_kernel, _ = time_launches(torch, graph.replay, args.steps, args.warmup, args.settle_ms)
    if pyc_amd.w8a16_chain_error() != 0:
        raise RuntimeError("decode chain: a workgroup timed out waiting (output invalid)")
    weight_bytes = L * (2 * D * F + 4 * (F + D))
    bytes_replay = L * (2 * D * F + 4 * F + 4 * D + M * D * 2 + 2 * M * F * 2 + M * D * 2)
    gbs = bytes_replay / (ms_step * 1e-3) / 1e9
    copy = hbm_copy_gbs(torch)
    extra = {}
    if not args.no_cpu:
        # CPU leg: the oracle's fp8-weight layer (the reference has no fp8
        # executor), the whole 16-layer chain on the host cores, and one
        # layer on one thread (extrapolated to the chain)
        import oracle
        host = [(q.cpu().numpy(), s_.cpu().numpy(), relu) for q, s_, relu in chain_layers]
        xh = x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        threads = min(_host_cores(), 32)
        t0 = time.perf_counter()
        cur = xh
        for q, s_, relu in host:
            cur = oracle.w8a16_layer(cur, q, s_, relu, threads)
        dt = time.perf_counter() - t0
        extra["cpu_baseline"] = {"value": bytes_replay / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
                                 "sample": f"the whole 16-layer chain (one replay), oracle fp8-weight layer in fp32 "
                                           f"threaded over output channels, {dt:.2f} s"}
        t0 = time.perf_counter()
        oracle.w8a16_layer(xh, host[0][0], host[0][1], True, 1)
        dt1 = (time.perf_counter() - t0) * len(host)
        extra["cpu_baseline_1thread"] = {"value": bytes_replay / dt1 / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                                         "sample": f"one 32x4096x11008 layer on 1 thread, {dt1 / len(host):.2f} s, "
                                                   "extrapolated to the 16 layers"}
        got = oracle.bf16_to_f32(y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
        ref = oracle.bf16_to_f32(cur)
        extra["parity_sample_max_rel_err"] = float(np.abs(got - ref).max() / np.abs(ref).max())
        extra["speedup_vs_cpu"] = gbs / extra["cpu_baseline"]["value"]
    return {**extra,
        "value": gbs, "unit": "GB/s", "ms_per_step": ms_step, "dtype": "fp8-e4m3 weights, bf16 activations",
        "config": {"workload": "decode_w8a16_chain_8x(32x4096x11008)", "replay": "hipGraph", "launches": 1,
                   "kernel": "w8a16_chain_kernel (16 GEMM steps in one persistent launch)"},
        "roofline": {"bound": "hbm", "achieved": bytes_replay / (ms_kernel * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": bytes_replay / (ms_kernel * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "traffic": load_traffic("decode_chain"), "kernel_ms": ms_kernel,
                     "algorithmic_bytes_per_replay": bytes_replay,
                     "weight_bytes": weight_bytes, "measured_copy": copy},
    }


def wl_attention(torch, args):
    """Config 3: causal attention [8,32,2048,128] bf16, scale 1/sqrt(128)."""
    import pyc_amd
    B, H, S, D = 8, 32, 2048, 128
    gens = [torch.Generator(device="cuda").manual_seed(s) for s in (3, 4, 5)]
    Q, K, V = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for g in gens)
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    launch = lambda: pyc_amd.attention("hip_attention_bf16", Q, K, V, O, True, scale)  # noqa: E731
    ms_step, ms_kernel, _ = time_launches(torch, launch, args.steps, args.warmup, args.settle_ms)
    flops = 2.0 * B * H * S * S * D  # causal FA convention (half of 4*B*H*S^2*D)
    res = {
        "value": flops / (ms_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": {"workload": "attention_causal_bf16_8x32x2048x128", "flop_convention": "2*B*H*S^2*D"},
        "roofline": {"bound": "mfma", "achieved": flops / (ms_kernel * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (ms_kernel * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic("attention_cfg3"), "kernel_ms": ms_kernel},
    }
    if not args.no_cpu:
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        threads = min(_host_cores(), 32, H)
        q, k, v = (t[0:1, 0:threads].float().cpu().numpy() for t in (Q, K, V))
        # the oracle's attention per (b,h) head, one head per thread (its C
        # loop runs without the GIL)
        t0 = time.perf_counter()
        with ThreadPoolExecutor(threads) as ex:
            parts = list(ex.map(lambda h: oracle.attention_f32(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], True,
                                                               scale), range(threads)))
        dt = time.perf_counter() - t0
        ref = np.concatenate(parts, axis=1)
        res["cpu_baseline"] = {"value": flops * threads / (B * H) / dt / 1e12, "unit": "TFLOP/s", "cores": threads,
                               "kind": "port", "sample": f"{threads} of {B * H} (b,h) heads, oracle fp32 attention, "
                                                         f"one head per thread, {dt:.2f} s, extrapolated linearly"}
        t0 = time.perf_counter()
        oracle.attention_f32(q[:, 0:1], k[:, 0:1], v[:, 0:1], True, scale)
        dt1 = time.perf_counter() - t0
        res["cpu_baseline_1thread"] = {"value": flops / (B * H) / dt1 / 1e12, "unit": "TFLOP/s", "cores": 1,
                                       "kind": "port", "sample": f"1 of {B * H} heads on 1 thread, {dt1:.2f} s, "
                                                                 "extrapolated linearly"}
        got = O[0:1, 0:threads].float().cpu().numpy()
        res["parity_sample_max_rel_err"] = float(np.abs(got - ref).max() / np.abs(ref).max())
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    return res


def wl_conv(torch, args):
    """Config 4: NHWC conv 32x56x56x256 -> 256, 3x3 s1 p1, + bias + ReLU, bf16."""
    import pyc_amd
    N, H, W, C, K = 32, 56, 56, 256, 256
    gx, gw, gb = (torch.Generator(device="cuda").manual_seed(s) for s in (6, 7, 8))
    X = torch.rand((N, H, W, C), generator=gx, device="cuda").to(torch.bfloat16)
    Wd = (torch.randn((K, 3, 3, C), generator=gw, device="cuda") * np.sqrt(2.0 / 2304)).to(torch.bfloat16)
    Bv = 0.01 * torch.randn(K, generator=gb, device="cuda")
    Y = torch.empty((N, H, W, K), dtype=torch.bfloat16, device="cuda")
    launch = lambda: pyc_amd.conv2d("hip_conv2d_bf16", X, Wd, Y, pad=(1, 1), stride=(1, 1), bias=Bv, relu=True)  # noqa: E731
    ms_step, ms_kernel, _ = time_launches(torch, launch, args.steps, args.warmup, args.settle_ms)
    flops = 2.0 * N * H * W * K * C * 9
    res = {
        "value": flops / (ms_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": {"workload": "conv2d_nhwc_bf16_32x56x56x256_k256_3x3"},
        "roofline": {"bound": "mfma", "achieved": flops / (ms_kernel * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (ms_kernel * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic("conv_cfg4"), "kernel_ms": ms_kernel},
    }
    if not args.no_cpu:
        # The reference's CPU executor has no conv op, so the oracle's direct
        # convolution is the CPU implementation timed: one image per thread on
        # min(cores, 32) threads (its C loop runs without the GIL), and one
        # image on one thread (the reference executor's default thread count).
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        threads = min(_host_cores(), 32, N)
        x = X[0:threads].float().cpu().numpy()
        w = Wd.float().cpu().numpy()
        bias = Bv.cpu().numpy()
        t0 = time.perf_counter()
        with ThreadPoolExecutor(threads) as ex:
            parts = list(ex.map(lambda i: oracle.conv2d_nhwc_f32(x[i:i + 1], w, bias, (1, 1), (1, 1), True),
                                range(threads)))
        dt = time.perf_counter() - t0
        ref = np.concatenate(parts, axis=0)
        res["cpu_baseline"] = {"value": flops * threads / N / dt / 1e12, "unit": "TFLOP/s", "cores": threads,
                               "kind": "port", "sample": f"{threads} of {N} images, oracle direct conv (fp32), one "
                                                         f"image per thread, {dt:.2f} s, extrapolated linearly"}
        t0 = time.perf_counter()
        oracle.conv2d_nhwc_f32(x[0:1], w, bias, (1, 1), (1, 1), True)
        dt1 = time.perf_counter() - t0
        res["cpu_baseline_1thread"] = {"value": flops / N / dt1 / 1e12, "unit": "TFLOP/s", "cores": 1,
                                       "kind": "port", "sample": f"1 of {N} images on 1 thread, {dt1:.2f} s, "
                                                                 "extrapolated linearly"}
        got = Y[0:threads].float().cpu().numpy()
        res["parity_sample_max_rel_err"] = float(np.abs(got - ref).max() / np.abs(ref).max())
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    return res


def engine_device_kernel_ms(call, n):
    """Device time per run from the backend's HIP events: PYC_HIP_KERNEL_EVENTS=1
    makes cuda_kernel_ms the time between events around the run's kernels
    (without it, as in the reference, it is the host time of the enqueue, and
    the runs are ~4 us faster). Measured in a pass of its own after the timed
    runs, so the events do not slow the timed ones."""
    old = os.environ.get("PYC_HIP_KERNEL_EVENTS")
    os.environ["PYC_HIP_KERNEL_EVENTS"] = "1"
    try:
        ms = [call().cuda_kernel_ms for _ in range(n)]
    finally:
        if old is None:
            del os.environ["PYC_HIP_KERNEL_EVENTS"]
        else:
            os.environ["PYC_HIP_KERNEL_EVENTS"] = old
    return float(np.mean(ms))


def wl_engine_cfg1(torch, args):
    """BASELINE config 1 through the compiler-next run path itself:
    pyc_compile_model once, then pyc_run_model per step on the module
    in,in,in,matmul,add,relu,out with every tensor resident in device memory
    (bound to the captured graph in place, replayed). A step is one
    pyc_run_model call, timed by wall clock around the call (it returns after
    the device work finished); the engine's own pyc_run_stats fields are
    reported as the reference bench driver prints them. The same module with
    host buffers (H2D/D2H copies inside the call) is timed for the
    PCIe-inclusive rate."""
    import pyc_amd
    from pyc_amd import abi, engine
    os.environ["PYC_HIP_STRICT"] = "1"  # a CPU fallback is an error, not a measurement
    M = N = K = 1024
    r = np.random.default_rng(0)
    x = r.uniform(-1, 1, (M, K)).astype(np.float32)
    w = r.uniform(-1, 1, (K, N)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    F = abi.DTYPE_F32
    ops = [engine.op(abi.OP_INPUT, "x", (M, K)), engine.op(abi.OP_INPUT, "w", (K, N)),
           engine.op(abi.OP_INPUT, "bias", (N,)), engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1)),
           engine.op(abi.OP_ADD, "add0", (), (3, 2)), engine.op(abi.OP_RELU, "relu0", (), (4,)),
           engine.op(abi.OP_OUTPUT, "out0", (M, N), (5,))]
    model = engine.Model(ops, backend=abi.BACKEND_CUDA)
    if model.status != 0:
        raise RuntimeError(f"pyc_compile_model failed: {model.status}")
    X, W, Bv = (torch.from_numpy(t).cuda() for t in (x, w, b))
    Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ins = [engine.device_tensor(X, F), engine.device_tensor(W, F), engine.device_tensor(Bv, F)]
    outs = [engine.device_tensor(Y, F)]
    torch.cuda.synchronize()

    run = model.bind(ins, outs)  # the argument arrays built once, as a C caller keeps them

    def call():
        rc, st = run()
        if rc != 0:
            raise RuntimeError(f"pyc_run_model failed ({rc}): {st.execution_path.decode()}")
        return st

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        call()
    for _ in range(args.warmup):
        call()
    stats, wall = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        t1 = time.perf_counter()
        stats.append(call())
        wall.append((time.perf_counter() - t1) * 1e3)
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    eng = engine.run_stats_json(stats, wall, model)
    if not eng["execution_path"].startswith("hip_native"):
        raise RuntimeError(f"engine run did not take the native path: {eng['execution_path']}")
    kernel_ms = engine_device_kernel_ms(call, min(args.steps, 50))
    # the same module with host buffers: H2D/D2H copies inside each call
    yh = np.empty((M, N), dtype=np.float32)
    hins = [engine.host_tensor(a, F) for a in (x, w, b)]
    houts = [engine.host_tensor(yh, F)]
    hwall = []
    for i in range(min(args.steps, 50) + 5):
        t1 = time.perf_counter()
        rc, _ = model.run(hins, houts)
        if rc != 0:
            raise RuntimeError(f"pyc_run_model (host buffers) failed ({rc})")
        if i >= 5:
            hwall.append((time.perf_counter() - t1) * 1e3)
    if not np.array_equal(yh, Y.cpu().numpy()):
        raise RuntimeError("host-buffer and device-tensor runs differ")
    model.close()
    eng["host_buffers_latency_ms"] = latency_stats(hwall)
    flops = 2.0 * M * N * K + 2.0 * M * N
    res = {
        "value": flops / (ms_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "f32",
        "config": {"workload": "engine_pyc_run_model_gemm_f32_bias_relu_1024", "M": M, "N": N, "K": K,
                   "tensors": "device-resident", "module": "input,input,input,matmul,add,relu,output"},
        "roofline": {"bound": "mfma", "achieved": flops / (kernel_ms * 1e-3) / 1e12, "peak": PEAK_F32_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (kernel_ms * 1e-3) / 1e12 / PEAK_F32_TFLOPS,
                     "traffic": load_traffic("gemm_f32_cfg1"), "kernel_ms": kernel_ms},
        "latency_ms": eng.pop("latency_ms"),
        "engine": eng,
        # the reference's one published number for this metric: fp32 GEMM
        # 1024^3 via pyc_run_model, 28.3142 TFLOP/s (RTX 6000 Ada, cuBLASLt,
        # TF32 by default); this run is true fp32 plus the bias+ReLU epilogue
        "vs_baseline": flops / (ms_step * 1e-3) / 1e12 / 28.3142,
        "baseline_ref": "28.3142 TFLOP/s, fp32(TF32) 1024^3 via pyc_run_model, RTX 6000 Ada "
                        "(reference docs/reports/ada-box-technical-breakdown-2026-04-04.md:118)",
    }
    if not args.no_cpu:
        cpu, _ = cpu_baseline_gemm(x, w, flops, "full config-1 GEMM (bias+ReLU not timed)")
        res["cpu_baseline"] = cpu
        cpu1, _ = cpu_baseline_gemm(x[:256], w, flops, "256 of 1024 rows of the config-1 GEMM, 1 thread",
                                    threads=1)
        res["cpu_baseline_1thread"] = cpu1
    return res


def wl_engine_bf16(torch, args):
    """BASELINE config 2's GEMM as a module through pyc_run_model: in,in,
    matmul,out in bf16 with the weight stored [K,N] (the IR's matmul layout,
    the reference's default cutlass_gemm_tensorcore_bf16 symbol), every tensor
    resident in device memory, one pyc_run_model call per step timed by wall
    clock. The plan runs the persistent LDS-DMA kernel with B staged as
    k-rows."""
    from pyc_amd import abi, engine
    os.environ["PYC_HIP_STRICT"] = "1"
    M = N = K = 8192
    g1 = torch.Generator(device="cuda").manual_seed(1)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    X = (torch.randn((M, K), generator=g1, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    W = torch.randn((K, N), generator=g2, device="cuda").to(torch.bfloat16)
    Y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    BF = abi.DTYPE_BF16
    ops = [engine.op(abi.OP_INPUT, "x", (M, K), dtype=BF), engine.op(abi.OP_INPUT, "w", (K, N), dtype=BF),
           engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1), dtype=BF),
           engine.op(abi.OP_OUTPUT, "out0", (M, N), (2,), dtype=BF)]
    model = engine.Model(ops, backend=abi.BACKEND_CUDA)
    if model.status != 0:
        raise RuntimeError(f"pyc_compile_model failed: {model.status}")
    run = model.bind([engine.device_tensor(X, BF), engine.device_tensor(W, BF)], [engine.device_tensor(Y, BF)])
    torch.cuda.synchronize()

    def call():
        rc, st = run()
        if rc != 0:
            raise RuntimeError(f"pyc_run_model failed ({rc}): {st.execution_path.decode()}")
        return st

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        call()
    for _ in range(args.warmup):
        call()
    stats, wall = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        t1 = time.perf_counter()
        stats.append(call())
        wall.append((time.perf_counter() - t1) * 1e3)
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    eng = engine.run_stats_json(stats, wall, model)
    kernel_ms = engine_device_kernel_ms(call, min(args.steps, 20))
    model.close()
    if not eng["execution_path"].startswith("hip_native"):
        raise RuntimeError(f"engine run did not take the native path: {eng['execution_path']}")
    flops = 2.0 * M * N * K
    return {
        "value": flops / (ms_step * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": {"workload": "engine_pyc_run_model_gemm_bf16_kn_8192", "M": M, "N": N, "K": K,
                   "tensors": "device-resident", "weight_layout": "[K,N]", "module": "input,input,matmul,output"},
        "roofline": {"bound": "mfma", "achieved": flops / (kernel_ms * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / (kernel_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": load_traffic("gemm_bf16_nn_8192"), "kernel_ms": kernel_ms},
        "latency_ms": eng.pop("latency_ms"),
        "engine": eng,
        "vs_baseline": None,
    }


def wl_engine_chain(torch, args):
    """BASELINE config 5 as a module through pyc_compile_model / pyc_run_model:
    x -> 8 x (fp8 MATMUL up + ReLU, fp8 MATMUL down) -> y, with every weight,
    scale and activation resident in device memory. The backend plans the 16
    fp8 steps as one chain launch; a step of this workload is one
    pyc_run_model call (launch and wait), timed by wall clock, so the figure
    includes the engine's per-call host work on top of the kernel. The output
    is compared bit for bit with a direct pyc_hip_w8a16_chain_dispatch of the
    same chain."""
    import pyc_amd
    from pyc_amd import abi, engine
    os.environ["PYC_HIP_STRICT"] = "1"
    L, M, D, F = 8, 32, 4096, 11008
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((M, D), generator=g, device="cuda").to(torch.bfloat16)
    weights = []
    for l in range(L):
        gl = torch.Generator(device="cuda").manual_seed(10 + l)
        w_up = torch.randn((D, F), generator=gl, device="cuda") * np.sqrt(2.0 / D)
        w_dn = torch.randn((F, D), generator=gl, device="cuda") * np.sqrt(2.0 / F)
        for w in (w_up, w_dn):  # per-output-column scale, stored [N,K] e4m3fn
            s = (w.abs().amax(0) / 448.0).clamp_min(1e-30)
            q = (w / s).t().contiguous().to(torch.float8_e4m3fn).view(torch.uint8)
            weights += [q, s.float().contiguous()]
        del w_up, w_dn
    BF, F8, F32 = abi.DTYPE_BF16, abi.DTYPE_FP8_E4M3, abi.DTYPE_F32
    ops = [engine.op(abi.OP_INPUT, "x", (M, D), dtype=BF)]
    ins = [engine.device_tensor(x, BF)]
    cur = 0
    for l in range(L):
        qu, su, qd, sd = weights[4 * l:4 * l + 4]
        base = len(ops)
        ops += [engine.op(abi.OP_INPUT, f"wu{l}", (F, D), dtype=F8), engine.op(abi.OP_INPUT, f"su{l}", (F,)),
                engine.op(abi.OP_INPUT, f"wd{l}", (D, F), dtype=F8), engine.op(abi.OP_INPUT, f"sd{l}", (D,))]
        ins += [engine.device_tensor(qu, F8), engine.device_tensor(su, F32),
                engine.device_tensor(qd, F8), engine.device_tensor(sd, F32)]
        ops += [engine.op(abi.OP_MATMUL, f"up{l}", (), (cur, base, base + 1), dtype=BF),
                engine.op(abi.OP_RELU, f"relu{l}", (), (base + 4,), dtype=BF),
                engine.op(abi.OP_MATMUL, f"down{l}", (), (base + 5, base + 2, base + 3), dtype=BF)]
        cur = base + 6
    ops.append(engine.op(abi.OP_OUTPUT, "y", (M, D), (cur,), dtype=BF))
    y = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    model = engine.Model(ops, backend=abi.BACKEND_CUDA)
    if model.status != 0:
        raise RuntimeError(f"pyc_compile_model failed: {model.status}")
    run = model.bind(ins, [engine.device_tensor(y, BF)])
    torch.cuda.synchronize()

    def call():
        rc, st = run()
        if rc != 0:
            raise RuntimeError(f"pyc_run_model failed ({rc}): {st.execution_path.decode()}")
        return st

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        call()
    for _ in range(args.warmup):
        call()
    stats, wall = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        t1 = time.perf_counter()
        stats.append(call())
        wall.append((time.perf_counter() - t1) * 1e3)
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    eng = engine.run_stats_json(stats, wall, model)
    kernel_ms = engine_device_kernel_ms(call, min(args.steps, 20))
    model.close()
    if "hip_w8a16_chain_e4m3" not in eng["execution_path"]:
        raise RuntimeError(f"engine run did not take the chain launch: {eng['execution_path']}")
    # the same chain through the direct entry point: identical bits expected
    chain_layers = []
    for l in range(L):
        qu, su, qd, sd = weights[4 * l:4 * l + 4]
        chain_layers += [(qu, su, True), (qd, sd, False)]
    y_direct = torch.empty_like(y)
    pyc_amd.w8a16_chain(x, chain_layers, y_direct)
    torch.cuda.synchronize()
    same = bool(torch.equal(y.view(torch.int16), y_direct.view(torch.int16)))
    bytes_replay = L * (2 * D * F + 4 * F + 4 * D + M * D * 2 + 2 * M * F * 2 + M * D * 2)
    return {
        "value": bytes_replay / (ms_step * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms_step,
        "dtype": "fp8-e4m3 weights, bf16 activations",
        "config": {"workload": "engine_pyc_run_model_decode_chain_8x(32x4096x11008)", "tensors": "device-resident",
                   "module": "x, 8 x (matmul_fp8 + relu, matmul_fp8), y"},
        "roofline": {"bound": "hbm", "achieved": bytes_replay / (kernel_ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": bytes_replay / (kernel_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "traffic": load_traffic("decode_chain"), "kernel_ms": kernel_ms},
        "latency_ms": eng.pop("latency_ms"),
        "engine": eng,
        "matches_direct_chain": same,
        "vs_baseline": None,
    }


def _eltwise_line(name, config, nbytes, ms_step, ms_kernel):
    return {
        "value": nbytes / (ms_step * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms_step, "dtype": "bf16",
        "config": config,
        "roofline": {"bound": "hbm", "achieved": nbytes / (ms_kernel * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": nbytes / (ms_kernel * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "traffic": load_traffic(name), "kernel_ms": ms_kernel,
                     "algorithmic_bytes_per_launch": nbytes},
    }


def wl_gelu(torch, args):
    """GELU (exact erf form) over 64 Mi bf16 elements, read once and written
    once: 256 MiB of algorithmic HBM traffic per launch."""
    import pyc_amd
    n = 64 << 20
    x = torch.randn(n, generator=torch.Generator(device="cuda").manual_seed(13), device="cuda").to(torch.bfloat16)
    y = torch.empty_like(x)
    ms_step, ms_kernel, _ = time_launches(torch, lambda: pyc_amd.gelu(x, y), args.steps, args.warmup,
                                          args.settle_ms)
    return _eltwise_line("gelu", {"workload": "gelu_bf16_64Mi"}, 4.0 * n, ms_step, ms_kernel)


def wl_layernorm(torch, args):
    """LayerNorm over the last dimension of a [16384, 4096] bf16 tensor with
    bf16 gamma/beta: x read, y written once (gamma/beta 16 KiB): 256 MiB of
    algorithmic HBM traffic per launch."""
    import pyc_amd
    rows, D = 16384, 4096
    g = torch.Generator(device="cuda").manual_seed(14)
    x = (torch.randn((rows, D), generator=g, device="cuda") * 2 + 1).to(torch.bfloat16)
    gamma = torch.randn(D, generator=g, device="cuda").to(torch.bfloat16)
    beta = torch.randn(D, generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty_like(x)
    ms_step, ms_kernel, _ = time_launches(torch, lambda: pyc_amd.layernorm(x, y, gamma, beta), args.steps,
                                          args.warmup, args.settle_ms)
    return _eltwise_line("layernorm", {"workload": "layernorm_bf16_16384x4096_affine"},
                         4.0 * rows * D + 4.0 * D, ms_step, ms_kernel)


WORKLOADS = {"gemm_bf16": wl_gemm_bf16, "gemm_bf16_nn": wl_gemm_bf16_nn, "gemm_f32_cfg1": wl_gemm_f32_cfg1, "decode_chain": wl_decode_chain,
             "attention": wl_attention, "conv": wl_conv, "engine_cfg1": wl_engine_cfg1,
             "engine_bf16": wl_engine_bf16, "engine_chain": wl_engine_chain,
             "gelu": wl_gelu, "layernorm": wl_layernorm}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The GPU clock of an idle card ramps up over the first tens to hundreds
    # of milliseconds of load: the settle phase (--settle-ms) runs first, then
    # the warmup steps.
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="gemm_bf16", choices=sorted(WORKLOADS))
    ap.add_argument("--symbol", default=None, help="GEMM kernel symbol override")
    ap.add_argument("--cpu-rows", type=int, default=1024,
                    help="rows of the GEMM the CPU executor computes (about 10-30 CPU-seconds)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="default workload only: skip the nested config 1, 3, 4 and 5 blocks")
    ap.add_argument("--settle-ms", type=float, default=400.0,
                    help="untimed back-to-back launches before the warmup steps (clock ramp)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(no collectives); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import pyc_amd
    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    pyc_amd.lib()  # fail loudly if the HIP library is missing
    info = pyc_amd.device_info()
    log(f"device {info.gcn_arch.decode()} CUs={info.compute_units} sclk={info.clock_khz / 1e3:.0f} MHz")
    res = WORKLOADS[args.workload](torch, args)
    latency = res.get("latency_ms") or dict(_LAST_LATENCY)
    settled = dict(_LAST_SETTLE)
    nested = {}
    if args.workload == "gemm_bf16" and not args.no_extras:
        # The metric names bf16 GEMM and attention: config 3 rides along as a
        # nested block with its own roofline and CPU baseline, and config 1
        # through pyc_compile_model/pyc_run_model carries the reference bench
        # driver's engine fields (execution path, profile).
        att = wl_attention(torch, args)
        att["latency_ms"] = dict(_LAST_LATENCY)
        att["settle"] = dict(_LAST_SETTLE)
        nested["attention"] = att
        eng = wl_engine_cfg1(torch, args)
        nested["engine_cfg1"] = eng
        # configs 4 and 5, each with its own roofline, traffic and both CPU
        # legs: the conv (MFMA-bound) and the decode chain (HBM-bound, timed
        # as hipGraph replays of the whole 16-step chain)
        for name, fn in (("conv", wl_conv), ("decode_chain", wl_decode_chain)):
            blk = fn(torch, args)
            blk["latency_ms"] = dict(_LAST_LATENCY)
            blk["settle"] = dict(_LAST_SETTLE)
            nested[name] = blk
            torch.cuda.empty_cache()
    line = {
        "metric": METRIC, "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": res.get("vs_baseline"), "dtype": res["dtype"], "data": "synthetic",
        "config": res["config"], "roofline": res["roofline"],
    }
    line["latency_ms"] = latency
    line["settle"] = settled
    for k in ("cpu_baseline", "cpu_baseline_1thread", "parity_sample_max_rel_err", "speedup_vs_cpu", "baseline_ref",
              "engine", "matches_direct_chain"):
        if k in res:
            line[k] = res[k]
    line.update(nested)
    line["device"] = {"arch": info.gcn_arch.decode(), "cus": info.compute_units,
                      "sclk_mhz": info.clock_khz / 1e3}
    line["host"] = _host_info()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""The reference's own benchmark driver on this library.

oracle/Makefile.ref compiles the reference's pyc_compiler_next_bench.c from its
source, against this library's public headers, and links it to libpyc_amd.so
(reference benchmark/benchmarks/gpu/workloads/pyc_compiler_next_bench.c:605-1257;
its JSON fields at :1166-1249). These tests run that binary: it builds its
module through the public IR API, compiles it with pyc_compile_model and times
pyc_run_model, exactly as it does against the reference engine, so a user of
the reference's driver can point it at this backend unchanged. The driver does
not check results; parity of the same paths is covered by the engine tests."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "pyc_compiler_next_bench")

needs_driver = pytest.mark.skipif(not os.path.exists(DRIVER),
                                  reason="reference driver not built (needs the reference sources)")


def _run(args, **env):
    e = dict(os.environ)
    for k in list(e):
        if k.startswith(("PYC_", "BENCH_")):
            del e[k]
    e.update({k: str(v) for k, v in env.items()})
    r = subprocess.run([DRIVER, *map(str, args)], env=e, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@needs_driver
def test_reference_driver_cpu_mlp_and_gemm():
    """CPU backend: the driver's default MLP task and a bf16 GEMM task run on
    this library's CPU executor and report the reference's fields."""
    d = _run(["cpu", 64, 256, 5, 2])
    assert d["status"] == "ok" and d["execution_path"] == "cpu"
    assert d["latency_ms"]["mean"] > 0 and d["kernel_selection"]["count"] >= 1
    d = _run(["cpu", 64, 128, 3, 1], BENCH_TASK="gemm", BENCH_DTYPE="bfloat16", BENCH_M=48, BENCH_K=64,
             BENCH_N=80)
    assert d["status"] == "ok" and (d["m"], d["k"], d["n"]) == (48, 64, 80)
    assert d["throughput_tflops_per_sec"] > 0


@needs_driver
@pytest.mark.gpu
@pytest.mark.parametrize("dtype,mkn,symbol", [
    ("float32", (1024, 1024, 1024), "hip_gemm_f32"),   # config 1's GEMM shape
    ("bfloat16", (2048, 2048, 2048), "hip_gemm_bf16_nn"),
    ("float16", (512, 768, 256), "hip_gemm_f16"),
])
def test_reference_driver_cuda_gemm(dtype, mkn, symbol):
    """CUDA backend: the driver's GEMM task goes through pyc_cuda_dispatch to
    the HIP kernels (its defaults: static operands, no host output copy), on
    the native path every iteration."""
    m, k, n = mkn
    d = _run(["cuda", m, k, 20, 5], BENCH_TASK="gemm", BENCH_DTYPE=dtype, BENCH_M=m, BENCH_K=k, BENCH_N=n)
    assert d["status"] == "ok", d
    assert d["execution_path"].startswith("hip_native") and symbol in d["execution_path"], d["execution_path"]
    assert d["reliability"]["fallback_count"] == 0
    assert d["profile"]["cuda_kernel_ms"] > 0 and d["throughput_tflops_per_sec"] > 0


@needs_driver
@pytest.mark.gpu
def test_reference_driver_cuda_mlp():
    d = _run(["cuda", 64, 1024, 20, 5])
    assert d["status"] == "ok" and d["execution_path"].startswith("hip_native"), d

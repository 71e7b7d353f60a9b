"""The reference's own C11 engine driving this backend (the north star's
drop-in: the host engine stays, the CUDA backend is replaced).

pyc_amd/lib/libpyc_amd_backend.so is the backend alone: hip_backend.c,
hip_kernels.c, cpu_ops.c and the kernels, with no engine and no kernel
registry of its own. oracle/Makefile.ref links the reference's engine sources
(compiler_api.c, ir.c, pass_manager.c, runtime_allocator.c,
kernel_registry.c, runtime_control.c and the distributed stubs; not its
cuda_backend.c) to it, as a library (oracle/_ref/libpyc_ref_hip.so) and as the
reference's two CTest programs about the CUDA path. These CPU tests check the
link contract; tests/test_gpu_reference_engine.py runs the pairing on the
device."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from pyc_amd import abi
from tests import engine_util as eu

HIP_CTEST_DIR = os.path.join(eu.ROOT, "oracle", "_ref", "ctest_hip")
HIP_CTESTS = sorted(os.listdir(HIP_CTEST_DIR)) if os.path.isdir(HIP_CTEST_DIR) else []
REGISTRY_CALLS = {"pyc_kernel_collect", "pyc_kernel_promote_symbol", "pyc_kernel_promoted_symbol",
                  "pyc_kernel_register"}

needs_pairing = pytest.mark.skipif(not eu.ref_on_hip_available(),
                                   reason="needs oracle/Makefile.ref (the reference sources) and the backend library")


def _dyn_symbols(path, flag):
    out = subprocess.run(["nm", "-D", flag, path], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.split()}


@pytest.mark.skipif(not os.path.exists(eu.BACKEND_LIB), reason="backend library not built")
def test_backend_library_has_no_engine_or_registry():
    """The backend-only library defines the backend's C-ABI and leaves exactly
    the registry calls undefined, so they bind to the loading program's
    registry; no engine entry point is defined in it."""
    undef = {s for s in _dyn_symbols(eu.BACKEND_LIB, "--undefined-only") if s.startswith("pyc_")}
    assert undef == REGISTRY_CALLS, undef
    defined = _dyn_symbols(eu.BACKEND_LIB, "--defined-only")
    for s in ("pyc_cuda_dispatch", "pyc_cuda_dispatch_trace_init", "pyc_cuda_current_hardware_family",
              "pyc_cutlass_gemm_dispatch", "pyc_cutlass_conv2d_dispatch", "pyc_cutlass_attention_dispatch",
              "pyc_cutlass_kernel_count", "pyc_cutlass_registry_init"):
        assert s in defined, s
    for s in ("pyc_compile_model", "pyc_run_model", "pyc_kernel_register", "pyc_kernel_select",
              "pyc_ir_verify", "pyc_pass_pipeline_run"):
        assert s not in defined, s


@needs_pairing
def test_reference_registry_holds_the_hip_variants():
    """Loaded under the reference's engine, the backend registers its tile
    variants into the reference's registry (at load, as the reference's
    registry/init.cu:80-83 constructor does): pyc_kernel_collect of the
    reference engine returns them with their LDS figures, and the counts agree
    with the backend's own pyc_cutlass_kernel_count (which reads the same
    registry)."""
    L = eu.ref_on_hip()
    L.pyc_cutlass_kernel_count.argtypes = [C.c_char_p]
    L.pyc_cutlass_kernel_count.restype = C.c_int
    descs = (abi.KernelDesc * 64)()
    got = {}
    for key in ("matmul", "conv2d", "attention", "matmul_w8a16", "matmul_w8a16_chain"):
        n = L.pyc_kernel_collect(key.encode(), abi.BACKEND_CUDA, descs, 64)
        got[key] = {descs[i].symbol.decode(): descs[i] for i in range(n)}
        assert n == L.pyc_cutlass_kernel_count(key.encode()) > 0, key
    assert "hip_gemm_bf16_nt_256x256_lds" in got["matmul"]
    assert {"hip_conv2d_bf16", "hip_conv2d_bf16_persist", "hip_conv2d_bf16_tiled"} <= set(got["conv2d"])
    assert got["matmul"]["hip_gemm_bf16_nt_256x256_lds"].shared_mem_bytes == 163840
    assert got["matmul"]["hip_gemm_bf16_nt_256x256_lds"].preferred_hardware_family == abi.HW_CDNA4
    assert "hip_w8a16_chain_e4m3" in got["matmul_w8a16_chain"]


@needs_pairing
def test_reference_engine_cpu_run_through_backend(monkeypatch):
    """Without a device the reference's pyc_run_model reaches this backend's
    pyc_cuda_dispatch, which hands the module back to the reference's CPU
    executor with the reference's reason (here PYC_CUDA_FORCE_FALLBACK, so
    the result does not depend on a device being present); the outputs are
    the reference executor's, bit for bit."""
    monkeypatch.setenv("PYC_CUDA_FORCE_FALLBACK", "1")
    r = np.random.default_rng(3)
    x = r.uniform(-1, 1, (64, 48)).astype(np.float32)
    w = r.uniform(-1, 1, (48, 32)).astype(np.float32)
    ops = [eu.op(abi.OP_INPUT, "x", (64, 48)), eu.op(abi.OP_INPUT, "w", (48, 32)),
           eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1)), eu.op(abi.OP_OUTPUT, "out0", (64, 32), (2,))]
    got = eu.Model(eu.ref_on_hip(), ops, backend=abi.BACKEND_CUDA)
    assert got.status == 0
    st, (y,), s = got.run([x, w], [(64, 32)])
    got.close()
    assert st == 0 and s.execution_path.decode() == "cuda_forced_fallback" and s.fallback_count == 1
    refm = eu.Model(eu.ref(), ops, backend=abi.BACKEND_CPU)
    st, (yr,), _ = refm.run([x, w], [(64, 32)])
    refm.close()
    assert st == 0 and np.array_equal(y, yr)


@needs_pairing
@pytest.mark.skipif(not HIP_CTESTS, reason="reference CTest programs for the pairing not built")
@pytest.mark.parametrize("name", HIP_CTESTS)
def test_reference_cuda_ctest_on_reference_engine(name, tmp_path):
    """The reference's test_cuda_backend.c and test_production_cuda_contracts.c,
    linked to the reference's engine and this backend, pass (no device here:
    the dispatch contract's CPU paths)."""
    env = {k: v for k, v in os.environ.items() if not k.startswith("PYC_")}
    r = subprocess.run([os.path.join(HIP_CTEST_DIR, name)], cwd=tmp_path, env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, f"{name} exited {r.returncode}:\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
    assert "ok" in r.stdout.strip().splitlines()[-1], r.stdout[-500:]

"""GPU: the reference's own engine (its compiler_api.c pyc_compile_model /
pyc_run_model, ir.c, pass_manager.c, runtime_allocator.c, kernel_registry.c
and runtime_control.c, compiled from its sources) driving this backend through
pyc_cuda_dispatch, the drop-in the north star names: the C11 host engine
stays, hip_backend.c replaces cuda_backend.c. Host buffers in and out, as the
reference's callers pass them; every run must report the native HIP route and
match the oracle."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import oracle
from pyc_amd import abi
from tests import engine_util as eu
from tests.gpu_util import rel_max_err

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not eu.ref_on_hip_available(),
                                 reason="needs oracle/Makefile.ref's reference-engine build and the backend library")]

HIP_CTEST_DIR = os.path.join(eu.ROOT, "oracle", "_ref", "ctest_hip")
HIP_CTESTS = sorted(os.listdir(HIP_CTEST_DIR)) if os.path.isdir(HIP_CTEST_DIR) else []


@pytest.fixture(autouse=True)
def _env(monkeypatch, gpu):
    for k in list(os.environ):
        if k.startswith("PYC_"):
            monkeypatch.delenv(k, raising=False)


def _native(stats):
    path = stats.execution_path.decode()
    assert path.startswith("hip_native"), path
    assert stats.fallback_count == 0
    return path


def test_config1_on_reference_engine(monkeypatch):
    """Config 1 (in,in,in,matmul,add,relu,out F32 at 1024^3, U(-1,1) seed 0)
    through the reference's pyc_run_model: the backend lowers it to one fused
    GEMM+bias+ReLU kernel (graph capture, then replay); max|d|/max|ref| <= 1e-4
    against the oracle (the reference executor's GEMM order plus the row-bias
    and ReLU epilogue)."""
    monkeypatch.setenv("PYC_CUDA_ASSUME_STATIC_RHS", "1")
    r = np.random.default_rng(0)
    x = r.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    w = r.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b = r.uniform(-1, 1, 1024).astype(np.float32)
    ops = [eu.op(abi.OP_INPUT, "x", (1024, 1024)), eu.op(abi.OP_INPUT, "w", (1024, 1024)),
           eu.op(abi.OP_INPUT, "bias", (1024,)), eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1)),
           eu.op(abi.OP_ADD, "add0", (), (3, 2)), eu.op(abi.OP_RELU, "relu0", (), (4,)),
           eu.op(abi.OP_OUTPUT, "out0", (1024, 1024), (5,))]
    mdl = eu.Model(eu.ref_on_hip(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    ref = oracle.gemm_bias_relu_f32(x, w, b, relu=True, threads=8)
    paths = []
    for _ in range(3):
        st, (out,), s = mdl.run([x, w, b], [(1024, 1024)])
        assert st == 0
        paths.append(_native(s))
        assert rel_max_err(out, ref) <= 1e-4
    mdl.close()
    assert "graph_capture" in paths[0] and "graph_replay" in paths[-1], paths
    assert paths[0].endswith(":hip_gemm_f32_nn_64x64"), paths


def test_bf16_kn_8192_module_on_reference_engine(monkeypatch):
    """Config 2's GEMM as the reference engine's module in,in,matmul,out in
    bf16 with the weight [K,N] (the IR's matmul layout), 8192^3, host buffers:
    the persistent kernel's [K,N] form runs (hip_gemm_bf16_nn); 33 sampled
    rows (one in every 257) against the oracle (fp32 accumulation of the
    exactly decoded bf16 operands) within 2e-2 * max|ref|, and every column
    sum of the output against (1^T A) B in fp64."""
    monkeypatch.setenv("PYC_CUDA_ASSUME_STATIC_RHS", "1")
    monkeypatch.setenv("PYC_CUDA_ASSUME_STATIC_LHS", "1")
    M = N = K = 8192
    r = np.random.default_rng(1)
    a = oracle.f32_to_bf16((r.standard_normal((M, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32))
    b = oracle.f32_to_bf16((r.standard_normal((K, N), dtype=np.float32) / np.sqrt(K)).astype(np.float32))
    BF = abi.DTYPE_BF16
    ops = [eu.op(abi.OP_INPUT, "x", (M, K), dtype=BF), eu.op(abi.OP_INPUT, "w", (K, N), dtype=BF),
           eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1), dtype=BF),
           eu.op(abi.OP_OUTPUT, "out0", (M, N), (2,), dtype=BF)]
    mdl = eu.Model(eu.ref_on_hip(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    for _ in range(2):
        st, (y,), s = mdl.run([a, b], [(M, N)], in_dtypes=[BF, BF], out_dtypes=[BF], out_np_dtype=np.uint16)
        assert st == 0
        path = _native(s)
    mdl.close()
    assert path.endswith(":hip_gemm_bf16_nn"), path
    rows = np.unique(np.concatenate([np.arange(0, M, 257), [M - 1]]))
    ref_rows = oracle.gemm_bf16(a[rows], b, False, threads=16)
    assert rel_max_err(oracle.bf16_to_f32(y[rows]), ref_rows) <= 2e-2
    # size-independent property: the column sums of C equal (1^T A) B up to rounding
    af = oracle.bf16_to_f32(a).astype(np.float64)
    pred = af.sum(0) @ oracle.bf16_to_f32(b).astype(np.float64)
    del af
    colsum = oracle.bf16_to_f32(y).astype(np.float64).sum(0)
    assert np.abs(colsum - pred).max() <= 1e-2 * np.abs(pred).max()


def test_reference_registry_promotion_reaches_backend(monkeypatch):
    """A promotion made in the reference engine's registry is what the
    backend plans with: promote ada_gemm_k64_warp32_async_f32 for "matmul"
    through the reference's pyc_kernel_promote_symbol, enable the promoted
    GEMM (PYC_CUDA_ENABLE_PROMOTED_GEMM, reference cuda_backend.c:2643-2644),
    and the run reports that symbol; the result matches the oracle."""
    L = eu.ref_on_hip()
    monkeypatch.setenv("PYC_CUDA_ENABLE_PROMOTED_GEMM", "1")
    r = np.random.default_rng(5)
    x = r.uniform(-1, 1, (256, 128)).astype(np.float32)
    w = r.uniform(-1, 1, (128, 192)).astype(np.float32)
    ops = [eu.op(abi.OP_INPUT, "x", (256, 128)), eu.op(abi.OP_INPUT, "w", (128, 192)),
           eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1)), eu.op(abi.OP_OUTPUT, "out0", (256, 192), (2,))]
    try:
        assert L.pyc_kernel_promote_symbol(b"matmul", abi.BACKEND_CUDA, b"ada_gemm_k64_warp32_async_f32") == 0
        mdl = eu.Model(L, ops, backend=abi.BACKEND_CUDA)
        assert mdl.status == 0
        st, (y,), s = mdl.run([x, w], [(256, 192)])
        mdl.close()
    finally:
        L.pyc_kernel_promote_symbol(b"matmul", abi.BACKEND_CUDA, None)
    assert st == 0
    assert _native(s).endswith(":ada_gemm_k64_warp32_async_f32"), s.execution_path
    assert rel_max_err(y, oracle.matmul_f32(x, w)) <= 1e-4


@pytest.mark.skipif(not HIP_CTESTS, reason="reference CTest programs for the pairing not built")
@pytest.mark.parametrize("name", HIP_CTESTS)
def test_reference_cuda_ctest_on_reference_engine_with_device(name, tmp_path):
    """The reference's test_cuda_backend.c and test_production_cuda_contracts.c
    on its own engine and this backend, with the MI355X present."""
    env = {k: v for k, v in os.environ.items() if not k.startswith("PYC_")}
    r = subprocess.run([os.path.join(HIP_CTEST_DIR, name)], cwd=tmp_path, env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, f"{name} exited {r.returncode}:\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
    assert "ok" in r.stdout.strip().splitlines()[-1], r.stdout[-500:]

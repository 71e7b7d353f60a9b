"""GPU: measured autotune (the reference survey's third "next" item). With
enable_autotune, the first pyc_run_model on the GPU backend times every
registered tile variant of the module's GEMM at the live shape with HIP events
(pyc_hip_autotune_gemm), persists each as an `op|backend|symbol|best_ms` line
(the reference's format, compiler_api.c:2271-2340), promotes the fastest and
plans with it. Results are checked against the oracle, and the tuned plan
against the untuned one on the same inputs."""
import ctypes as C

import numpy as np
import pytest

import oracle
import pyc_amd
from pyc_amd import abi, engine
from tests.gpu_util import rel_max_err

pytestmark = pytest.mark.gpu

SYM = 64  # PYC_KERNEL_SYMBOL_MAX


def _autotune(L, dtype, M, N, K):
    f = L.pyc_hip_autotune_gemm
    f.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_size_t, C.POINTER(C.c_double), C.c_int]
    f.restype = C.c_int
    syms = C.create_string_buffer(SYM * 16)
    ms = (C.c_double * 16)()
    n = f(dtype, M, N, K, 3, syms, SYM, ms, 16)
    return n, [syms.raw[i * SYM:(i + 1) * SYM].split(b"\0")[0].decode() for i in range(max(n, 0))], list(ms[:max(n, 0)])


@pytest.mark.parametrize("dtype,expect", [(abi.DTYPE_BF16, {"hip_gemm_bf16_nn_256x256", "hip_gemm_bf16_nn_128x128",
                                                            "hip_gemm_bf16_nn", "cutlass_gemm_tensorcore_bf16"}),
                                          (abi.DTYPE_F32, {"hip_gemm_f32_nn_64x64"}),
                                          (abi.DTYPE_F16, {"hip_gemm_f16_nn"})])
def test_autotune_direct(gpu, dtype, expect):
    n, syms, ms = _autotune(pyc_amd.lib(), dtype, 1024, 768, 512)
    assert n == len(expect) and set(syms) == expect
    assert all(0.0 < t < 50.0 for t in ms), ms


def test_autotune_bad_arguments(gpu):
    L = pyc_amd.lib()
    n, _, _ = _autotune(L, abi.DTYPE_FP8_E4M3, 64, 64, 64)
    assert n == -1
    n, _, _ = _autotune(L, abi.DTYPE_BF16, 0, 64, 64)
    assert n == -1


@pytest.mark.parametrize("dt", [abi.DTYPE_BF16, abi.DTYPE_F32])
def test_run_model_autotune(gpu, dt, tmp_path, monkeypatch):
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    M, K, N = 1024, 512, 768
    r = np.random.default_rng(11)
    x = r.uniform(-1, 1, (M, K)).astype(np.float32)
    w = r.uniform(-1, 1, (K, N)).astype(np.float32)
    if dt == abi.DTYPE_BF16:
        xs, ws = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
        ref = oracle.gemm_bf16(xs, ws, False)
        y_dtype = np.uint16
    else:
        xs, ws, y_dtype = x, w, np.float32
        ref = oracle.matmul_f32(x, w)
    ops = [engine.op(abi.OP_INPUT, "x", (M, K), dtype=dt), engine.op(abi.OP_INPUT, "w", (K, N), dtype=dt),
           engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1), dtype=dt),
           engine.op(abi.OP_OUTPUT, "out0", (M, N), (2,), dtype=dt)]
    outs = {}
    for tune in (0, 1):
        db = tmp_path / f"tune{tune}.db"
        mdl = engine.Model(ops, backend=abi.BACKEND_CUDA, enable_autotune=tune, autotune_db_path=str(db).encode())
        assert mdl.status == 0
        y = np.zeros((M, N), y_dtype)
        for _ in range(2):  # capture, then replay
            rc, st = mdl.run([engine.host_tensor(xs, dt), engine.host_tensor(ws, dt)], [engine.host_tensor(y, dt)])
            assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
        path = st.execution_path.decode()
        mdl.close()
        outs[tune] = y.copy()
        if tune:
            assert st.autotune_saved == 1
            lines = [ln.split("|") for ln in db.read_text().splitlines() if ln.strip()]
            # bf16 has four [K,N] variants, fp32 one distinct kernel
            assert len(lines) >= (2 if dt == abi.DTYPE_BF16 else 1)
            assert all(ln[0] == "matmul_fused" and float(ln[3]) > 0 for ln in lines)
            best = min(lines, key=lambda ln: float(ln[3]))[2]
            assert path.endswith(":" + best), (path, lines)
    for tune, y in outs.items():
        got = oracle.bf16_to_f32(y) if dt == abi.DTYPE_BF16 else y
        assert rel_max_err(got, ref) <= (2e-2 if dt == abi.DTYPE_BF16 else 1e-5), tune


def test_run_model_autotune_every_gemm_shape(gpu, tmp_path, monkeypatch):
    """A module with two GEMMs of different shapes (x W1 -> ReLU -> W2, bf16):
    autotune times both shapes on the first run (each shape's variants are
    persisted and the shape is planned with its fastest), and the tuned
    module still matches the oracle."""
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    M, D, F = 512, 256, 768
    r = np.random.default_rng(12)
    x = oracle.f32_to_bf16(r.uniform(-1, 1, (M, D)).astype(np.float32))
    w1 = oracle.f32_to_bf16((r.uniform(-1, 1, (D, F)) / 16).astype(np.float32))
    w2 = oracle.f32_to_bf16((r.uniform(-1, 1, (F, D)) / 16).astype(np.float32))
    BF = abi.DTYPE_BF16
    ops = [engine.op(abi.OP_INPUT, "x", (M, D), dtype=BF), engine.op(abi.OP_INPUT, "w1", (D, F), dtype=BF),
           engine.op(abi.OP_INPUT, "w2", (F, D), dtype=BF), engine.op(abi.OP_MATMUL, "mm1", (), (0, 1), dtype=BF),
           engine.op(abi.OP_RELU, "relu1", (), (3,), dtype=BF), engine.op(abi.OP_MATMUL, "mm2", (), (4, 2), dtype=BF),
           engine.op(abi.OP_OUTPUT, "o", (M, D), (5,), dtype=BF)]
    db = tmp_path / "tune.db"
    mdl = engine.Model(ops, backend=abi.BACKEND_CUDA, enable_autotune=1, autotune_db_path=str(db).encode())
    assert mdl.status == 0
    y = np.zeros((M, D), np.uint16)
    for _ in range(2):
        rc, st = mdl.run([engine.host_tensor(a, BF) for a in (x, w1, w2)], [engine.host_tensor(y, BF)])
        assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
    mdl.close()
    assert st.autotune_saved == 1
    lines = [ln.split("|") for ln in db.read_text().splitlines() if ln.strip()]
    assert len(lines) >= 2 and all(float(ln[3]) > 0 for ln in lines)
    h = oracle.bf16_to_f32(oracle.f32_to_bf16(np.maximum(oracle.gemm_bf16(x, w1, False), 0)))
    ref = oracle.gemm_bf16(oracle.f32_to_bf16(h), w2, False)
    assert rel_max_err(oracle.bf16_to_f32(y), ref) <= 2e-2


def test_run_model_autotune_residual_add(gpu, tmp_path, monkeypatch):
    """Autotune with a matrix addend folded into the GEMM (bf16 4096x4096x256
    MATMUL + ADD [M,N]): the persistent [K,N] variant, which may win the
    timing at this shape, takes neither beta = 1 nor the addend, so the plan
    must fall back to a variant that does. The run stays native (strict
    mode) and matches the oracle's x @ w + addend."""
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    M, K, N = 4096, 256, 4096
    r = np.random.default_rng(13)
    x = oracle.f32_to_bf16(r.uniform(-1, 1, (M, K)).astype(np.float32))
    w = oracle.f32_to_bf16((r.uniform(-1, 1, (K, N)) / 8).astype(np.float32))
    add = oracle.f32_to_bf16(r.uniform(-1, 1, (M, N)).astype(np.float32))
    BF = abi.DTYPE_BF16
    ops = [engine.op(abi.OP_INPUT, "x", (M, K), dtype=BF), engine.op(abi.OP_INPUT, "w", (K, N), dtype=BF),
           engine.op(abi.OP_INPUT, "res", (M, N), dtype=BF), engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1), dtype=BF),
           engine.op(abi.OP_ADD, "add0", (), (3, 2), dtype=BF), engine.op(abi.OP_OUTPUT, "out0", (M, N), (4,), dtype=BF)]
    db = tmp_path / "tune.db"
    mdl = engine.Model(ops, backend=abi.BACKEND_CUDA, enable_autotune=1, autotune_db_path=str(db).encode())
    assert mdl.status == 0
    y = np.zeros((M, N), np.uint16)
    for _ in range(2):  # tune and capture, then replay
        rc, st = mdl.run([engine.host_tensor(a, BF) for a in (x, w, add)], [engine.host_tensor(y, BF)])
        assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
    path = st.execution_path.decode()
    mdl.close()
    assert st.autotune_saved == 1
    timed = {ln.split("|")[2] for ln in db.read_text().splitlines() if ln.strip()}
    assert "hip_gemm_bf16_nn_256x256" in timed, timed  # the persistent variant was a candidate
    assert not path.endswith(":hip_gemm_bf16_nn_256x256"), path
    ref = oracle.gemm_bf16(x, w, False, threads=8) + oracle.bf16_to_f32(add)
    assert rel_max_err(oracle.bf16_to_f32(y), ref) <= 2e-2

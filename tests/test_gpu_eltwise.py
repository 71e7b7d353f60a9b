"""GPU parity: GELU and LayerNorm (pyc_hip_gelu_dispatch /
pyc_hip_layernorm_dispatch), directly through the C-ABI and inside modules run
by pyc_compile_model / pyc_run_model. The reference reports these ops as graph
breaks and executes them nowhere, so the oracle is oracle.gelu_f64 /
oracle.layernorm_f64 (float64, pinned against torch in tests/test_oracle.py).
Tolerances: fp32 max|got-ref| <= 1e-5 * max|ref| (erff is accurate to a few
ulp); bf16/fp16 BASELINE's max|got-ref| <= 2e-2 * max|ref|, and elementwise at
most one rounding of the output type plus 1e-6 * max|ref|."""
import numpy as np
import pytest

import oracle
import pyc_amd
from pyc_amd import abi, engine
from tests.gpu_util import rel_max_err

pytestmark = pytest.mark.gpu

HALF_ULP = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11}


def _tdtype(torch, name):
    return {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[name]


def _check(got, ref, name):
    if name == "f32":
        assert rel_max_err(got, ref) <= 1e-5
    else:
        assert rel_max_err(got, ref) <= 2e-2
        bound = HALF_ULP[name] * np.abs(ref) + 1e-6 * np.abs(ref).max() + 1e-30
        assert np.all(np.abs(got.astype(np.float64) - ref) <= bound), float(np.max(np.abs(got - ref) - bound))


@pytest.mark.parametrize("name", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 1000003, 4 << 20])
def test_gelu(gpu, name, n):
    """Odd sizes (element tail after the 16-byte chunks), one element, and a
    4 Mi-element tensor; values spanning the erf's range including 0."""
    torch = gpu
    g = torch.Generator(device="cuda").manual_seed(n)
    x = (torch.randn(n, generator=g, device="cuda") * 4.0).to(_tdtype(torch, name))
    x[0] = 0.0
    y = torch.empty_like(x)
    pyc_amd.gelu(x, y)
    torch.cuda.synchronize()
    xin = x.float().cpu().numpy()  # the input as the kernel saw it (already rounded)
    _check(y.float().cpu().numpy(), oracle.gelu_f64(xin), name)
    assert y[0].item() == 0.0


def test_gelu_unaligned(gpu):
    """A view starting one element into its storage takes the element path."""
    torch = gpu
    base = torch.randn(4097, device="cuda")
    x = base[1:]
    y = torch.empty(4097, device="cuda")[1:]
    pyc_amd.gelu(x, y)
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), oracle.gelu_f64(x.cpu().numpy()), "f32")


@pytest.mark.parametrize("name", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,D,affine,eps", [(257, 1000, False, 1e-5), (64, 4096, True, 1e-5),
                                               (3, 768, True, 1e-3), (1, 8, True, 1e-5), (130, 5, False, 0.0),
                                               (33, 8192, True, 1e-5), (20, 6144, False, 1e-5)])
def test_layernorm(gpu, name, rows, D, affine, eps):
    """Rows of mean far from 0 (two-pass variance), D not a multiple of the
    16-byte chunk (element path), with and without gamma/beta, several eps;
    D = 4096, 6144 and 8192 reach the register-resident kernel's 8- and
    16-chunk forms (bf16: 8, 12 and 16 chunks per lane)."""
    torch = gpu
    t = _tdtype(torch, name)
    g = torch.Generator(device="cuda").manual_seed(rows * D)
    x = (torch.randn((rows, D), generator=g, device="cuda") * 3.0 + 5.0).to(t)
    gamma = torch.randn(D, generator=g, device="cuda").to(t) if affine else None
    beta = torch.randn(D, generator=g, device="cuda").to(t) if affine else None
    y = torch.empty_like(x)
    pyc_amd.layernorm(x, y, gamma, beta, eps)
    torch.cuda.synchronize()
    ref = oracle.layernorm_f64(x.float().cpu().numpy(), None if gamma is None else gamma.float().cpu().numpy(),
                               None if beta is None else beta.float().cpu().numpy(), eps)
    got = y.float().cpu().numpy()
    if name == "f32":
        assert rel_max_err(got, ref) <= 1e-5
    else:
        _check(got, ref, name)


def test_bad_arguments(gpu):
    torch = gpu
    L = pyc_amd.lib()
    x = torch.zeros(16, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert L.pyc_hip_gelu_dispatch(b"hip_layernorm_f32", 16, x.data_ptr(), x.data_ptr(), st) == -1
    assert L.pyc_hip_gelu_dispatch(b"no_such_symbol", 16, x.data_ptr(), x.data_ptr(), st) == -1
    assert L.pyc_hip_layernorm_dispatch(b"hip_layernorm_f32", 4, 0, 1e-5, x.data_ptr(), None, None,
                                        x.data_ptr(), st) == -1
    assert L.pyc_hip_layernorm_dispatch(b"hip_layernorm_f32", 4, 4, -1.0, x.data_ptr(), None, None,
                                        x.data_ptr(), st) == -1
    assert L.pyc_hip_gelu_dispatch(b"hip_gelu_f32", 0, None, None, st) == 0


# ------------------------------------------------------------------ through pyc_run_model


@pytest.fixture
def strict(monkeypatch):
    for k in ("PYC_CUDA_SIMULATE_AVAILABLE", "PYC_CUDA_DISABLE", "PYC_CUDA_FORCE_FALLBACK", "PYC_CUDA_FORCE_ERROR",
              "PYC_CUDA_SKIP_HOST_OUTPUT_COPY", "PYC_CUDA_ASSUME_STATIC_LHS", "PYC_CUDA_ASSUME_STATIC_RHS"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("PYC_HIP_STRICT", "1")


def test_run_model_matmul_gelu_f32(gpu, strict):
    """in,in,matmul,gelu,out with host buffers: the GEMM and the GELU both run
    natively (a graph break in the reference stays on the device here)."""
    M, K, N = 96, 128, 80
    r = np.random.default_rng(5)
    x, w = r.uniform(-1, 1, (M, K)).astype(np.float32), r.uniform(-1, 1, (K, N)).astype(np.float32)
    ops = [engine.op(abi.OP_INPUT, "x", (M, K)), engine.op(abi.OP_INPUT, "w", (K, N)),
           engine.op(abi.OP_MATMUL, "matmul0", (), (0, 1)), engine.op(abi.OP_GELU, "gelu0", (), (2,)),
           engine.op(abi.OP_OUTPUT, "out0", (M, N), (3,))]
    mdl = engine.Model(ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    y = np.zeros((M, N), np.float32)
    for _ in range(2):  # capture, then replay
        rc, st = mdl.run([engine.host_tensor(x, abi.DTYPE_F32), engine.host_tensor(w, abi.DTYPE_F32)],
                         [engine.host_tensor(y, abi.DTYPE_F32)])
        assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
    mdl.close()
    ref = oracle.gelu_f64(oracle.matmul_f32(x, w))
    assert rel_max_err(y, ref) <= 1e-4


def test_run_model_layernorm_affine_device(gpu, strict):
    """in(x),in(gamma),in(beta),layernorm@eps1e-6,out on device tensors (bf16),
    and the same module with fp32 host buffers."""
    torch = gpu
    rows, D = 48, 1024
    r = np.random.default_rng(6)
    x = (r.standard_normal((rows, D)) * 2 + 1).astype(np.float32)
    gm, bt = r.standard_normal(D).astype(np.float32), r.standard_normal(D).astype(np.float32)
    for dt, tdt in ((abi.DTYPE_BF16, torch.bfloat16), (abi.DTYPE_F32, torch.float32)):
        ops = [engine.op(abi.OP_INPUT, "x", (rows, D), dtype=dt), engine.op(abi.OP_INPUT, "gamma", (D,), dtype=dt),
               engine.op(abi.OP_INPUT, "beta", (D,), dtype=dt),
               engine.op(abi.OP_LAYERNORM, "ln0@eps1e-6", (), (0, 1, 2), dtype=dt),
               engine.op(abi.OP_OUTPUT, "out0", (rows, D), (3,), dtype=dt)]
        mdl = engine.Model(ops, backend=abi.BACKEND_CUDA)
        assert mdl.status == 0
        if dt == abi.DTYPE_BF16:
            X, G, B = (torch.from_numpy(a).cuda().to(tdt) for a in (x, gm, bt))
            Y = torch.empty_like(X)
            rc, st = mdl.run([engine.device_tensor(t, dt) for t in (X, G, B)], [engine.device_tensor(Y, dt)])
            got = Y.float().cpu().numpy()
            ref = oracle.layernorm_f64(X.float().cpu().numpy(), G.float().cpu().numpy(), B.float().cpu().numpy(), 1e-6)
            tol = 2e-2
        else:
            y = np.zeros((rows, D), np.float32)
            rc, st = mdl.run([engine.host_tensor(a, dt) for a in (x, gm, bt)], [engine.host_tensor(y, dt)])
            got, ref, tol = y, oracle.layernorm_f64(x, gm, bt, 1e-6), 1e-5
        mdl.close()
        assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
        assert rel_max_err(got, ref) <= tol

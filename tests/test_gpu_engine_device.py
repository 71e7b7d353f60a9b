"""GPU: pyc_run_model with tensors that live in device memory (the device-
resident tensors of the reference survey's first "next" item). The backend
binds such tensors to the plan directly (no staging, no host copies) and
includes their addresses in the graph signature; host and device tensors may
be mixed. Every run here is checked bit for bit against the same module run
with host buffers (the same kernels on the same values) and, directly,
against the oracle: fp32 within 1e-4 and bf16 / fp8-weight within 2e-2 of
max|ref| (max|got - ref| / max|ref|)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from pyc_amd import abi
from tests import engine_util as eu
from tests.gpu_util import rel_max_err

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _strict(monkeypatch, gpu):
    for k in ("PYC_CUDA_SIMULATE_AVAILABLE", "PYC_CUDA_DISABLE", "PYC_CUDA_FORCE_FALLBACK", "PYC_CUDA_FORCE_ERROR",
              "PYC_CUDA_SKIP_HOST_OUTPUT_COPY", "PYC_CUDA_ASSUME_STATIC_LHS", "PYC_CUDA_ASSUME_STATIC_RHS"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("PYC_HIP_STRICT", "1")


def _dt(t, dtype):
    """pyc_tensor describing a torch device tensor."""
    x = abi.Tensor()
    x.data = t.data_ptr()
    x.size_bytes = t.numel() * t.element_size()
    x.dtype = dtype
    x.shape = abi.make_shape(tuple(t.shape))
    return x


def _ht(a, dtype):
    return eu.tensor(a, dtype)


def _run(mdl, ins, outs):
    I = (abi.Tensor * len(ins))(*ins)
    O = (abi.Tensor * len(outs))(*outs)
    st = abi.RunStats()
    rc = mdl.L.pyc_run_model(mdl.h, I, len(ins), O, len(outs), C.byref(st))
    return rc, st


def _gemm_module(M, K, N, dtype=abi.DTYPE_F32, bias_dtype=None):
    bias_dtype = dtype if bias_dtype is None else bias_dtype
    ops = [eu.op(abi.OP_INPUT, "x", (M, K), dtype=dtype), eu.op(abi.OP_INPUT, "w", (K, N), dtype=dtype),
           eu.op(abi.OP_INPUT, "bias", (N,), dtype=bias_dtype), eu.op(abi.OP_MATMUL, "matmul0", (), (0, 1), dtype=dtype),
           eu.op(abi.OP_ADD, "add0", (), (3, 2), dtype=dtype), eu.op(abi.OP_RELU, "relu0", (), (4,), dtype=dtype),
           eu.op(abi.OP_OUTPUT, "out0", (M, N), (5,), dtype=dtype)]
    return eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)


def test_device_tensors_f32_gemm_bias_relu(gpu):
    """Config 1's module shape (smaller): every tensor on the device; equal to
    the host-buffer run; no copy time; a direct launch (one kernel)."""
    torch = gpu
    M, K, N = 512, 384, 256
    r = np.random.default_rng(0)
    x, w = (r.uniform(-1, 1, s).astype(np.float32) for s in ((M, K), (K, N)))
    b = r.uniform(-1, 1, N).astype(np.float32)
    mdl = _gemm_module(M, K, N)
    assert mdl.status == 0
    st, (host_out,), s = mdl.run([x, w, b], [(M, N)])
    assert st == 0 and s.execution_path.decode().startswith("hip_native")
    oref = oracle.gemm_bias_relu_f32(x, w, b, relu=True, threads=8)
    X, W, Bv = (torch.from_numpy(t).cuda() for t in (x, w, b))
    Y = torch.full((M, N), float("nan"), device="cuda")
    torch.cuda.synchronize()
    paths = []
    for _ in range(2):
        rc, s = _run(mdl, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _dt(Bv, abi.DTYPE_F32)],
                     [_dt(Y, abi.DTYPE_F32)])
        assert rc == 0, s.execution_path
        paths.append(s.execution_path.decode())
        assert np.array_equal(Y.cpu().numpy(), host_out)
        assert rel_max_err(Y.cpu().numpy(), oref) <= 1e-4
        assert s.cuda_copy_in_ms < 0.5 and s.cuda_copy_out_ms < 0.5
    mdl.close()
    # one kernel and no copies: launched directly, no graph of one node
    assert all(p.startswith("hip_native:") for p in paths), paths


@pytest.mark.parametrize("M,K,N", [(1024, 1024, 1024), (200, 136, 72)])
def test_device_tensors_back_to_back_runs_read_at_once(gpu, M, K, N):
    """Runs with device tensors return on a completion word: at 1024^3 the
    fp32 GEMM stores it itself once every workgroup's C is complete (its last
    waves may still be exiting); at 200x136x72, off the LDS-DMA kernel's tile
    multiples, a one-lane kernel stores it behind the GEMM. Each run's output is
    read by a torch kernel on the default stream as soon as the call returns,
    with no synchronization between, and every run's inputs differ from the
    previous one's (written in place on the default stream before the call),
    so a stale or partial output fails the bit-for-bit check against the
    host-buffer run of the same inputs. 12 runs exercise the counter's re-arm."""
    torch = gpu
    r = np.random.default_rng(7)
    mdl = _gemm_module(M, K, N)
    assert mdl.status == 0
    cases = []
    for _ in range(3):
        x, w = (r.uniform(-1, 1, sh).astype(np.float32) for sh in ((M, K), (K, N)))
        b = r.uniform(-1, 1, N).astype(np.float32)
        st, (ref,), _ = mdl.run([x, w, b], [(M, N)])
        assert st == 0
        cases.append((torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda(), ref.copy()))
    assert rel_max_err(cases[0][3], oracle.gemm_bias_relu_f32(*(t.cpu().numpy() for t in cases[0][:3]), relu=True,
                                                               threads=8)) <= 1e-4
    X, W, Bv = (torch.empty_like(t) for t in cases[0][:3])
    Y = torch.full((M, N), float("nan"), device="cuda")
    got = []
    torch.cuda.synchronize()
    for i in range(12):
        x, w, b, _ = cases[i % 3]
        X.copy_(x)
        W.copy_(w)
        Bv.copy_(b)
        rc, s = _run(mdl, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _dt(Bv, abi.DTYPE_F32)],
                     [_dt(Y, abi.DTYPE_F32)])
        assert rc == 0, s.execution_path
        assert s.execution_path.decode().startswith("hip_native:"), s.execution_path
        got.append(Y.clone())
    torch.cuda.synchronize()
    for i, g in enumerate(got):
        assert np.array_equal(g.cpu().numpy(), cases[i % 3][3]), f"run {i}"
    mdl.close()


@pytest.mark.parametrize("M,K,N", [(512, 512, 512), (200, 128, 72), (2048, 2048, 2048)])
def test_device_tensors_back_to_back_runs_bf16(gpu, M, K, N):
    """The bf16 form of the test above (these GEMMs end on the one-lane
    kernel's completion word): 512^3, a ragged 200x128x72 and 2048^3. Each
    run's output is read on the default stream as soon as the call returns;
    bit for bit against the host-buffer run of the same inputs, and the first
    case within 2e-2 of max|ref| of the oracle."""
    torch = gpu
    r = np.random.default_rng(11)
    mdl = _gemm_module(M, K, N, dtype=abi.DTYPE_BF16)
    assert mdl.status == 0
    cases = []
    for _ in range(3):
        a = oracle.f32_to_bf16((r.standard_normal((M, K)) / 16).astype(np.float32))
        w = oracle.f32_to_bf16(r.standard_normal((K, N)).astype(np.float32))
        b = oracle.f32_to_bf16(r.standard_normal(N).astype(np.float32))
        st, (ref,), s = mdl.run([a, w, b], [(M, N)], in_dtypes=[abi.DTYPE_BF16] * 3, out_dtypes=[abi.DTYPE_BF16],
                                out_np_dtype=np.uint16)
        assert st == 0, s.execution_path
        cases.append(([torch.from_numpy(t.view(np.int16)).cuda() for t in (a, w, b)], ref.copy(), (a, w, b)))
    a, w, b = cases[0][2]
    oref = np.maximum(oracle.gemm_bf16(a, w, False, threads=8) + oracle.bf16_to_f32(b)[None, :], 0.0)
    assert rel_max_err(oracle.bf16_to_f32(cases[0][1]), oref) <= 2e-2
    X, W, Bv = (torch.empty_like(t) for t in cases[0][0])
    Y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    got = []
    torch.cuda.synchronize()
    for i in range(12):
        x, w_, b_ = cases[i % 3][0]
        X.copy_(x)
        W.copy_(w_)
        Bv.copy_(b_)
        rc, s = _run(mdl, [_dt(X, abi.DTYPE_BF16), _dt(W, abi.DTYPE_BF16), _dt(Bv, abi.DTYPE_BF16)],
                     [_dt(Y, abi.DTYPE_BF16)])
        assert rc == 0, s.execution_path
        assert s.execution_path.decode().startswith("hip_native:"), s.execution_path
        got.append(Y.clone())
    torch.cuda.synchronize()
    for i, g in enumerate(got):
        assert np.array_equal(g.cpu().numpy().view(np.uint16), cases[i % 3][1]), f"run {i}"
    mdl.close()


def test_device_runs_alternate_completion_paths(gpu):
    """Two models called in turn, 16 times each: an fp32 1024^3 GEMM, whose
    kernel stores the run's completion word itself, and a bf16 512^3 GEMM,
    which ends on the one-lane kernel. Both share the backend's sequence
    number and counters; each output is read on the default stream as soon as
    its call returns and must equal its host-buffer run bit for bit."""
    torch = gpu
    r = np.random.default_rng(5)
    f32 = _gemm_module(1024, 1024, 1024)
    b16 = _gemm_module(512, 512, 512, dtype=abi.DTYPE_BF16)
    assert f32.status == 0 and b16.status == 0
    x, w = (r.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(2))
    b = r.uniform(-1, 1, 1024).astype(np.float32)
    st, (ref32,), _ = f32.run([x, w, b], [(1024, 1024)])
    assert st == 0
    a16 = oracle.f32_to_bf16((r.standard_normal((512, 512)) / 16).astype(np.float32))
    w16 = oracle.f32_to_bf16(r.standard_normal((512, 512)).astype(np.float32))
    b16v = oracle.f32_to_bf16(r.standard_normal(512).astype(np.float32))
    st, (ref16,), _ = b16.run([a16, w16, b16v], [(512, 512)], in_dtypes=[abi.DTYPE_BF16] * 3,
                              out_dtypes=[abi.DTYPE_BF16], out_np_dtype=np.uint16)
    assert st == 0
    X, W, Bv = (torch.from_numpy(t).cuda() for t in (x, w, b))
    A16, W16, B16 = (torch.from_numpy(t.view(np.int16)).cuda() for t in (a16, w16, b16v))
    Y32 = torch.full((1024, 1024), float("nan"), device="cuda")
    Y16 = torch.zeros((512, 512), dtype=torch.int16, device="cuda")
    got32, got16 = [], []
    torch.cuda.synchronize()
    for _ in range(16):
        Y32.fill_(float("nan"))
        rc, s = _run(f32, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _dt(Bv, abi.DTYPE_F32)],
                     [_dt(Y32, abi.DTYPE_F32)])
        assert rc == 0, s.execution_path
        got32.append(Y32.clone())
        Y16.zero_()
        rc, s = _run(b16, [_dt(A16, abi.DTYPE_BF16), _dt(W16, abi.DTYPE_BF16), _dt(B16, abi.DTYPE_BF16)],
                     [_dt(Y16, abi.DTYPE_BF16)])
        assert rc == 0, s.execution_path
        got16.append(Y16.clone())
    torch.cuda.synchronize()
    for i in range(16):
        assert np.array_equal(got32[i].cpu().numpy(), ref32), f"fp32 run {i}"
        assert np.array_equal(got16[i].cpu().numpy().view(np.uint16), ref16), f"bf16 run {i}"
    assert rel_max_err(ref32, oracle.gemm_bias_relu_f32(x, w, b, relu=True, threads=8)) <= 1e-4
    f32.close()
    b16.close()


def test_device_tensors_rebind_and_mixed(gpu):
    """New device addresses capture a new graph (a graph bakes in the addresses
    it was captured with); host and device tensors in one call; a host run
    after device runs."""
    torch = gpu
    M, K, N = 256, 128, 192
    r = np.random.default_rng(1)
    mdl = _gemm_module(M, K, N)
    cases = []
    for seed in range(3):
        x, w = (r.uniform(-1, 1, s).astype(np.float32) for s in ((M, K), (K, N)))
        b = r.uniform(-1, 1, N).astype(np.float32)
        st, (ref,), _ = mdl.run([x, w, b], [(M, N)])
        assert st == 0
        cases.append((x, w, b, ref.copy()))
    outs = [torch.empty((M, N), device="cuda") for _ in range(2)]
    seen = set()
    for i, (x, w, b, ref) in enumerate(cases):
        X, W = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
        Y = outs[i % 2]
        torch.cuda.synchronize()
        # x on the device, w on the device, bias from host memory, output on the device
        rc, s = _run(mdl, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _ht(b, abi.DTYPE_F32)], [_dt(Y, abi.DTYPE_F32)])
        assert rc == 0, s.execution_path
        # a graph bakes in device addresses: new ones are captured, addresses
        # the allocator handed out again replay the graph kept for them
        key = (X.data_ptr(), W.data_ptr(), Y.data_ptr())
        assert ("graph_replay" if key in seen else "graph_capture") in s.execution_path.decode(), (key, seen)
        seen.add(key)
        assert np.array_equal(Y.cpu().numpy(), ref), f"case {i}"
        assert rel_max_err(Y.cpu().numpy(), oracle.gemm_bias_relu_f32(x, w, b, relu=True, threads=8)) <= 1e-4
        # host output from the same device inputs
        host_y = np.zeros((M, N), np.float32)
        rc, s = _run(mdl, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _ht(b, abi.DTYPE_F32)],
                     [_ht(host_y, abi.DTYPE_F32)])
        assert rc == 0 and np.array_equal(host_y, ref), f"case {i} host output"
    x, w, b, ref = cases[0]
    st, (out,), _ = mdl.run([x, w, b], [(M, N)])
    assert st == 0 and np.array_equal(out, ref)
    mdl.close()


def test_device_tensors_bf16_half_bias(gpu):
    """A bf16 GEMM whose bias is a bf16 device vector: the backend reads it back
    for its fp32 copy (the host path converts it in host memory)."""
    torch = gpu
    M, K, N = 256, 512, 384
    r = np.random.default_rng(2)
    a = oracle.f32_to_bf16((r.standard_normal((M, K)) / 16).astype(np.float32))
    w = oracle.f32_to_bf16(r.standard_normal((K, N)).astype(np.float32))
    b = oracle.f32_to_bf16(r.standard_normal(N).astype(np.float32))
    mdl = _gemm_module(M, K, N, dtype=abi.DTYPE_BF16)
    assert mdl.status == 0
    st, (ref,), s = mdl.run([a, w, b], [(M, N)], in_dtypes=[abi.DTYPE_BF16] * 3, out_dtypes=[abi.DTYPE_BF16],
                            out_np_dtype=np.uint16)
    assert st == 0, s.execution_path
    A, Wd, Bd = (torch.from_numpy(t.view(np.int16)).cuda() for t in (a, w, b))
    Y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    rc, s = _run(mdl, [_dt(A, abi.DTYPE_BF16), _dt(Wd, abi.DTYPE_BF16), _dt(Bd, abi.DTYPE_BF16)],
                 [_dt(Y, abi.DTYPE_BF16)])
    mdl.close()
    assert rc == 0, s.execution_path
    got = Y.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    # oracle: fp32 GEMM of the decoded operands, + bias, ReLU
    oref = np.maximum(oracle.gemm_bf16(a, w, False, threads=8) + oracle.bf16_to_f32(b)[None, :], 0.0)
    assert rel_max_err(oracle.bf16_to_f32(got), oref) <= 2e-2


def test_device_tensors_decode_chain(gpu):
    """The fp8 decode-chain module (one chain launch) with all weights, scales,
    activations and the output on the device."""
    torch = gpu
    M, D, F = 32, 256, 512
    r = np.random.default_rng(3)
    x = oracle.f32_to_bf16(r.standard_normal((M, D)).astype(np.float32))
    ops, ins, dts = [eu.op(abi.OP_INPUT, "x", (M, D), dtype=abi.DTYPE_BF16)], [x], [abi.DTYPE_BF16]
    cur = 0
    for l in range(2):
        wu, su = oracle.quantize_e4m3_per_col((r.standard_normal((D, F)) * np.sqrt(2 / D)).astype(np.float32))
        wd, sd = oracle.quantize_e4m3_per_col((r.standard_normal((F, D)) * np.sqrt(2 / F)).astype(np.float32))
        base = len(ops)
        ops += [eu.op(abi.OP_INPUT, f"wu{l}", (F, D), dtype=abi.DTYPE_FP8_E4M3), eu.op(abi.OP_INPUT, f"su{l}", (F,)),
                eu.op(abi.OP_INPUT, f"wd{l}", (D, F), dtype=abi.DTYPE_FP8_E4M3), eu.op(abi.OP_INPUT, f"sd{l}", (D,))]
        ins += [wu, su, wd, sd]
        dts += [abi.DTYPE_FP8_E4M3, abi.DTYPE_F32, abi.DTYPE_FP8_E4M3, abi.DTYPE_F32]
        ops += [eu.op(abi.OP_MATMUL, f"up{l}", (), (cur, base, base + 1), dtype=abi.DTYPE_BF16),
                eu.op(abi.OP_RELU, f"relu{l}", (), (base + 4,), dtype=abi.DTYPE_BF16),
                eu.op(abi.OP_MATMUL, f"down{l}", (), (base + 5, base + 2, base + 3), dtype=abi.DTYPE_BF16)]
        cur = base + 6
    ops.append(eu.op(abi.OP_OUTPUT, "y", (M, D), (cur,), dtype=abi.DTYPE_BF16))
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    st, (ref,), s = mdl.run(ins, [(M, D)], in_dtypes=dts, out_dtypes=[abi.DTYPE_BF16], out_np_dtype=np.uint16)
    assert st == 0 and "hip_w8a16_chain_e4m3" in s.execution_path.decode()
    dev = [torch.from_numpy(np.ascontiguousarray(a).view(np.uint8)).cuda() for a in ins]
    Y = torch.zeros((M, D), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    tens = []
    for t, a, d in zip(dev, ins, dts):
        x_ = _dt(t, d)
        x_.shape = abi.make_shape(a.shape)
        tens.append(x_)
    rc, s = _run(mdl, tens, [_dt(Y, abi.DTYPE_BF16)])
    mdl.close()
    assert rc == 0, s.execution_path
    assert "hip_w8a16_chain_e4m3" in s.execution_path.decode()
    got = Y.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    # oracle: the fp8-weight layers one after another (bf16 between layers)
    h = x
    for l in range(2):
        wu, su, wd, sd = ins[1 + 4 * l: 5 + 4 * l]
        h = oracle.w8a16_layer(oracle.w8a16_layer(h, wu, su, True), wd, sd, False)
    assert rel_max_err(oracle.bf16_to_f32(got), oracle.bf16_to_f32(h)) <= 2e-2


def test_device_tensors_never_reach_cpu_executor(gpu, monkeypatch):
    """A forced CPU fallback with device tensors is an error (the CPU executor
    reads host memory), not a run of the CPU executor on device addresses."""
    torch = gpu
    monkeypatch.delenv("PYC_HIP_STRICT", raising=False)
    monkeypatch.setenv("PYC_CUDA_FORCE_FALLBACK", "1")
    M, K, N = 64, 64, 64
    mdl = _gemm_module(M, K, N)
    X, W = torch.rand((M, K), device="cuda"), torch.rand((K, N), device="cuda")
    Bv, Y = torch.rand(N, device="cuda"), torch.empty((M, N), device="cuda")
    torch.cuda.synchronize()
    rc, s = _run(mdl, [_dt(X, abi.DTYPE_F32), _dt(W, abi.DTYPE_F32), _dt(Bv, abi.DTYPE_F32)], [_dt(Y, abi.DTYPE_F32)])
    assert rc == abi.STATUS_RUNTIME_FAILED, rc
    assert "device_tensors_no_cpu_fallback" in s.execution_path.decode(), s.execution_path
    # the same module with host buffers still falls back as the reference does
    x = np.ones((M, K), np.float32)
    st, (out,), s = mdl.run([x, np.ones((K, N), np.float32), np.zeros(N, np.float32)], [(M, N)])
    mdl.close()
    assert st == 0 and s.fallback_count >= 1
    assert np.allclose(out, K)

"""GPU: the dispatch contract around the native path of pyc_run_model.

- The native run and the CPU-executor run of the same module agree (configs
  3-5's module shapes at reduced sizes): the fallback the reference takes on
  any native failure (cuda_backend.c:2883-2908) now exists for conv,
  attention and the fp8-weight chain, and gives the same answer.
- A decode-chain wait that times out is a native failure (workspace release
  plus cuda_native_failed_fallback, or an error for strict mode / device
  tensors), not a silent OK. The timeout word is set from the host
  (pyc_hip_w8a16_chain_error_raise); no kernel has to wait out for it.
- Chains whose hidden width the chain kernel cannot take run per layer.
- A promoted unit-epilogue GEMM symbol is not planned for a matrix addend.
- Device tensors produced on another stream are read only after that
  stream's work, also without graph replay.
- The hardware family of the MI355X is CDNA4 (reference
  cuda_backend.c:235-301 maps the device to a family)."""
import ctypes as C

import numpy as np
import pytest

import oracle
import pyc_amd
from pyc_amd import abi
from tests import engine_util as eu
from tests.gpu_util import rel_max_err

pytestmark = pytest.mark.gpu

BF = abi.DTYPE_BF16
FP8 = abi.DTYPE_FP8_E4M3


@pytest.fixture(autouse=True)
def _env(monkeypatch, gpu):
    for k in ("PYC_CUDA_SIMULATE_AVAILABLE", "PYC_CUDA_DISABLE", "PYC_CUDA_FORCE_FALLBACK", "PYC_CUDA_FORCE_ERROR",
              "PYC_CUDA_SKIP_HOST_OUTPUT_COPY", "PYC_CUDA_ASSUME_STATIC_LHS", "PYC_CUDA_ASSUME_STATIC_RHS",
              "PYC_HIP_STRICT", "PYC_CUDA_ENABLE_GRAPH_REPLAY", "PYC_CUDA_ENABLE_PROMOTED_GEMM"):
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("PYC_NUM_THREADS", "8")


def _lib():
    L = pyc_amd.lib()
    L.pyc_hip_w8a16_chain_error_raise.argtypes = []
    L.pyc_hip_w8a16_chain_error_raise.restype = C.c_int
    L.pyc_cuda_current_hardware_family.argtypes = []
    L.pyc_cuda_current_hardware_family.restype = C.c_int
    return L


def _fp8_chain(M, dims, seed):
    """Module x -> [fp8 matmul (+relu on even layers)]* -> y, its host inputs,
    and the oracle's output."""
    r = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(r.standard_normal((M, dims[0])).astype(np.float32))
    ops = [eu.op(abi.OP_INPUT, "x", (M, dims[0]), dtype=BF)]
    ins, dts, host = [x], [BF], []
    cur = 0
    for l, (K, N) in enumerate(zip(dims[:-1], dims[1:])):
        wq, sc = oracle.quantize_e4m3_per_col((r.standard_normal((K, N)) * np.sqrt(2 / K)).astype(np.float32))
        host.append((wq, sc, l % 2 == 0))
        base = len(ops)
        ops += [eu.op(abi.OP_INPUT, f"w{l}", (N, K), dtype=FP8), eu.op(abi.OP_INPUT, f"s{l}", (N,)),
                eu.op(abi.OP_MATMUL, f"mm{l}", (), (cur, base, base + 1), dtype=BF)]
        ins += [wq, sc]
        dts += [FP8, abi.DTYPE_F32]
        cur = base + 2
        if l % 2 == 0:
            ops.append(eu.op(abi.OP_RELU, f"relu{l}", (), (cur,), dtype=BF))
            cur += 1
    ops.append(eu.op(abi.OP_OUTPUT, "y", (M, dims[-1]), (cur,), dtype=BF))
    ref = x
    for wq, sc, relu in host:
        ref = oracle.w8a16_layer(ref, wq, sc, relu)
    return ops, ins, dts, (M, dims[-1]), ref


def _attention(seed):
    B, H, S, D = 1, 2, 200, 128
    r = np.random.default_rng(seed)
    qkv = [oracle.f32_to_bf16(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3)]
    ops = [eu.op(abi.OP_INPUT, n, (B, H, S, D), dtype=BF) for n in "qkv"]
    ops += [eu.op(abi.OP_ATTENTION, "attn_causal", (), (0, 1, 2), dtype=BF),
            eu.op(abi.OP_OUTPUT, "o", (B, H, S, D), (3,), dtype=BF)]
    ref = oracle.attention_f32(*(oracle.bf16_to_f32(t) for t in qkv), True, 1.0 / np.sqrt(D))
    return ops, qkv, [BF] * 3, (B, H, S, D), ref


def _conv(seed):
    N, H, W, C, K = 2, 14, 14, 64, 128
    r = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(r.uniform(0, 1, (N, H, W, C)).astype(np.float32))
    w = oracle.f32_to_bf16((r.standard_normal((K, 3, 3, C)) * np.sqrt(2 / (9 * C))).astype(np.float32))
    b = (0.01 * r.standard_normal(K)).astype(np.float32)
    ops = [eu.op(abi.OP_INPUT, "x", (N, H, W, C), dtype=BF), eu.op(abi.OP_INPUT, "w", (K, 3, 3, C), dtype=BF),
           eu.op(abi.OP_INPUT, "b", (K,)), eu.op(abi.OP_CONV2D, "conv@s1x1p1x1", (), (0, 1), dtype=BF),
           eu.op(abi.OP_ADD, "add", (), (3, 2), dtype=BF), eu.op(abi.OP_RELU, "relu", (), (4,), dtype=BF),
           eu.op(abi.OP_OUTPUT, "y", (N, H, W, K), (5,), dtype=BF)]
    ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(x), oracle.bf16_to_f32(w), b, (1, 1), (1, 1), True)
    return ops, [x, w, b], [BF, BF, abi.DTYPE_F32], (N, H, W, K), ref


def _run(ops, ins, dts, oshape):
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    st, (out,), s = mdl.run(ins, [oshape], in_dtypes=dts, out_dtypes=[BF], out_np_dtype=np.uint16)
    log = eu.log_fields(mdl.log())
    mdl.close()
    return st, oracle.bf16_to_f32(out), s, log


@pytest.mark.parametrize("case", ["attention", "conv", "fp8_chain"])
def test_native_and_cpu_fallback_agree(monkeypatch, case):
    if case == "attention":
        ops, ins, dts, oshape, ref = _attention(1)
    elif case == "conv":
        ops, ins, dts, oshape, ref = _conv(2)
    else:
        ops, ins, dts, oshape, ref = _fp8_chain(16, [512, 1024, 512, 1024, 512], 3)
    st, native, s, _ = _run(ops, ins, dts, oshape)
    assert st == 0 and s.execution_path.decode().startswith("hip_native") and s.fallback_count == 0
    monkeypatch.setenv("PYC_CUDA_FORCE_FALLBACK", "1")
    st, cpu, s, log = _run(ops, ins, dts, oshape)
    assert st == 0 and s.fallback_count == 1 and log["cuda_reason"] == "cuda_forced_fallback"
    for got in (native, cpu):
        assert rel_max_err(got, oracle.bf16_to_f32(ref) if ref.dtype == np.uint16 else ref) <= 2e-2
    assert rel_max_err(native, cpu) <= 2e-2


def test_chain_timeout_is_a_native_failure(monkeypatch):
    """The chain's timeout word set before a run: the run reports the native
    failure and falls back to the CPU executor (host tensors), fails under
    PYC_HIP_STRICT, fails with the reason for device tensors; the word is
    cleared, so the next run is native again."""
    torch = pytest.importorskip("torch")
    L = _lib()
    ops, ins, dts, oshape, ref = _fp8_chain(8, [256, 512, 256], 4)
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0

    def run():
        st, (out,), s = mdl.run(ins, [oshape], in_dtypes=dts, out_dtypes=[BF], out_np_dtype=np.uint16)
        return st, out, s, eu.log_fields(mdl.log())

    st, out, s, _ = run()
    assert st == 0 and "hip_w8a16_chain_e4m3" in s.execution_path.decode()
    assert np.array_equal(out, ref) or rel_max_err(oracle.bf16_to_f32(out), oracle.bf16_to_f32(ref)) <= 2e-2

    assert L.pyc_hip_w8a16_chain_error_raise() == 0
    st, out, s, log = run()
    assert st == 0 and log["cuda_fallback"] == "1" and log["cuda_reason"] == "cuda_native_failed_fallback", log
    assert np.array_equal(out, ref)  # the CPU executor's result is the oracle's, bit for bit
    st, out, s, log = run()
    assert st == 0 and log["cuda_fallback"] == "0" and s.execution_path.decode().startswith("hip_native"), log

    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    assert L.pyc_hip_w8a16_chain_error_raise() == 0
    st, _, s, _ = run()
    assert st == abi.STATUS_RUNTIME_FAILED
    monkeypatch.delenv("PYC_HIP_STRICT")

    # device tensors: no CPU fallback exists, the reason names the timeout
    dev = []
    for a, d in zip(ins, dts):
        t = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
        dev.append(t)
    Y = torch.zeros(oshape, dtype=torch.int16, device="cuda")
    I = (abi.Tensor * len(dev))(*[_dt(t, d) for t, d in zip(dev, dts)])
    O = (abi.Tensor * 1)(_dt(Y, BF))
    torch.cuda.synchronize()
    assert L.pyc_hip_w8a16_chain_error_raise() == 0
    stats = abi.RunStats()
    st = mdl.L.pyc_run_model(mdl.h, I, len(dev), O, 1, C.byref(stats))
    log = eu.log_fields(mdl.log())
    assert st == abi.STATUS_RUNTIME_FAILED
    assert "hip_chain_wait_timeout" in log["cuda_reason"] and "device_tensors_no_cpu_fallback" in log["cuda_reason"]
    stats = abi.RunStats()
    st = mdl.L.pyc_run_model(mdl.h, I, len(dev), O, 1, C.byref(stats))
    assert st == 0 and stats.execution_path.decode().startswith("hip_native")
    assert np.array_equal(Y.cpu().numpy().view(np.uint16), out)
    mdl.close()
    assert pyc_amd.w8a16_chain_error() == 0


def _dt(t, dtype):
    x = abi.Tensor()
    x.data = t.data_ptr()
    x.size_bytes = t.numel() * t.element_size()
    x.dtype = dtype
    x.shape = abi.make_shape(tuple(t.shape))
    return x


def test_chain_hidden_width_outside_chain_kernel_runs_per_layer(monkeypatch):
    """4096 -> 1088 -> 4096: 1088 % 128 != 0, so the chain kernel cannot take
    the down projection's K; both steps run on the per-layer kernel."""
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    ops, ins, dts, oshape, ref = _fp8_chain(8, [4096, 1088, 4096], 5)
    st, out, s, _ = _run(ops, ins, dts, oshape)
    path = s.execution_path.decode()
    assert st == 0 and path.startswith("hip_native") and "chain" not in path, path
    assert "hip_gemm_w8a16_e4m3" in path
    assert rel_max_err(out, oracle.bf16_to_f32(ref)) <= 2e-2


def test_promoted_unit_epilogue_symbol_not_used_for_matrix_add(monkeypatch):
    """ada_gemm_k64_warp32_async_f32 takes alpha = 1, beta = 0 only; promoted
    under PYC_CUDA_ENABLE_PROMOTED_GEMM, it must not be planned for a MATMUL
    whose ADD is a full matrix (beta = 1)."""
    M, K, N = 96, 64, 80
    r = np.random.default_rng(6)
    x, w, c = (r.uniform(-1, 1, s).astype(np.float32) for s in ((M, K), (K, N), (M, N)))
    ops = [eu.op(abi.OP_INPUT, "x", (M, K)), eu.op(abi.OP_INPUT, "w", (K, N)), eu.op(abi.OP_INPUT, "c", (M, N)),
           eu.op(abi.OP_MATMUL, "mm", (), (0, 1)), eu.op(abi.OP_ADD, "add", (), (3, 2)),
           eu.op(abi.OP_OUTPUT, "o", (M, N), (4,))]
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    monkeypatch.setenv("PYC_CUDA_ENABLE_PROMOTED_GEMM", "1")
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    L = mdl.L
    assert L.pyc_kernel_promote_symbol(b"matmul", abi.BACKEND_CUDA, b"ada_gemm_k64_warp32_async_f32") == 0
    try:
        st, (out,), s = mdl.run([x, w, c], [(M, N)])
    finally:
        L.pyc_kernel_promote_symbol(b"matmul", abi.BACKEND_CUDA, b"")
        mdl.close()
    assert st == 0 and s.execution_path.decode().startswith("hip_native"), s.execution_path
    ref = oracle.matmul_f32(x, w) + c
    assert rel_max_err(out, ref) <= 1e-4


def test_device_inputs_from_another_stream_without_graph(monkeypatch, gpu):
    """PYC_CUDA_ENABLE_GRAPH_REPLAY=0: inputs (and a bf16 bias the backend
    reads back to convert) are written by a copy queued on another
    non-blocking stream behind a long kernel chain and handed over to the
    default stream with wait_stream (no host wait); the run, ordered after the
    default stream, must see them."""
    torch = gpu
    monkeypatch.setenv("PYC_CUDA_ENABLE_GRAPH_REPLAY", "0")
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    M, K, N = 256, 512, 384
    ops = [eu.op(abi.OP_INPUT, "x", (M, K), dtype=BF), eu.op(abi.OP_INPUT, "w", (K, N), dtype=BF),
           eu.op(abi.OP_INPUT, "bias", (N,), dtype=BF), eu.op(abi.OP_MATMUL, "mm", (), (0, 1), dtype=BF),
           eu.op(abi.OP_ADD, "add", (), (3, 2), dtype=BF), eu.op(abi.OP_OUTPUT, "o", (M, N), (4,), dtype=BF)]
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CUDA)
    assert mdl.status == 0
    r = np.random.default_rng(7)
    x = oracle.f32_to_bf16(r.standard_normal((M, K)).astype(np.float32))
    w = oracle.f32_to_bf16((r.standard_normal((K, N)) / 16).astype(np.float32))
    b = oracle.f32_to_bf16(r.standard_normal(N).astype(np.float32))
    src = [torch.from_numpy(a.view(np.int16)).cuda() for a in (x, w, b)]
    dst = [torch.zeros_like(t) for t in src]
    Y = torch.zeros((M, N), dtype=torch.int16, device="cuda")
    big = torch.randn((4096, 4096), device="cuda")
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for _ in range(30):
            big = big @ big / 64.0  # ~4 ms of work ahead of the copies
        for d, s_ in zip(dst, src):
            d.copy_(s_)
    # the hand-over to the default stream, without a host wait: the run is
    # ordered after the default stream's work, which now includes the copies
    torch.cuda.current_stream().wait_stream(side)
    I = (abi.Tensor * 3)(*[_dt(t, BF) for t in dst])
    O = (abi.Tensor * 1)(_dt(Y, BF))
    stats = abi.RunStats()
    st = mdl.L.pyc_run_model(mdl.h, I, 3, O, 1, C.byref(stats))
    torch.cuda.synchronize()
    mdl.close()
    assert st == 0 and stats.execution_path.decode().startswith("hip_native"), stats.execution_path
    got = oracle.bf16_to_f32(Y.cpu().numpy().view(np.uint16))
    ref = oracle.gemm_bf16(x, w, False) + oracle.bf16_to_f32(b)[None, :]
    assert rel_max_err(got, ref) <= 2e-2


def test_hardware_family_is_cdna4(monkeypatch):
    monkeypatch.delenv("PYC_CUDA_FORCE_HARDWARE_FAMILY", raising=False)
    L = _lib()
    assert L.pyc_cuda_current_hardware_family() == abi.HW_CDNA4
    info = pyc_amd.device_info()
    assert info.gcn_arch.decode().startswith("gfx950")

"""GPU: the kernel registry describes the kernels the backend launches, and
conv2d's paths are registered variants that the measured autotune times.

The registry's shared_mem_bytes and estimated_occupancy feed every score
(the pressure penalty, the allocator-aware co-selection and the reuse bonus,
reference src/compiler/runtime/kernel_registry.c:58,73,120,161-172). Each
registered symbol's figures are the compiled-in figures of the kernel it
launches; here they are compared with what the loaded code object reports
(hipFuncGetAttributes: the static LDS; hipOccupancyMaxActiveBlocksPerMultiprocessor:
the resident workgroups per CU, so the waves per SIMD)."""
import ctypes as C

import numpy as np
import pytest

import oracle
import pyc_amd
from pyc_amd import abi, engine
from tests.gpu_util import dev_bits16, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu

OP_KEYS = ("matmul", "attention", "conv2d", "matmul_w8a16", "matmul_w8a16_chain", "gelu", "layernorm")


def _registered():
    L = pyc_amd.lib()
    descs = (abi.KernelDesc * 64)()
    out = []
    for key in OP_KEYS:
        n = L.pyc_kernel_collect(key.encode(), abi.BACKEND_CUDA, descs, 64)
        out += [abi.KernelDesc.from_buffer_copy(descs[i]) for i in range(n)]
    return out


def test_registry_lds_and_occupancy_match_the_code_object(gpu):
    descs = _registered()
    assert len(descs) >= 38
    for d in descs:
        sym = d.symbol.decode()
        r = pyc_amd.kernel_resources(sym)
        assert r.device == 1, sym
        assert d.shared_mem_bytes == r.lds_bytes == r.attr_lds_bytes, (sym, d.shared_mem_bytes, r.attr_lds_bytes)
        assert r.attr_max_threads >= r.threads, sym
        waves = r.attr_blocks_per_cu * (r.threads // 64) / 4
        assert r.attr_blocks_per_cu >= 1, sym
        assert r.waves_per_simd == waves, (sym, r.kernel, r.waves_per_simd, waves)
        assert abs(d.estimated_occupancy - waves / 8.0) < 1e-12, sym


def test_hot_kernels_resources(gpu):
    """The four largest LDS users, by name: the persistent GEMM and conv
    (160 KiB), attention (160 KiB) and the fp32 GEMM (128 KiB), one workgroup
    per CU each."""
    for sym, lds in (("hip_gemm_bf16_nt_256x256_lds", 163840), ("hip_attention_bf16", 163840),
                     ("hip_conv2d_bf16", 163840), ("hip_gemm_f32_nn_64x64", 131072)):
        r = pyc_amd.kernel_resources(sym)
        assert r.attr_lds_bytes == lds and r.attr_blocks_per_cu == 1, (sym, r.attr_lds_bytes, r.attr_blocks_per_cu)


def _conv_inputs(N, H, W, C, K, seed):
    r = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(r.uniform(0, 1, (N, H, W, C)).astype(np.float32))
    w = oracle.f32_to_bf16((r.standard_normal((K, 3, 3, C)) * np.sqrt(2.0 / (9 * C))).astype(np.float32))
    b = (0.01 * r.standard_normal(K)).astype(np.float32)
    return x, w, b


@pytest.mark.parametrize("sym", ["hip_conv2d_bf16", "hip_conv2d_bf16_persist", "hip_conv2d_bf16_tiled"])
def test_conv_paths_config4_against_oracle(gpu, sym):
    """Every registered conv2d path at config 4's shape (32x56x56x256 ->
    256, 3x3, pad 1, +bias +ReLU; 392 tiles of 256 x 256, so the persistent
    path runs two rounds and the automatic one a round plus the tail kernel)
    against the oracle's direct convolution on images 0 and 31."""
    torch = gpu
    N, H, W, C, K = 32, 56, 56, 256, 256
    x, w, b = _conv_inputs(N, H, W, C, K, 44)
    X, Wd = dev_bits16(torch, x), dev_bits16(torch, w)
    Bv = torch.from_numpy(b).cuda()
    Y = torch.empty((N, H, W, K), dtype=torch.bfloat16, device="cuda")
    pyc_amd.conv2d(sym, X, Wd, Y, pad=(1, 1), stride=(1, 1), bias=Bv, relu=True)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(host_bits16(Y))
    for n in (0, N - 1):
        ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(x[n:n + 1]), oracle.bf16_to_f32(w), b, (1, 1), (1, 1), True)
        assert rel_max_err(got[n:n + 1], ref) <= 2e-2, (sym, n)


def test_conv_autotune_direct(gpu):
    """pyc_hip_autotune_conv2d times the three bf16 paths at a live geometry."""
    res = pyc_amd.autotune_conv2d(abi.DTYPE_BF16, 8, 32, 32, 64, 256, 3, 3, iters=3)
    assert {s for s, _ in res} == {"hip_conv2d_bf16", "hip_conv2d_bf16_persist", "hip_conv2d_bf16_tiled"}
    assert all(0.0 < t < 50.0 for _, t in res), res
    L = pyc_amd.lib()
    names = C.create_string_buffer(64 * 8)
    ms = (C.c_double * 8)()
    assert L.pyc_hip_autotune_conv2d(abi.DTYPE_F32, 8, 32, 32, 64, 256, 3, 3, 1, 1, 1, 1, 3, names, 64, ms, 8) == -1


def test_run_model_conv_autotune(gpu, tmp_path, monkeypatch):
    """enable_autotune on a conv module (x, w, bias, conv, add, relu, out in
    bf16): the first run times every conv2d path at the module's geometry,
    persists each as a `conv2d|backend|symbol|ms` line, plans the conv with
    the fastest (the run's execution path names it) and the result matches
    the oracle."""
    monkeypatch.setenv("PYC_HIP_STRICT", "1")
    N, H, W, C, K = 8, 32, 32, 64, 256
    x, w, b = _conv_inputs(N, H, W, C, K, 45)
    BF, F = abi.DTYPE_BF16, abi.DTYPE_F32
    ops = [engine.op(abi.OP_INPUT, "x", (N, H, W, C), dtype=BF), engine.op(abi.OP_INPUT, "w", (K, 3, 3, C), dtype=BF),
           engine.op(abi.OP_INPUT, "bias", (K,), dtype=F), engine.op(abi.OP_CONV2D, "conv0@s1x1p1x1", (), (0, 1), dtype=BF),
           engine.op(abi.OP_ADD, "add0", (), (3, 2), dtype=BF), engine.op(abi.OP_RELU, "relu0", (), (4,), dtype=BF),
           engine.op(abi.OP_OUTPUT, "out0", (N, H, W, K), (5,), dtype=BF)]
    db = tmp_path / "tune.db"
    mdl = engine.Model(ops, backend=abi.BACKEND_CUDA, enable_autotune=1, autotune_db_path=str(db).encode())
    assert mdl.status == 0
    y = np.zeros((N, H, W, K), np.uint16)
    for _ in range(2):
        rc, st = mdl.run([engine.host_tensor(x, BF), engine.host_tensor(w, BF), engine.host_tensor(b, F)],
                         [engine.host_tensor(y, BF)])
        assert rc == 0 and st.execution_path.decode().startswith("hip_native"), st.execution_path
    mdl.close()
    assert st.autotune_saved == 1
    lines = [ln.split("|") for ln in db.read_text().splitlines() if ln.strip()]
    conv = [ln for ln in lines if ln[0] == "conv2d"]
    assert {ln[2] for ln in conv} == {"hip_conv2d_bf16", "hip_conv2d_bf16_persist", "hip_conv2d_bf16_tiled"}
    best = min(conv, key=lambda ln: float(ln[3]))[2]
    assert st.execution_path.decode().endswith(":" + best), (st.execution_path, conv)
    ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(x), oracle.bf16_to_f32(w), b, (1, 1), (1, 1), True)
    assert rel_max_err(oracle.bf16_to_f32(y), ref) <= 2e-2

"""GPU parity: weight-only fp8 (e4m3fn) decode GEMM against the CPU oracle.

Tolerance: max|got-ref| <= 2e-2 * max|ref|, and each bf16
output within two bf16 roundings of the oracle's bf16 output."""
import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, dev_f32, dev_u8, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu


def _layer(M, N, K, seed):
    r = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(r.standard_normal((M, K)).astype(np.float32))
    w = (r.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32)
    wq, scale = oracle.quantize_e4m3_per_col(w)
    return x, wq, scale


@pytest.mark.parametrize("M,N,K", [(32, 11008, 4096), (32, 4096, 11008), (1, 96, 64), (7, 40, 48),
                                   (17, 300, 1040)])
@pytest.mark.parametrize("relu", [False, True])
def test_w8a16_layer(gpu, M, N, K, relu):
    torch = gpu
    x, wq, scale = _layer(M, N, K, M + N + K)
    X, Wq, S = dev_bits16(torch, x), dev_u8(torch, wq), dev_f32(torch, scale)
    Y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pyc_amd.w8a16_gemm(X, Wq, S, Y, relu)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(host_bits16(Y))
    ref = oracle.bf16_to_f32(oracle.w8a16_layer(x, wq, scale, relu))
    assert rel_max_err(got, ref) <= 2e-2
    assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-3 * np.abs(ref).max())


def test_w8a16_rejects_bad_shapes(gpu):
    torch = gpu
    L = pyc_amd.lib()
    X = torch.zeros((33, 64), dtype=torch.bfloat16, device="cuda")
    Wq = torch.zeros((16, 64), dtype=torch.uint8, device="cuda")
    S = torch.ones(16, dtype=torch.float32, device="cuda")
    Y = torch.zeros((33, 16), dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.pyc_hip_w8a16_gemm_dispatch(b"hip_gemm_w8a16_e4m3", 33, 16, 64, X.data_ptr(),
                                         Wq.data_ptr(), S.data_ptr(), 0, Y.data_ptr(), s) == -1
    assert L.pyc_hip_w8a16_gemm_dispatch(b"hip_gemm_w8a16_e4m3", 4, 16, 60, X.data_ptr(),
                                         Wq.data_ptr(), S.data_ptr(), 0, Y.data_ptr(), s) == -1


@pytest.mark.parametrize("M,N,K", [(32, 1000, 4096), (32, 2048, 2048), (5, 64, 11008)])
def test_w8a16_split_k_repeat(gpu, M, N, K):
    """Shapes whose channel units are split over several workgroups: every
    unit is finished by its last contributor, which re-arms the unit's counter;
    two launches in a row with different inputs must both match."""
    torch = gpu
    _, wq, scale = _layer(M, N, K, N + K)
    Wq, S = dev_u8(torch, wq), dev_f32(torch, scale)
    Y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    for seed in (1, 2):
        x = oracle.f32_to_bf16(np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32))
        pyc_amd.w8a16_gemm(dev_bits16(torch, x), Wq, S, Y, True)
        torch.cuda.synchronize()
        got = oracle.bf16_to_f32(host_bits16(Y))
        ref = oracle.bf16_to_f32(oracle.w8a16_layer(x, wq, scale, True))
        assert rel_max_err(got, ref) <= 2e-2
        assert np.all(np.abs(got - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-3 * np.abs(ref).max())


def test_w8a16_chain_graph_replay(gpu):
    """Up -> ReLU -> down captured in one graph and replayed with new inputs
    and eager launches in between; each replay must equal the eager chain."""
    torch = gpu
    M, D, F = 32, 2048, 3072
    _, wu, su = _layer(M, F, D, 31)
    _, wd, sd = _layer(M, D, F, 32)
    Wu, Su, Wd, Sd = dev_u8(torch, wu), dev_f32(torch, su), dev_u8(torch, wd), dev_f32(torch, sd)
    X = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    H = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
    Yg = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    He = torch.empty_like(H)
    Ye = torch.empty_like(Yg)

    def chain(x, h, y, stream=None):
        pyc_amd.w8a16_gemm(x, Wu, Su, h, True, stream=stream)
        pyc_amd.w8a16_gemm(h, Wd, Sd, y, False, stream=stream)

    X.copy_(torch.randn((M, D), device="cuda").to(torch.bfloat16))
    chain(X, He, Ye)  # eager first: allocates the split-K workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        graph.capture_begin()
        chain(X, H, Yg, stream=s.cuda_stream)
        graph.capture_end()
    torch.cuda.synchronize()
    for rep in range(3):
        X.copy_(torch.randn((M, D), device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        chain(X, He, Ye)
        torch.cuda.synchronize()
        assert torch.equal(H, He), f"replay {rep}: hidden differs"
        assert torch.equal(Yg, Ye), f"replay {rep}: output differs"
    x = host_bits16(X)
    h_ref = oracle.w8a16_layer(x, wu, su, True)
    y_ref = oracle.bf16_to_f32(oracle.w8a16_layer(h_ref, wd, sd, False))
    got = oracle.bf16_to_f32(host_bits16(Yg))
    assert rel_max_err(got, y_ref) <= 2e-2

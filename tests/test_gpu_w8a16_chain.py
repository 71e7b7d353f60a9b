"""GPU parity: the whole fp8-weight decode chain in one launch
(pyc_hip_w8a16_chain_dispatch).

The chain kernel splits every step's items as the single-layer kernel does
but sums each item's two k halves in different waves, so its fp32 sums are
ordered differently: it is checked against the same layers run one launch at
a time (themselves checked against the CPU oracle in tests/test_gpu_w8a16.py)
and, for chains the oracle finishes quickly, against the oracle directly,
both to BASELINE's bar max|got-ref| <= 2e-2 * max|ref|. Repeated launches and
graph replays of one chain must agree bit for bit (the kernel is
deterministic)."""
import ctypes as C

import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, dev_f32, dev_u8, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu


def _weights(dims, seed):
    """Quantized weights of a chain dims[0] -> dims[1] -> ... (w stored [N,K])."""
    r = np.random.default_rng(seed)
    out = []
    for K, N in zip(dims[:-1], dims[1:]):
        w = (r.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32)
        out.append(oracle.quantize_e4m3_per_col(w))
    return out


def _dev_layers(torch, ws, relus):
    return [(dev_u8(torch, wq), dev_f32(torch, s), r) for (wq, s), r in zip(ws, relus)]


def _sequential(torch, x, layers):
    cur = x
    for wq, s, relu in layers:
        y = torch.empty((x.shape[0], wq.shape[0]), dtype=torch.bfloat16, device="cuda")
        pyc_amd.w8a16_gemm(cur, wq, s, y, relu)
        cur = y
    return cur


@pytest.mark.parametrize("M,dims,relus", [
    (32, [4096, 11008, 4096], [True, False]),
    (5, [256, 512, 384, 128], [True, False, True]),
    (1, [128, 64], [False]),
    (17, [2048, 3072, 2048, 3072, 2048], [True, False, True, False]),
])
def test_chain_matches_layers(gpu, M, dims, relus):
    torch = gpu
    ws = _weights(dims, M + len(dims))
    layers = _dev_layers(torch, ws, relus)
    x = oracle.f32_to_bf16(np.random.default_rng(M).standard_normal((M, dims[0])).astype(np.float32))
    X = dev_bits16(torch, x)
    Y = torch.empty((M, dims[-1]), dtype=torch.bfloat16, device="cuda")
    pyc_amd.w8a16_chain(X, layers, Y)
    ref_dev = _sequential(torch, X, layers)
    torch.cuda.synchronize()
    assert pyc_amd.w8a16_chain_error() == 0
    got = Y.float().cpu().numpy()
    assert rel_max_err(got, ref_dev.float().cpu().numpy()) <= 2e-2, "chain vs layer-by-layer launches"
    if dims[0] * dims[1] <= 2048 * 3072:
        cur = x
        for (wq, s), r in zip(ws, relus):
            cur = oracle.w8a16_layer(cur, wq, s, r)
        ref = oracle.bf16_to_f32(cur)
        assert rel_max_err(oracle.bf16_to_f32(host_bits16(Y)), ref) <= 2e-2


def test_chain_decode_config(gpu):
    """BASELINE config 5's shape (8 x [4096 -> 11008 -> ReLU -> 4096]) twice in
    a row with different inputs: the step counters re-arm between launches."""
    torch = gpu
    dims = [4096] + [11008, 4096] * 8
    relus = [True, False] * 8
    layers = _dev_layers(torch, _weights(dims, 5), relus)
    Y = torch.empty((32, 4096), dtype=torch.bfloat16, device="cuda")
    for seed in (1, 2):
        X = torch.randn((32, 4096), generator=torch.Generator(device="cuda").manual_seed(seed),
                        device="cuda").to(torch.bfloat16)
        pyc_amd.w8a16_chain(X, layers, Y)
        ref = _sequential(torch, X, layers)
        torch.cuda.synchronize()
        assert pyc_amd.w8a16_chain_error() == 0
        assert rel_max_err(Y.float().cpu().numpy(), ref.float().cpu().numpy()) <= 2e-2, f"input {seed}"
        Y2 = torch.empty_like(Y)
        pyc_amd.w8a16_chain(X, layers, Y2)
        torch.cuda.synchronize()
        assert torch.equal(Y, Y2), f"input {seed}: a second launch differs"


def test_chain_decode_config_vs_oracle(gpu):
    """BASELINE config 5 end to end against the CPU oracle: 8 x [x(32x4096)
    -> W_up(4096x11008, fp8) -> ReLU -> W_down(11008x4096, fp8)], x ~ N(0,1)
    seed 9, layer l's weights ~ N(0, sqrt(2/K)) from seed 10+l quantized per
    output channel (the bench's inputs), the whole chain in one launch. The
    oracle runs the 16 layers in fp32 with bf16 activations between them
    (threaded over output channels; the result does not depend on it).
    Tolerance: max|got-ref| <= 2e-2 * max|ref|."""
    import os
    torch = gpu
    L, M, D, F = 8, 32, 4096, 11008
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn((M, D), generator=g, device="cuda").to(torch.bfloat16)
    layers, host = [], []
    for l in range(L):
        gl = torch.Generator(device="cuda").manual_seed(10 + l)
        w_up = torch.randn((D, F), generator=gl, device="cuda") * np.sqrt(2.0 / D)
        w_dn = torch.randn((F, D), generator=gl, device="cuda") * np.sqrt(2.0 / F)
        for w, relu in ((w_up, True), (w_dn, False)):
            s = (w.abs().amax(0) / 448.0).clamp_min(1e-30)
            q = (w / s).t().contiguous().to(torch.float8_e4m3fn).view(torch.uint8)
            s = s.float().contiguous()
            layers.append((q, s, relu))
            host.append((q.cpu().numpy(), s.cpu().numpy(), relu))
        del w_up, w_dn
    y = torch.empty((M, D), dtype=torch.bfloat16, device="cuda")
    pyc_amd.w8a16_chain(x, layers, y)
    torch.cuda.synchronize()
    assert pyc_amd.w8a16_chain_error() == 0
    threads = min(16, len(os.sched_getaffinity(0)))
    cur = host_bits16(x)
    for wq, s, relu in host:
        cur = oracle.w8a16_layer(cur, wq, s, relu, threads)
    ref = oracle.bf16_to_f32(cur)
    got = oracle.bf16_to_f32(host_bits16(y))
    assert np.isfinite(got).all()
    assert rel_max_err(got, ref) <= 2e-2


def test_chain_graph_replay(gpu):
    """The chain launch captured in a graph and replayed with new inputs, with
    eager launches (of this and of another chain shape) in between: every
    replay must equal the eager result."""
    torch = gpu
    M = 32
    dims = [2048, 3072, 2048, 3072, 2048]
    relus = [True, False, True, False]
    layers = _dev_layers(torch, _weights(dims, 7), relus)
    other = _dev_layers(torch, _weights([512, 1024, 256], 8), [True, False])
    X = torch.empty((M, dims[0]), dtype=torch.bfloat16, device="cuda")
    Yg = torch.empty((M, dims[-1]), dtype=torch.bfloat16, device="cuda")
    Ye = torch.empty_like(Yg)
    pyc_amd.w8a16_chain_reserve(M, layers)
    pyc_amd.w8a16_chain_reserve(M, other)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        graph.capture_begin()
        pyc_amd.w8a16_chain(X, layers, Yg, stream=s.cuda_stream)
        graph.capture_end()
    torch.cuda.synchronize()
    Xo = torch.randn((M, 512), device="cuda").to(torch.bfloat16)
    Yo = torch.empty((M, 256), dtype=torch.bfloat16, device="cuda")
    for rep in range(3):
        X.copy_(torch.randn((M, dims[0]), device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        pyc_amd.w8a16_chain(X, layers, Ye)
        pyc_amd.w8a16_chain(Xo, other, Yo)
        torch.cuda.synchronize()
        assert torch.equal(Yg, Ye), f"replay {rep} differs from the eager chain"
    assert rel_max_err(Yo.float().cpu().numpy(), _sequential(torch, Xo, other).float().cpu().numpy()) <= 2e-2
    assert rel_max_err(Ye.float().cpu().numpy(), _sequential(torch, X, layers).float().cpu().numpy()) <= 2e-2
    assert pyc_amd.w8a16_chain_error() == 0


def test_chain_rejects_bad_shapes(gpu):
    torch = gpu
    L = pyc_amd.lib()
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((128, 256), dtype=torch.uint8, device="cuda")
    s = torch.ones(128, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream

    def call(symbol, M, Ns, Ks):
        n = len(Ns)
        wq = (C.c_void_p * n)(*([w.data_ptr()] * n))
        sc = (C.c_void_p * n)(*([s.data_ptr()] * n))
        N = (C.c_int * n)(*Ns)
        K = (C.c_int * n)(*Ks)
        r = (C.c_int * n)(*([0] * n))
        return L.pyc_hip_w8a16_chain_dispatch(symbol, M, n, x.data_ptr(), C.cast(wq, C.c_void_p),
                                              C.cast(sc, C.c_void_p), C.cast(N, C.c_void_p),
                                              C.cast(K, C.c_void_p), C.cast(r, C.c_void_p), y.data_ptr(), st)

    assert call(b"hip_w8a16_chain_e4m3", 4, [128], [256]) == 0
    assert call(b"hip_gemm_w8a16_e4m3", 4, [128], [256]) == -1  # wrong symbol
    assert call(b"hip_w8a16_chain_e4m3", 33, [128], [256]) == -1  # M > 32
    assert call(b"hip_w8a16_chain_e4m3", 4, [96], [256]) == -1  # N % 64
    assert call(b"hip_w8a16_chain_e4m3", 4, [128], [192]) == -1  # K % 128
    assert call(b"hip_w8a16_chain_e4m3", 4, [256, 128], [256, 128]) == -1  # K[1] != N[0]
    torch.cuda.synchronize()
    assert pyc_amd.w8a16_chain_error() == 0

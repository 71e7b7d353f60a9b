"""GPU: the allocation-free decode-chain entry point
(pyc_hip_w8a16_chain_dispatch_noalloc), called through the C-ABI.

It runs the same kernels as pyc_hip_w8a16_chain_dispatch with its workspace
in a static device array, so its output must equal that entry point's bit for
bit (the chain kernel is deterministic for a given shape): checked on two
calls in a row, the second with a smaller chain (the scratch keeps the first
call's contents), and on graph replays of a capture made without any reserve
call. A chain whose workspace exceeds the scratch is refused with -3 before
anything is launched."""
import ctypes as C

import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, dev_f32, dev_u8, rel_max_err

pytestmark = pytest.mark.gpu

SYM = b"hip_w8a16_chain_e4m3"


def _layers(torch, dims, seed):
    r = np.random.default_rng(seed)
    out = []
    for i, (K, N) in enumerate(zip(dims[:-1], dims[1:])):
        wq, s = oracle.quantize_e4m3_per_col((r.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32))
        out.append((dev_u8(torch, wq), dev_f32(torch, s), i % 2 == 0))
    return out


def _noalloc(torch, x, layers, y, stream=None):
    n = len(layers)
    wq = (C.c_void_p * n)(*[w.data_ptr() for w, _, _ in layers])
    sc = (C.c_void_p * n)(*[s.data_ptr() for _, s, _ in layers])
    N = (C.c_int * n)(*[int(w.shape[0]) for w, _, _ in layers])
    K = (C.c_int * n)(*[int(w.shape[1]) for w, _, _ in layers])
    relu = (C.c_int * n)(*[int(r) for _, _, r in layers])
    st = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    return pyc_amd.lib().pyc_hip_w8a16_chain_dispatch_noalloc(
        SYM, int(x.shape[0]), n, x.data_ptr(), C.cast(wq, C.c_void_p), C.cast(sc, C.c_void_p),
        C.cast(N, C.c_void_p), C.cast(K, C.c_void_p), C.cast(relu, C.c_void_p), y.data_ptr(), st)


def test_noalloc_matches_allocating_entry_point(gpu):
    torch = gpu
    cases = [(32, [4096] + [11008, 4096] * 8, 1),  # 63.6 MiB of the 64 MiB scratch
             (5, [256, 512, 384, 128], 2)]          # then a smaller chain
    for M, dims, seed in cases:
        layers = _layers(torch, dims, seed)
        x = torch.randn((M, dims[0]), generator=torch.Generator(device="cuda").manual_seed(seed),
                        device="cuda").to(torch.bfloat16)
        y_ref = torch.empty((M, dims[-1]), dtype=torch.bfloat16, device="cuda")
        y = torch.full_like(y_ref, float("nan"))
        pyc_amd.w8a16_chain(x, layers, y_ref)
        assert _noalloc(torch, x, layers, y) == 0
        torch.cuda.synchronize()
        assert pyc_amd.w8a16_chain_error() == 0
        assert torch.equal(y, y_ref), f"M={M} dims={dims[:3]}...: differs from pyc_hip_w8a16_chain_dispatch"
        if M == 5:
            cur = oracle.f32_to_bf16(x.float().cpu().numpy())
            for w, s, r in layers:
                cur = oracle.w8a16_layer(cur, w.cpu().numpy(), s.cpu().numpy(), r)
            assert rel_max_err(y.float().cpu().numpy(), oracle.bf16_to_f32(cur)) <= 2e-2


def test_noalloc_rejects_chain_larger_than_scratch(gpu):
    torch = gpu
    # 9 layers of config 5's shape need more than 64 MiB: refused, nothing launched
    w_up = torch.zeros((11008, 4096), dtype=torch.uint8, device="cuda")
    w_dn = torch.zeros((4096, 11008), dtype=torch.uint8, device="cuda")
    s_up = torch.ones(11008, device="cuda")
    s_dn = torch.ones(4096, device="cuda")
    layers = [(w_up, s_up, True), (w_dn, s_dn, False)] * 9
    x = torch.zeros((32, 4096), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros_like(x)
    assert _noalloc(torch, x, layers, y) == -3
    assert _noalloc(torch, x, layers[:16], y) == 0  # the config-5 length still fits
    bad = [(w_up[:, :100], s_up, True)]  # K % 128 != 0
    assert _noalloc(torch, x[:, :100].contiguous(), bad, y[:, :100].contiguous()) == -1
    torch.cuda.synchronize()
    assert pyc_amd.w8a16_chain_error() == 0


def test_noalloc_graph_capture_without_reserve(gpu):
    """Captured with no reserve call first (nothing to allocate), replayed with
    new inputs and eager launches of another shape in between: every replay
    equals the allocating entry point's eager result."""
    torch = gpu
    M, dims = 16, [2048, 3072, 2048, 3072, 2048]
    layers = _layers(torch, dims, 3)
    other = _layers(torch, [512, 1024, 256], 4)
    X = torch.empty((M, dims[0]), dtype=torch.bfloat16, device="cuda")
    Yg = torch.empty((M, dims[-1]), dtype=torch.bfloat16, device="cuda")
    Ye = torch.empty_like(Yg)
    Xo = torch.randn((M, 512), device="cuda").to(torch.bfloat16)
    Yo = torch.empty((M, 256), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        graph.capture_begin()
        rc = _noalloc(torch, X, layers, Yg, stream=s.cuda_stream)
        graph.capture_end()
    assert rc == 0
    torch.cuda.synchronize()
    for rep in range(3):
        X.copy_(torch.randn((M, dims[0]), device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        pyc_amd.w8a16_chain(X, layers, Ye)
        assert _noalloc(torch, Xo, other, Yo) == 0
        torch.cuda.synchronize()
        assert torch.equal(Yg, Ye), f"replay {rep} differs from the eager chain"
    Yo_ref = torch.empty_like(Yo)
    pyc_amd.w8a16_chain(Xo, other, Yo_ref)
    torch.cuda.synchronize()
    assert torch.equal(Yo, Yo_ref)
    assert pyc_amd.w8a16_chain_error() == 0

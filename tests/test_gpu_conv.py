"""GPU parity: NHWC/KRSC implicit-GEMM convolution (+bias +ReLU) against the CPU oracle.

The oracle's direct convolution is pinned against scipy.signal.correlate and
closed-form invariants in tests/test_oracle.py (the reference's CUTLASS conv is
not buildable here). Tolerance: BASELINE's max|got-ref| <= 2e-2 * max|ref| and
elementwise one bf16 rounding plus a K-dependent accumulation-order term."""
import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, dev_f32, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu


def _check(got, ref, kred):
    assert rel_max_err(got, ref) <= 2e-2
    bad = np.abs(got - ref) > 2.0 ** -8 * np.abs(ref) + 4e-6 * np.sqrt(kred) * np.abs(ref).max()
    assert not bad.any(), f"{bad.sum()} off, first at {np.argwhere(bad)[0]}"


CASES = [
    # N, H, W, C, K, R, S, pad, stride, bias/relu
    (1, 8, 8, 8, 16, 3, 3, (1, 1), (1, 1), False),
    (2, 9, 7, 16, 24, 3, 3, (1, 1), (2, 2), True),
    (1, 5, 5, 8, 8, 1, 1, (0, 0), (1, 1), False),
    (2, 14, 14, 64, 64, 3, 3, (1, 1), (1, 1), True),
    (1, 6, 7, 8, 130, 5, 3, (2, 1), (1, 2), True),
    (3, 16, 16, 32, 256, 3, 3, (1, 1), (1, 1), True),
]


@pytest.mark.parametrize("N,H,W,C,K,R,S,pad,stride,epi", CASES)
def test_conv_vs_oracle(gpu, N, H, W, C, K, R, S, pad, stride, epi):
    torch = gpu
    r = np.random.default_rng(N + H + W + C + K)
    x = oracle.f32_to_bf16(r.uniform(0, 1, (N, H, W, C)).astype(np.float32))
    w = oracle.f32_to_bf16(r.normal(0, np.sqrt(2.0 / (R * S * C)), (K, R, S, C)).astype(np.float32))
    bias = r.normal(0, 0.1, K).astype(np.float32) if epi else None
    P = (H + 2 * pad[0] - R) // stride[0] + 1
    Q = (W + 2 * pad[1] - S) // stride[1] + 1
    X, Wd = dev_bits16(torch, x), dev_bits16(torch, w)
    Y = torch.empty((N, P, Q, K), dtype=torch.bfloat16, device="cuda")
    pyc_amd.conv2d("hip_conv2d_bf16", X, Wd, Y, pad=pad, stride=stride,
                   bias=dev_f32(torch, bias) if epi else None, relu=epi)
    torch.cuda.synchronize()
    ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(x), oracle.bf16_to_f32(w), bias, pad, stride, relu=epi)
    _check(oracle.bf16_to_f32(host_bits16(Y)), ref, R * S * C)


def test_conv_config4_sampled_images(gpu):
    """Config 4 at full size: x[32,56,56,256] ~ U(0,1) (seed 6), w[256,3,3,256] ~
    N(0, sqrt(2/2304)) (seed 7), bias 0.01*N(0,1) (seed 8), pad 1, ReLU; images 0
    and 31 against the oracle, and a size-independent check on every image: a
    1x1 slice of the filter reproduces a GEMM."""
    torch = gpu
    N, H, W, C, K = 32, 56, 56, 256, 256
    gx = torch.Generator(device="cuda").manual_seed(6)
    gw = torch.Generator(device="cuda").manual_seed(7)
    gb = torch.Generator(device="cuda").manual_seed(8)
    X = torch.rand((N, H, W, C), generator=gx, device="cuda").to(torch.bfloat16)
    Wd = (torch.randn((K, 3, 3, C), generator=gw, device="cuda") * np.sqrt(2.0 / 2304)).to(torch.bfloat16)
    Bv = 0.01 * torch.randn(K, generator=gb, device="cuda")
    Y = torch.empty((N, H, W, K), dtype=torch.bfloat16, device="cuda")
    pyc_amd.conv2d("hip_conv2d_bf16", X, Wd, Y, pad=(1, 1), stride=(1, 1), bias=Bv, relu=True)
    torch.cuda.synchronize()
    w = oracle.bf16_to_f32(host_bits16(Wd))
    b = Bv.cpu().numpy()
    for n in (0, 31):
        x = oracle.bf16_to_f32(host_bits16(X[n:n + 1]))
        ref = oracle.conv2d_nhwc_f32(x, w, b, (1, 1), (1, 1), relu=True)
        _check(oracle.bf16_to_f32(host_bits16(Y[n:n + 1])), ref, 2304)
    # every image: center tap only (1x1 filter) == GEMM over channels
    W1 = Wd[:, 1:2, 1:2, :].contiguous()
    Y1 = torch.empty((N, H, W, K), dtype=torch.bfloat16, device="cuda")
    pyc_amd.conv2d("hip_conv2d_bf16", X, W1, Y1, pad=(0, 0), stride=(1, 1))
    torch.cuda.synchronize()
    ref1 = X.reshape(-1, C).float() @ W1.reshape(K, C).float().t()
    err = (Y1.reshape(-1, K).float() - ref1).abs().max().item()
    assert err <= 2e-2 * ref1.abs().max().item()


def test_conv_reference_abi_and_rejections(gpu):
    torch = gpu
    L = pyc_amd.lib()
    r = np.random.default_rng(5)
    x = r.uniform(0, 1, (1, 8, 8, 16)).astype(np.float16)
    w = r.normal(0, 0.1, (8, 3, 3, 16)).astype(np.float16)
    X, Wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    Y = torch.empty((1, 8, 8, 8), dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.pyc_cutlass_conv2d_dispatch(b"cutlass_conv2d_fprop_f16", 1, 8, 8, 16, 8, 3, 3, 1, 1, 1, 1,
                                         X.data_ptr(), Wd.data_ptr(), Y.data_ptr(), s) == 0
    torch.cuda.synchronize()
    ref = oracle.conv2d_nhwc_f32(x.astype(np.float32), w.astype(np.float32), None, (1, 1), (1, 1), False)
    assert rel_max_err(Y.float().cpu().numpy(), ref) <= 2e-2
    # C_in % 8 != 0 and negative padding are refused before any launch
    assert L.pyc_cutlass_conv2d_dispatch(b"cutlass_conv2d_fprop_f16", 1, 8, 8, 12, 8, 3, 3, 1, 1, 1, 1,
                                         X.data_ptr(), Wd.data_ptr(), Y.data_ptr(), s) == -1
    assert L.pyc_cutlass_conv2d_dispatch(b"cutlass_conv2d_fprop_f16", 1, 8, 8, 16, 8, 3, 3, -1, 1, 1, 1,
                                         X.data_ptr(), Wd.data_ptr(), Y.data_ptr(), s) == -1


TILE_CASES = [
    # N, H, W, C, K of a 3x3, pad 1, stride 1 conv on the persistent kernel: tile rounds
    (8, 56, 56, 256, 256, "bf16"),    # 98 tiles on 256 CUs: one partial round
    # between one and two rounds: one round of 256-pixel tiles, the rest in
    # 144-pixel tiles (the tail kernel), the last of them partly past the end
    (32, 56, 56, 128, 256, "bf16"),   # 392 tiles of 18 K stages -> 256 + 242 tail tiles
    (16, 28, 28, 512, 256, "bf16"),   # 49 tiles of 72 K stages
    (12, 56, 56, 256, 512, "bf16"),   # 294 tiles, two output-channel tiles per pixel block -> 256 + 68
    (24, 56, 56, 256, 256, "f16"),    # 294 tiles -> 256 + 68 tail tiles, fp16
]


@pytest.mark.parametrize("N,H,W,C,K,dt", TILE_CASES)
def test_conv_persistent_tile_rounds(gpu, N, H, W, C, K, dt):
    """The persistent implicit-GEMM conv across tile counts below, at and above
    one round of the grid (so workgroups move on to a second tile, through the
    next-tile prologue, or the remainder goes to the tail kernel). Every output
    element against a plain PyTorch fp32 convolution (an im2col matmul on the
    device, one image at a time), the first and last images against the
    oracle, and a second launch gives identical bits."""
    torch = gpu
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    gx = torch.Generator(device="cuda").manual_seed(N + C)
    gw = torch.Generator(device="cuda").manual_seed(K + 1)
    gb = torch.Generator(device="cuda").manual_seed(K + 2)
    X = torch.rand((N, H, W, C), generator=gx, device="cuda").to(tdt)
    Wd = (torch.randn((K, 3, 3, C), generator=gw, device="cuda") * np.sqrt(2.0 / (9 * C))).to(tdt)
    Bv = 0.01 * torch.randn(K, generator=gb, device="cuda")
    Y = torch.empty((N, H, W, K), dtype=tdt, device="cuda")
    Y2 = torch.empty_like(Y)
    pyc_amd.conv2d(f"hip_conv2d_{dt}", X, Wd, Y, pad=(1, 1), stride=(1, 1), bias=Bv, relu=True)
    pyc_amd.conv2d(f"hip_conv2d_{dt}", X, Wd, Y2, pad=(1, 1), stride=(1, 1), bias=Bv, relu=True)
    torch.cuda.synchronize()
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))
    kred = 9 * C
    wmat = Wd.float().permute(0, 3, 1, 2).reshape(K, kred)  # [K, (c, r, s)] as unfold orders columns
    for n in range(N):
        cols = torch.nn.functional.unfold(X[n:n + 1].float().permute(0, 3, 1, 2), 3, padding=1)[0]
        ref = (wmat @ cols + Bv[:, None]).relu().t()  # [H*W, K]
        got = Y[n].reshape(H * W, K).float()
        err = (got - ref).abs()
        bound = 2.0 ** -8 * ref.abs() + 4e-6 * np.sqrt(kred) * ref.abs().max()
        assert not bool((err > bound).any()), f"image {n}: {int((err > bound).sum())} off"
        assert float(err.max() / ref.abs().max()) <= 2e-2
    b = Bv.cpu().numpy()
    if dt == "bf16":
        w = oracle.bf16_to_f32(host_bits16(Wd))
        for n in (0, N - 1):
            x = oracle.bf16_to_f32(host_bits16(X[n:n + 1]))
            ref = oracle.conv2d_nhwc_f32(x, w, b, (1, 1), (1, 1), relu=True)
            _check(oracle.bf16_to_f32(host_bits16(Y[n:n + 1])), ref, kred)
    else:
        w = Wd.float().cpu().numpy()
        for n in (0, N - 1):
            ref = oracle.conv2d_nhwc_f32(X[n:n + 1].float().cpu().numpy(), w, b, (1, 1), (1, 1), relu=True)
            _check(Y[n:n + 1].float().cpu().numpy(), ref, kred)


def test_conv_unaligned_bias_takes_general_kernel(gpu):
    """A bias that is not 16-byte aligned (a slice one float in) is refused by
    the persistent and tail kernels, which read it as float4; the general
    implicit-GEMM kernel runs the same conv and matches the aligned run."""
    torch = gpu
    N, H, W, C, K = 4, 32, 32, 64, 256  # 16 whole tiles: persistent-eligible when aligned
    g = torch.Generator(device="cuda").manual_seed(31)
    X = torch.rand((N, H, W, C), generator=g, device="cuda").to(torch.bfloat16)
    Wd = (torch.randn((K, 3, 3, C), generator=g, device="cuda") * np.sqrt(2.0 / (9 * C))).to(torch.bfloat16)
    Bfull = 0.01 * torch.randn(K + 1, generator=g, device="cuda")
    Bmis = Bfull[1:]
    assert Bmis.data_ptr() % 16 != 0
    Balign = Bmis.clone()
    Y1 = torch.empty((N, H, W, K), dtype=torch.bfloat16, device="cuda")
    Y2 = torch.empty_like(Y1)
    pyc_amd.conv2d("hip_conv2d_bf16", X, Wd, Y1, pad=(1, 1), stride=(1, 1), bias=Bmis, relu=True)
    pyc_amd.conv2d("hip_conv2d_bf16", X, Wd, Y2, pad=(1, 1), stride=(1, 1), bias=Balign, relu=True)
    torch.cuda.synchronize()
    ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(host_bits16(X[:1])), oracle.bf16_to_f32(host_bits16(Wd)),
                                 Balign.cpu().numpy(), (1, 1), (1, 1), relu=True)
    _check(oracle.bf16_to_f32(host_bits16(Y1[:1])), ref, 9 * C)
    d = (Y1.float() - Y2.float()).abs().max().item()
    assert d <= 2e-2 * Y2.float().abs().max().item()

"""GPU parity: MFMA GEMMs (bf16 / fp16 / fp32) against the CPU oracle.

Tolerances:
  * fp32 GEMM: max|got-ref| / max|ref| <= 1e-4 against the CPU executor;
  * bf16 / fp16 paths: max|got-ref| <= 2e-2 * max|ref| against the fp32 CPU
    result; additionally every element must sit within one output rounding
    (2^-8 relative for bf16) plus a K-dependent accumulation-order term, which
    a dropped k-tile or a transposed operand would break.
"""
import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, dev_f32, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
F32_TOL = 1e-4


def _bf16_inputs(m, n, k, seed, b_trans):
    r = np.random.default_rng(seed)
    a = oracle.f32_to_bf16((r.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32))
    shape = (n, k) if b_trans else (k, n)
    b = oracle.f32_to_bf16(r.standard_normal(shape).astype(np.float32))
    return a, b


def _check_half(got_bits, ref, k):
    got = oracle.bf16_to_f32(got_bits)
    assert rel_max_err(got, ref) <= BF16_TOL
    bound = 2.0 ** -8 * np.abs(ref) + 4e-6 * np.sqrt(k) * np.abs(ref).max()
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{bad.sum()} elements off, first at {np.argwhere(bad)[0]}"


SHAPES = [(256, 256, 64), (512, 768, 256), (300, 200, 72), (1, 1, 8), (33, 65, 40),
          (1024, 1024, 1024), (130, 257, 520), (700, 300, 192), (4096, 4096, 512)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("layout", ["nt", "nn"])
@pytest.mark.parametrize("tile", ["", "_128x128", "_256x256", "_256x256_lds"])
def test_bf16_gemm_vs_oracle(gpu, m, n, k, layout, tile):
    torch = gpu
    bt = layout == "nt"
    if tile.endswith("lds") and layout == "nn" and not (m % 256 == 0 and n % 256 == 0 and k % 64 == 0 and
                                                        (m // 256) * (n // 256) >= 256):
        # the NN persistent kernel alone: shapes outside it are refused, nothing launched
        a, b = _bf16_inputs(m, n, k, 1, bt)
        A, B = dev_bits16(torch, a), dev_bits16(torch, b)
        Cd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        rc = pyc_amd.lib().pyc_hip_gemm_dispatch(b"hip_gemm_bf16_nn_256x256_lds", m, n, k, A.data_ptr(),
                                                 B.data_ptr(), Cd.data_ptr(), 1.0, 0.0, None, 0, None)
        assert rc == -1
        return
    a, b = _bf16_inputs(m, n, k, m * 7 + n + k, bt)
    A, B = dev_bits16(torch, a), dev_bits16(torch, b)
    Cd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    pyc_amd.gemm(f"hip_gemm_bf16_{layout}{tile}", A, B, Cd, m, n, k)
    torch.cuda.synchronize()
    _check_half(host_bits16(Cd), oracle.gemm_bf16(a, b, bt, threads=8), k)


def test_bf16_gemm_8192_sampled_rows(gpu):
    """Config 2 at full size: every row block of the GPU result is checked on a
    row sample (rows spread over all 32 tile rows) against the oracle."""
    torch = gpu
    m = n = k = 8192
    g = torch.Generator(device="cuda").manual_seed(1)
    A = (torch.randn((m, k), generator=g, device="cuda") / np.sqrt(k)).to(torch.bfloat16)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    B = (torch.randn((n, k), generator=g2, device="cuda") / np.sqrt(k)).to(torch.bfloat16)
    Cd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    pyc_amd.gemm("hip_gemm_bf16_nt", A, B, Cd, m, n, k)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, m, 257), [m - 1]]))
    a = host_bits16(A[torch.from_numpy(rows).cuda()])
    b = host_bits16(B)
    ref = oracle.gemm_bf16(a, b, True, threads=16)
    _check_half(host_bits16(Cd[torch.from_numpy(rows).cuda()]), ref, k)
    # size-independent property: the column sums of C equal (1^T A) B^T up to rounding
    colsum = Cd.float().sum(0).double()
    pred = (A.double().sum(0, keepdim=True) @ B.double().t()).squeeze(0)
    assert (colsum - pred).abs().max().item() <= 1e-2 * pred.abs().max().item()


def test_bf16_nt_lds_more_tiles_than_cus(gpu):
    """17 x 17 tiles of 256 x 256 on 256 CUs: the persistent direct-LDS kernel
    runs two tiles on some workgroups (next tile's loads overlap the previous
    tile's stores). Every element is checked."""
    torch = gpu
    m = n = 17 * 256
    k = 128
    a, b = _bf16_inputs(m, n, k, 17, True)
    A, B = dev_bits16(torch, a), dev_bits16(torch, b)
    Cd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    pyc_amd.gemm("hip_gemm_bf16_nt_256x256_lds", A, B, Cd, m, n, k)
    torch.cuda.synchronize()
    _check_half(host_bits16(Cd), oracle.gemm_bf16(a, b, True, threads=8), k)


@pytest.mark.parametrize("alpha,beta,epi", [(0.5, 0.0, 3), (-2.0, 0.0, 1), (0.75, 0.5, 3)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("layout", ["nt", "nn"])
@pytest.mark.parametrize("m,n,k", [(192, 320, 448), (128, 64, 1024), (64, 64, 64),
                                   (2048, 2048, 256), (1024, 4096, 320), (2048, 2048, 64),
                                   # ragged M and N (N % 4 == 0): partial tiles, 64 and 128 wide
                                   (100, 196, 128), (2000, 2052, 128)])
def test_small_gemm_lds_ring(gpu, alpha, beta, epi, dtype, layout, m, n, k):
    """Whole-tile shapes below the persistent kernel's range take the LDS-DMA
    ring kernel: 64 x 64 tiles (7, 16 and 1 k-steps: a ring that is filled by
    the prologue, one that wraps twice, and a single step) and, where 128 x 128
    tiles fill the chip, 128 x 128 tiles (4, 5 and 1 k-steps through a 4-stage
    ring); both B layouts, every epilogue, against the oracle; a second launch
    gives identical bits."""
    torch = gpu
    bt = layout == "nt"
    r = np.random.default_rng(m + n + k + epi + (7 if bt else 0))
    a32 = (r.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b32 = r.standard_normal((n, k) if bt else (k, n)).astype(np.float32)
    c32 = r.standard_normal((m, n)).astype(np.float32)
    bias = r.standard_normal(n).astype(np.float32)
    sym = f"hip_gemm_{dtype}_{layout}"
    outs = []
    for _ in range(2):
        if dtype == "bf16":
            a, b, c0 = oracle.f32_to_bf16(a32), oracle.f32_to_bf16(b32), oracle.f32_to_bf16(c32)
            A, B, Cd = dev_bits16(torch, a), dev_bits16(torch, b), dev_bits16(torch, c0.copy())
        else:
            a, b, c0 = a32.astype(np.float16), b32.astype(np.float16), c32.astype(np.float16)
            A, B, Cd = (torch.from_numpy(x.copy()).cuda() for x in (a, b, c0))
        pyc_amd.gemm(sym, A, B, Cd, m, n, k, alpha=alpha, beta=beta,
                      bias=dev_f32(torch, bias) if epi & 1 else None, epilogue=epi)
        torch.cuda.synchronize()
        outs.append(Cd.clone())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    af, bf_ = (a.astype(np.float32), b.astype(np.float32)) if dtype == "f16" else \
        (oracle.bf16_to_f32(a), oracle.bf16_to_f32(b))
    prod = oracle.matmul_f32(af, np.ascontiguousarray(bf_.T) if bt else bf_)
    cin = c0.astype(np.float32) if dtype == "f16" else oracle.bf16_to_f32(c0)
    ref = alpha * prod + beta * cin + (bias if epi & 1 else 0.0)
    if epi & 2:
        ref = np.maximum(ref, 0.0)
    if dtype == "bf16":
        _check_half(host_bits16(outs[0]), ref, k)
    else:
        got = outs[0].float().cpu().numpy()
        assert rel_max_err(got, ref) <= BF16_TOL
        assert np.all(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * np.sqrt(k) * np.abs(ref).max())


@pytest.mark.parametrize("alpha,beta,epi", [(0.5, 0.0, 3), (1.0, 0.0, 2), (-2.0, 0.0, 1), (0.75, 0.5, 3)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_nt_lds_epilogues_full_tiles(gpu, alpha, beta, epi, dtype):
    """Whole 256 x 256 tiles: beta == 0 takes the persistent kernel (bias /
    ReLU compiled in), beta != 0 the one-shot kernel that reads C back."""
    torch = gpu
    m, n, k = 512, 768, 256
    r = np.random.default_rng(abs(int(alpha * 100)) + epi)
    a32 = (r.standard_normal((m, k)) / np.sqrt(k)).astype(np.float32)
    b32 = r.standard_normal((n, k)).astype(np.float32)
    c32 = r.standard_normal((m, n)).astype(np.float32)
    bias = r.standard_normal(n).astype(np.float32)
    if dtype == "bf16":
        a, b, c0 = oracle.f32_to_bf16(a32), oracle.f32_to_bf16(b32), oracle.f32_to_bf16(c32)
        A, B, Cd = dev_bits16(torch, a), dev_bits16(torch, b), dev_bits16(torch, c0.copy())
        prod, cin = oracle.gemm_bf16(a, b, True), oracle.bf16_to_f32(c0)
    else:
        a, b, c0 = a32.astype(np.float16), b32.astype(np.float16), c32.astype(np.float16)
        A, B, Cd = (torch.from_numpy(x.copy()).cuda() for x in (a, b, c0))
        prod = oracle.matmul_f32(a.astype(np.float32), np.ascontiguousarray(b.astype(np.float32).T))
        cin = c0.astype(np.float32)
    pyc_amd.gemm(f"hip_gemm_{dtype}_nt_256x256_lds", A, B, Cd, m, n, k, alpha=alpha, beta=beta,
                 bias=dev_f32(torch, bias) if epi & 1 else None, epilogue=epi)
    torch.cuda.synchronize()
    ref = alpha * prod + beta * cin + (bias if epi & 1 else 0.0)
    if epi & 2:
        ref = np.maximum(ref, 0.0)
    if dtype == "bf16":
        _check_half(host_bits16(Cd), ref, k)
    else:
        got = Cd.float().cpu().numpy()
        assert rel_max_err(got, ref) <= BF16_TOL
        assert np.all(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * np.sqrt(k) * np.abs(ref).max())


@pytest.mark.parametrize("layout", ["nt", "nn"])
def test_bf16_gemm_epilogue(gpu, layout):
    torch = gpu
    m, n, k = 192, 320, 136
    bt = layout == "nt"
    a, b = _bf16_inputs(m, n, k, 5, bt)
    r = np.random.default_rng(6)
    c0 = oracle.f32_to_bf16(r.standard_normal((m, n)).astype(np.float32))
    bias = r.standard_normal(n).astype(np.float32)
    A, B = dev_bits16(torch, a), dev_bits16(torch, b)
    Cd = dev_bits16(torch, c0.copy())
    pyc_amd.gemm(f"hip_gemm_bf16_{layout}", A, B, Cd, m, n, k, alpha=0.5, beta=-1.25,
                 bias=dev_f32(torch, bias), epilogue=pyc_amd.abi.EPI_BIAS | pyc_amd.abi.EPI_RELU)
    torch.cuda.synchronize()
    ref = np.maximum(0.5 * oracle.gemm_bf16(a, b, bt) - 1.25 * oracle.bf16_to_f32(c0) + bias, 0)
    _check_half(host_bits16(Cd), ref, k)


def test_f16_gemm(gpu):
    torch = gpu
    m, n, k = 200, 136, 264
    r = np.random.default_rng(21)
    a = (r.standard_normal((m, k)) / np.sqrt(k)).astype(np.float16)
    b = r.standard_normal((n, k)).astype(np.float16)
    A = torch.from_numpy(a).cuda()
    B = torch.from_numpy(b).cuda()
    Cd = torch.empty((m, n), dtype=torch.float16, device="cuda")
    pyc_amd.gemm("hip_gemm_f16_nt", A, B, Cd, m, n, k)
    torch.cuda.synchronize()
    ref = oracle.matmul_f32(a.astype(np.float32), np.ascontiguousarray(b.astype(np.float32).T))
    got = Cd.float().cpu().numpy()
    assert rel_max_err(got, ref) <= BF16_TOL
    assert np.all(np.abs(got - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * np.sqrt(k) * np.abs(ref).max())


def test_config1_f32_gemm_bias_relu(gpu):
    """Config 1: X[1024x1024] @ W[1024x1024] + bias[1024] -> ReLU, U(-1,1) seed 0."""
    torch = gpu
    r = np.random.default_rng(0)
    x = r.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    w = r.uniform(-1, 1, (1024, 1024)).astype(np.float32)
    bias = r.uniform(-1, 1, 1024).astype(np.float32)
    X, W, Bv = dev_f32(torch, x), dev_f32(torch, w), dev_f32(torch, bias)
    Y = torch.empty((1024, 1024), dtype=torch.float32, device="cuda")
    pyc_amd.gemm("hip_gemm_f32_nn_64x64", X, W, Y, 1024, 1024, 1024, bias=Bv,
                 epilogue=pyc_amd.abi.EPI_BIAS | pyc_amd.abi.EPI_RELU)
    torch.cuda.synchronize()
    ref = oracle.gemm_bias_relu_f32(x, w, bias, relu=True, threads=8)
    assert rel_max_err(Y.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (5, 7, 3), (64, 64, 32), (100, 70, 50), (257, 129, 65),
                                   # whole 64 x 64 x 64 tiles (the LDS-DMA ring): 1, 2, 3 and 5 k-tiles;
                                   # 35 tiles (no XCD renumbering, a last tile-row group of one) and
                                   # 512 tiles (two per CU, renumbered per XCD)
                                   (64, 64, 64), (128, 64, 128), (64, 192, 192), (192, 128, 320),
                                   (320, 448, 128), (1024, 2048, 192)])
@pytest.mark.parametrize("symbol,bt", [("hip_gemm_f32_nn_64x64", False), ("hip_gemm_f32_nt_64x64", True),
                                       ("cutlass_gemm_simt_f32", True),
                                       ("ada_gemm_k64_warp32_async_f32", False)])
def test_f32_gemm_shapes(gpu, m, n, k, symbol, bt):
    torch = gpu
    r = np.random.default_rng(m + n + k)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (n, k) if bt else (k, n)).astype(np.float32)
    Cd = torch.empty((m, n), dtype=torch.float32, device="cuda")
    pyc_amd.gemm(symbol, dev_f32(torch, a), dev_f32(torch, b), Cd, m, n, k)
    torch.cuda.synchronize()
    ref = oracle.matmul_f32(a, np.ascontiguousarray(b.T) if bt else b)
    assert rel_max_err(Cd.cpu().numpy(), ref) <= F32_TOL


@pytest.mark.parametrize("alpha,beta,epi", [(0.5, 0.0, 3), (1.0, 0.0, 2), (-2.0, 0.0, 1), (0.75, 0.5, 3)])
@pytest.mark.parametrize("symbol,bt", [("hip_gemm_f32_nn_64x64", False), ("hip_gemm_f32_nt_64x64", True)])
def test_f32_gemm_whole_tile_epilogues(gpu, alpha, beta, epi, symbol, bt):
    """fp32 C = epi(alpha * A op(B) + beta * C) on whole 64 x 64 x 64 tiles
    (the LDS-DMA kernel), against the oracle's fp32 matmul; a second launch
    gives identical bits (fixed k-half summation order)."""
    torch = gpu
    m, n, k = 256, 192, 512
    r = np.random.default_rng(abs(int(alpha * 100)) + epi + 7 * bt)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (n, k) if bt else (k, n)).astype(np.float32)
    c0 = r.uniform(-1, 1, (m, n)).astype(np.float32)
    bias = r.uniform(-1, 1, n).astype(np.float32)
    A, B = dev_f32(torch, a), dev_f32(torch, b)
    outs = []
    for _ in range(2):
        Cd = dev_f32(torch, c0.copy())
        pyc_amd.gemm(symbol, A, B, Cd, m, n, k, alpha=alpha, beta=beta,
                     bias=dev_f32(torch, bias) if epi & 1 else None, epilogue=epi)
        torch.cuda.synchronize()
        outs.append(Cd.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = alpha * oracle.matmul_f32(a, np.ascontiguousarray(b.T) if bt else b) + beta * c0
    ref = ref + (bias if epi & 1 else 0.0)
    if epi & 2:
        ref = np.maximum(ref, 0.0)
    assert rel_max_err(outs[0], ref) <= F32_TOL


def test_reference_symbols_and_rejections(gpu):
    torch = gpu
    L = pyc_amd.lib()
    m = n = k = 128
    a, b = _bf16_inputs(m, n, k, 3, False)
    A, B = dev_bits16(torch, a), dev_bits16(torch, b)
    Cd = torch.zeros((m, n), dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    # reference default bf16 symbol: all operands row-major (NN)
    assert L.pyc_cutlass_gemm_dispatch(b"cutlass_gemm_tensorcore_bf16", m, n, k, A.data_ptr(),
                                       B.data_ptr(), Cd.data_ptr(), 1.0, 0.0, s) == 0
    torch.cuda.synchronize()
    _check_half(host_bits16(Cd), oracle.gemm_bf16(a, b, False), k)
    assert L.pyc_cutlass_gemm_dispatch(b"no_such_kernel", m, n, k, A.data_ptr(), B.data_ptr(),
                                       Cd.data_ptr(), 1.0, 0.0, s) == -1
    # the async fp32 kernel accepts alpha=1, beta=0 only (reference ada_async_kernel.cu:285-287)
    assert L.pyc_cutlass_gemm_dispatch(b"ada_gemm_k64_warp32_async_f32", m, n, k, A.data_ptr(),
                                       B.data_ptr(), Cd.data_ptr(), 1.0, 1.0, s) == -1
    assert L.pyc_hip_gemm_dispatch(b"hip_gemm_bf16_nt", 0, n, k, A.data_ptr(), B.data_ptr(),
                                   Cd.data_ptr(), 1.0, 0.0, None, 0, s) == -1


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 512), (17 * 256, 17 * 256, 128), (8192, 4096, 1024)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_nn_lds_equals_nt_on_transpose(gpu, m, n, k, dtype):
    """The persistent kernel with a [K,N] operand (transpose reads from LDS)
    feeds the MFMAs the same values in the same order as the [N,K] form, so
    C = A B equals the NT kernel's A (B^T)^T bit for bit; the NT kernel is
    itself checked against the oracle above."""
    torch = gpu
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    g = torch.Generator(device="cuda").manual_seed(m + n + k)
    A = (torch.randn((m, k), generator=g, device="cuda") / np.sqrt(k)).to(tdt)
    B = torch.randn((k, n), generator=g, device="cuda").to(tdt)
    Bt = B.t().contiguous()
    Cn = torch.empty((m, n), dtype=tdt, device="cuda")
    Ct = torch.empty_like(Cn)
    pyc_amd.gemm(f"hip_gemm_{dtype}_nn_256x256_lds", A, B, Cn, m, n, k)
    pyc_amd.gemm(f"hip_gemm_{dtype}_nt_256x256_lds", A, Bt, Ct, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(Cn.view(torch.int16), Ct.view(torch.int16))


@pytest.mark.parametrize("alpha,epi", [(0.5, 3), (1.0, 2), (-2.0, 1)])
def test_nn_lds_epilogues(gpu, alpha, epi):
    """Bias / ReLU / alpha through the NN persistent kernel equal the NT
    kernel's on the transposed operand, and the oracle's to the bf16 bar."""
    torch = gpu
    m = n = 4096
    k = 256
    r = np.random.default_rng(epi)
    a, b = _bf16_inputs(m, n, k, 40 + epi, False)
    bias = r.standard_normal(n).astype(np.float32)
    A, B = dev_bits16(torch, a), dev_bits16(torch, b)
    Bt = B.t().contiguous()
    Bv = dev_f32(torch, bias)
    Cn = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    Ct = torch.empty_like(Cn)
    pyc_amd.gemm("hip_gemm_bf16_nn", A, B, Cn, m, n, k, alpha=alpha, bias=Bv, epilogue=epi)
    pyc_amd.gemm("hip_gemm_bf16_nt", A, Bt, Ct, m, n, k, alpha=alpha, bias=Bv, epilogue=epi)
    torch.cuda.synchronize()
    assert torch.equal(Cn.view(torch.int16), Ct.view(torch.int16))
    rows = np.arange(0, m, 61)
    ref = alpha * oracle.gemm_bf16(a[rows], b, False, threads=8)
    if epi & 1:
        ref = ref + bias[None, :]
    if epi & 2:
        ref = np.maximum(ref, 0)
    got = oracle.bf16_to_f32(host_bits16(Cn[torch.from_numpy(rows).cuda()]))
    assert rel_max_err(got, ref) <= BF16_TOL


def test_reference_bf16_symbol_8192_row_major_b(gpu):
    """The reference's default bf16 symbol (cutlass_gemm_tensorcore_bf16, B
    row-major [K,N], reference gemm/kernel.cu:175-187) at config 2's size: it
    runs the NN persistent kernel; rows sampled over every tile row against the
    oracle, plus the column-sum property on all of C."""
    torch = gpu
    m = n = k = 8192
    g = torch.Generator(device="cuda").manual_seed(1)
    A = (torch.randn((m, k), generator=g, device="cuda") / np.sqrt(k)).to(torch.bfloat16)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    B = (torch.randn((k, n), generator=g2, device="cuda") / np.sqrt(k)).to(torch.bfloat16)
    Cd = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    L = pyc_amd.lib()
    assert L.pyc_cutlass_gemm_dispatch(b"cutlass_gemm_tensorcore_bf16", m, n, k, A.data_ptr(), B.data_ptr(),
                                       Cd.data_ptr(), 1.0, 0.0, None) == 0
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, m, 263), [m - 1]]))
    a = host_bits16(A[torch.from_numpy(rows).cuda()])
    b = host_bits16(B)
    ref = oracle.gemm_bf16(a, b, False, threads=16)
    _check_half(host_bits16(Cd[torch.from_numpy(rows).cuda()]), ref, k)
    colsum = Cd.float().sum(0).double()
    pred = (A.double().sum(0, keepdim=True) @ B.double()).squeeze(0)
    assert (colsum - pred).abs().max().item() <= 1e-2 * pred.abs().max().item()

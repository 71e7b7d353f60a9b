"""GPU parity: fused causal / non-causal attention against the CPU oracle.

The reference pins nothing here (its attention kernel is an identity copy), so
the oracle itself is pinned in tests/test_oracle.py against torch's fp64
scaled_dot_product_attention and closed-form invariants. Tolerance: BASELINE's
max|got-ref| <= 2e-2 * max|ref|, and elementwise |got-ref| <= 2^-7|ref| +
1e-2 max|ref| (bf16 output rounding plus bf16 rounding of the probabilities)."""
import numpy as np
import pytest

import oracle
import pyc_amd
from tests.gpu_util import dev_bits16, host_bits16, rel_max_err

pytestmark = pytest.mark.gpu


def _qkv(B, H, S, D, seed):
    r = np.random.default_rng(seed)
    return [oracle.f32_to_bf16(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3)]


def _check(got, ref):
    assert rel_max_err(got, ref) <= 2e-2
    bad = np.abs(got - ref) > 2.0 ** -7 * np.abs(ref) + 1e-2 * np.abs(ref).max()
    assert not bad.any(), f"{bad.sum()} off, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("B,H,S,D", [(1, 2, 128, 128), (1, 2, 256, 128), (2, 2, 300, 64), (1, 1, 37, 128),
                                     (1, 1, 1, 64), (1, 3, 520, 128), (2, 1, 64, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_vs_oracle(gpu, B, H, S, D, causal):
    torch = gpu
    q, k, v = _qkv(B, H, S, D, B * 1000 + H * 100 + S + D)
    Q, K, V = (dev_bits16(torch, t) for t in (q, k, v))
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    pyc_amd.attention("hip_attention_bf16", Q, K, V, O, causal, scale)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(host_bits16(O))
    ref = oracle.attention_f32(*(oracle.bf16_to_f32(t) for t in (q, k, v)), causal, scale)
    _check(got, ref)


@pytest.mark.parametrize("case", ["large_logits", "growing_keys", "negative_scale", "zero_scale",
                                  "all_underflow"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_softmax_paths(gpu, case, D, causal):
    """Online-softmax paths: logits whose block maxima jump far above the
    current reference (large_logits, growing_keys: key j scaled by 1 + j/32 so
    every later block raises the max), scales <= 0, and exponents that all
    underflow against the initial reference (all_underflow: positive q.k
    around 100 times a scale of -4, so every exp2 of the first block is 0
    until the reference moves down to the block max)."""
    torch = gpu
    B, H, S = 1, 2, 300
    r = np.random.default_rng(len(case) * 10 + D + causal)
    q = r.standard_normal((B, H, S, D)).astype(np.float32)
    k = r.standard_normal((B, H, S, D)).astype(np.float32)
    v = r.standard_normal((B, H, S, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    if case == "large_logits":
        q *= 4.0
        k *= 4.0
    elif case == "growing_keys":
        k *= (1.0 + np.arange(S, dtype=np.float32) / 32.0)[None, None, :, None]
    elif case == "negative_scale":
        scale = -0.3 / np.sqrt(D)
    elif case == "all_underflow":
        q = np.abs(q) + 1.0
        k = np.abs(k) + 1.0
        scale = -4.0
    else:
        scale = 0.0
    q, k, v = (oracle.f32_to_bf16(t) for t in (q, k, v))
    Q, K, V = (dev_bits16(torch, t) for t in (q, k, v))
    O = torch.empty_like(Q)
    pyc_amd.attention("hip_attention_bf16", Q, K, V, O, causal, scale)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(host_bits16(O))
    ref = oracle.attention_f32(*(oracle.bf16_to_f32(t) for t in (q, k, v)), causal, scale)
    _check(got, ref)


def test_attention_config3_sampled_heads(gpu):
    """Config 3 at full size ([8,32,2048,128], causal, scale 1/sqrt(128)): two (b,h)
    pairs against the oracle, plus the size-independent invariant O[:,:,0] = V[:,:,0]
    for every head."""
    torch = gpu
    B, H, S, D = 8, 32, 2048, 128
    gens = [torch.Generator(device="cuda").manual_seed(s) for s in (3, 4, 5)]
    Q, K, V = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for g in gens)
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    pyc_amd.attention("hip_attention_bf16", Q, K, V, O, True, scale)
    torch.cuda.synchronize()
    for b, h in [(0, 0), (7, 31)]:
        q, k, v = (oracle.bf16_to_f32(host_bits16(t[b:b + 1, h:h + 1])) for t in (Q, K, V))
        ref = oracle.attention_f32(q, k, v, True, scale)
        _check(oracle.bf16_to_f32(host_bits16(O[b:b + 1, h:h + 1])), ref)
    torch.testing.assert_close(O[:, :, 0].float(), V[:, :, 0].float(), rtol=2 ** -7, atol=1e-3)


def test_attention_config3_every_head_vs_torch_fp32(gpu):
    """Config 3 at full size, all 256 (b,h) heads against a plain PyTorch fp32
    reference of the same op (scores, causal mask, softmax and P.V in fp32 on the
    device, one batch at a time), with the same bounds as the oracle checks."""
    torch = gpu
    B, H, S, D = 8, 32, 2048, 128
    gens = [torch.Generator(device="cuda").manual_seed(s) for s in (3, 4, 5)]
    Q, K, V = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for g in gens)
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    pyc_amd.attention("hip_attention_bf16", Q, K, V, O, True, scale)
    torch.cuda.synchronize()
    mask = torch.ones((S, S), dtype=torch.bool, device="cuda").triu(1)
    worst = 0.0
    for b in range(B):
        q, k, v = (t[b].float() for t in (Q, K, V))
        sc = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
        sc.masked_fill_(mask, float("-inf"))
        ref = torch.matmul(torch.softmax(sc, dim=-1), v)
        del sc
        got = O[b].float()
        err = (got - ref).abs()
        worst = max(worst, float(err.max() / ref.abs().max()))
        bound = 2.0 ** -7 * ref.abs() + 1e-2 * ref.abs().max()
        assert not bool((err > bound).any()), f"batch {b}: {int((err > bound).sum())} off"
    assert worst <= 2e-2, worst


def test_attention_f16_and_reference_abi(gpu):
    torch = gpu
    S, D = 192, 128
    r = np.random.default_rng(77)
    q, k, v = (r.standard_normal((S, D)).astype(np.float16) for _ in range(3))
    Q, K, V = (torch.from_numpy(t).cuda() for t in (q, k, v))
    O = torch.empty_like(Q)
    L = pyc_amd.lib()
    s = torch.cuda.current_stream().cuda_stream
    # reference ABI: one head, seq_len x d_head, non-causal (reference cuda_backend.h:128-138)
    assert L.pyc_cutlass_attention_dispatch(b"cutlass_attention_f16", S, D, Q.data_ptr(), K.data_ptr(),
                                            V.data_ptr(), O.data_ptr(), 0.1, s) == 0
    torch.cuda.synchronize()
    ref = oracle.attention_f32(*(t.astype(np.float32)[None, None] for t in (q, k, v)), False, 0.1)[0, 0]
    _check(O.float().cpu().numpy(), ref)
    assert L.pyc_cutlass_attention_dispatch(b"cutlass_attention_f16", S, 96, Q.data_ptr(), K.data_ptr(),
                                            V.data_ptr(), O.data_ptr(), 0.1, s) == -1


@pytest.mark.parametrize("B,H,S,D,causal", [
    (4, 150, 300, 128, True),    # 600 units: every workgroup streams three rounds of one-part units
    (2, 160, 700, 128, True),    # nqb = 3: pairs (2, 0) and the middle q-block alone; 640 units
    (3, 100, 520, 64, False),    # non-causal, 3 q-blocks per head, 900 units
    (1, 300, 1100, 128, True),   # nqb = 5, ragged last q-block, 900 units with 1 or 2 parts
])
def test_attention_persistent_rounds(gpu, B, H, S, D, causal):
    """More units than CUs, so each workgroup of the persistent grid streams
    several units (and their q-blocks) through one K/V ring: the hand-over
    from one part to the next (the next part's Q and first blocks loaded
    during the current part's tail) and from one head to another. Heads from
    the first, middle and last units of the grid are checked against the
    oracle; every head against O[:, :, 0] = V[:, :, 0] (causal)."""
    torch = gpu
    gens = [torch.Generator(device="cuda").manual_seed(s) for s in (11, 12, 13)]
    Q, K, V = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.bfloat16) for g in gens)
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    pyc_amd.attention("hip_attention_bf16", Q, K, V, O, causal, scale)
    torch.cuda.synchronize()
    picks = {(0, 0), (B - 1, H - 1), (B // 2, H // 2), (0, H - 1), (B - 1, 1)}
    for b, h in sorted(picks):
        q, k, v = (oracle.bf16_to_f32(host_bits16(t[b:b + 1, h:h + 1])) for t in (Q, K, V))
        ref = oracle.attention_f32(q, k, v, causal, scale)
        _check(oracle.bf16_to_f32(host_bits16(O[b:b + 1, h:h + 1])), ref)
    if causal:
        torch.testing.assert_close(O[:, :, 0].float(), V[:, :, 0].float(), rtol=2 ** -7, atol=1e-3)


def test_attention_f16_persistent_rounds(gpu):
    """The f16 instantiation across several rounds per workgroup."""
    torch = gpu
    B, H, S, D = 2, 200, 600, 128
    g = torch.Generator(device="cuda").manual_seed(21)
    Q, K, V = (torch.randn((B, H, S, D), generator=g, device="cuda").to(torch.float16) for _ in range(3))
    O = torch.empty_like(Q)
    scale = 1.0 / np.sqrt(D)
    pyc_amd.attention("hip_attention_f16", Q, K, V, O, True, scale)
    torch.cuda.synchronize()
    for b, h in [(0, 0), (1, 199), (1, 77)]:
        q, k, v = (t[b:b + 1, h:h + 1].float().cpu().numpy() for t in (Q, K, V))
        ref = oracle.attention_f32(q, k, v, True, scale)
        _check(O[b:b + 1, h:h + 1].float().cpu().numpy(), ref)

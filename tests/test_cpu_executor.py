"""CPU: the engine's own CPU executor over the ops and types the GPU backend
lowers (the reference executor, compiler_api.c:1877-2092, runs F32
MATMUL/ADD/RELU only). This is the executor pyc_cuda_dispatch falls back to
(reference cuda_backend.c:2883-2908), so every module the GPU runs must also
run here.

Each op is checked against the oracle (tests/test_oracle.py pins it): the
executor decodes half inputs to fp32, computes each op in the oracle's
accumulation order and rounds the result to its value's type, so GEMM,
fp8-weight GEMM, conv and attention results equal the oracle's rounded to
bf16 bit for bit. GELU and LayerNorm are within one bf16 rounding of the
fp64 definition. The number-format helpers are checked against numpy's
float16 (all 65536 codes) and the oracle's e4m3 table."""
import ctypes as C

import numpy as np
import pytest

import oracle
from pyc_amd import abi
from tests import engine_util as eu

BF = abi.DTYPE_BF16


@pytest.fixture(autouse=True)
def _threads(monkeypatch):
    monkeypatch.setenv("PYC_NUM_THREADS", "4")


def _lib():
    L = eu.mine()
    L.pyc_cpu_f16_to_f32.argtypes = [C.c_uint16]
    L.pyc_cpu_f16_to_f32.restype = C.c_float
    L.pyc_cpu_f32_to_f16.argtypes = [C.c_float]
    L.pyc_cpu_f32_to_f16.restype = C.c_uint16
    L.pyc_cpu_e4m3_to_f32.argtypes = [C.c_uint8]
    L.pyc_cpu_e4m3_to_f32.restype = C.c_float
    return L


def test_f16_decode_all_codes():
    L = _lib()
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([L.pyc_cpu_f16_to_f32(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_matches_numpy():
    L = _lib()
    r = np.random.default_rng(0)
    vals = np.concatenate([
        r.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** r.integers(-9, 6, 4000).astype(np.float32),
        # every half value, and the midpoints between neighbours (ties to even)
        np.arange(0, 0x7c00, 37, dtype=np.uint16).view(np.float16).astype(np.float32),
        ((np.arange(0, 0x7bff, 41, dtype=np.uint16).view(np.float16).astype(np.float64) +
          np.arange(1, 0x7c00, 41, dtype=np.uint16).view(np.float16).astype(np.float64)) / 2).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25], np.float32),
    ])
    vals = np.concatenate([vals, -vals])
    got = np.array([L.pyc_cpu_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_e4m3_decode_all_codes():
    L = _lib()
    want = oracle.e4m3_table()
    got = np.array([L.pyc_cpu_e4m3_to_f32(c) for c in range(256)], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


def _run(ops, ins, dts, out_shape, out_dtype=BF):
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CPU)
    assert mdl.status == 0
    np_out = np.uint16 if out_dtype != abi.DTYPE_F32 else np.float32
    st, (out,), s = mdl.run(ins, [out_shape], in_dtypes=dts, out_dtypes=[out_dtype], out_np_dtype=np_out)
    mdl.close()
    assert st == 0, s.execution_path
    return out


def test_bf16_gemm_bias_relu_module():
    m, k, n = 48, 80, 56
    r = np.random.default_rng(1)
    a = oracle.f32_to_bf16(r.standard_normal((m, k)).astype(np.float32))
    b = oracle.f32_to_bf16(r.standard_normal((k, n)).astype(np.float32))
    bias = r.standard_normal(n).astype(np.float32)
    ops = [eu.op(abi.OP_INPUT, "a", (m, k), dtype=BF), eu.op(abi.OP_INPUT, "b", (k, n), dtype=BF),
           eu.op(abi.OP_INPUT, "bias", (n,)), eu.op(abi.OP_MATMUL, "mm", (), (0, 1), dtype=BF),
           eu.op(abi.OP_ADD, "add", (), (3, 2), dtype=BF), eu.op(abi.OP_RELU, "relu", (), (4,), dtype=BF),
           eu.op(abi.OP_OUTPUT, "o", (m, n), (5,), dtype=BF)]
    out = _run(ops, [a, b, bias], [BF, BF, abi.DTYPE_F32], (m, n))
    # the value of every op is stored as bf16: GEMM rounded, then bias added and rounded
    mm = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.gemm_bf16(a, b, False)))
    want = oracle.f32_to_bf16(np.maximum(oracle.bf16_to_f32(oracle.f32_to_bf16(mm + bias[None, :])), 0))
    assert np.array_equal(out, want)


def _fp8_chain_module(M, dims, seed):
    r = np.random.default_rng(seed)
    x = oracle.f32_to_bf16(r.standard_normal((M, dims[0])).astype(np.float32))
    ops = [eu.op(abi.OP_INPUT, "x", (M, dims[0]), dtype=BF)]
    ins, dts, host = [x], [BF], []
    cur = 0
    for l, (K, N) in enumerate(zip(dims[:-1], dims[1:])):
        wq, sc = oracle.quantize_e4m3_per_col((r.standard_normal((K, N)) * np.sqrt(2 / K)).astype(np.float32))
        host.append((wq, sc, l % 2 == 0))
        base = len(ops)
        ops += [eu.op(abi.OP_INPUT, f"w{l}", (N, K), dtype=abi.DTYPE_FP8_E4M3), eu.op(abi.OP_INPUT, f"s{l}", (N,)),
                eu.op(abi.OP_MATMUL, f"mm{l}", (), (cur, base, base + 1), dtype=BF)]
        ins += [wq, sc]
        dts += [abi.DTYPE_FP8_E4M3, abi.DTYPE_F32]
        cur = base + 2
        if l % 2 == 0:
            ops.append(eu.op(abi.OP_RELU, f"relu{l}", (), (cur,), dtype=BF))
            cur += 1
    ops.append(eu.op(abi.OP_OUTPUT, "y", (M, dims[-1]), (cur,), dtype=BF))
    ref = x
    for wq, sc, relu in host:
        ref = oracle.w8a16_layer(ref, wq, sc, relu)
    return ops, ins, dts, ref


def test_fp8_chain_module():
    M, dims = 7, [256, 384, 128, 192]
    ops, ins, dts, ref = _fp8_chain_module(M, dims, 2)
    out = _run(ops, ins, dts, (M, dims[-1]))
    assert np.array_equal(out, ref)


def test_conv2d_module():
    N, H, W, C, K, R, S = 2, 9, 7, 16, 24, 3, 3
    r = np.random.default_rng(3)
    x = oracle.f32_to_bf16(r.uniform(0, 1, (N, H, W, C)).astype(np.float32))
    w = oracle.f32_to_bf16((r.standard_normal((K, R, S, C)) * 0.2).astype(np.float32))
    ops = [eu.op(abi.OP_INPUT, "x", (N, H, W, C), dtype=BF), eu.op(abi.OP_INPUT, "w", (K, R, S, C), dtype=BF),
           eu.op(abi.OP_CONV2D, "conv@s2x1p1x0", (), (0, 1), dtype=BF)]
    P, Q = (H + 2 - R) // 2 + 1, (W - S) // 1 + 1
    ops.append(eu.op(abi.OP_OUTPUT, "y", (N, P, Q, K), (2,), dtype=BF))
    out = _run(ops, [x, w], [BF, BF], (N, P, Q, K))
    ref = oracle.conv2d_nhwc_f32(oracle.bf16_to_f32(x), oracle.bf16_to_f32(w), None, (1, 0), (2, 1), False)
    assert np.array_equal(out, oracle.f32_to_bf16(ref))


@pytest.mark.parametrize("causal", [True, False])
def test_attention_module(causal):
    B, H, S, D = 2, 3, 37, 64
    r = np.random.default_rng(4)
    q, k, v = (oracle.f32_to_bf16(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    name = "attn_causal" if causal else "attn"
    ops = [eu.op(abi.OP_INPUT, n, (B, H, S, D), dtype=BF) for n in "qkv"]
    ops += [eu.op(abi.OP_ATTENTION, name, (), (0, 1, 2), dtype=BF),
            eu.op(abi.OP_OUTPUT, "o", (B, H, S, D), (3,), dtype=BF)]
    out = _run(ops, [q, k, v], [BF] * 3, (B, H, S, D))
    ref = oracle.attention_f32(*(oracle.bf16_to_f32(t) for t in (q, k, v)), causal, 1.0 / np.sqrt(D))
    assert np.array_equal(out, oracle.f32_to_bf16(ref))


def test_gelu_layernorm_module():
    rows, D = 6, 40
    r = np.random.default_rng(5)
    x = oracle.f32_to_bf16((r.standard_normal((rows, D)) * 2).astype(np.float32))
    g = oracle.f32_to_bf16(r.standard_normal(D).astype(np.float32))
    be = oracle.f32_to_bf16(r.standard_normal(D).astype(np.float32))
    ops = [eu.op(abi.OP_INPUT, "x", (rows, D), dtype=BF), eu.op(abi.OP_INPUT, "g", (D,), dtype=BF),
           eu.op(abi.OP_INPUT, "b", (D,), dtype=BF), eu.op(abi.OP_GELU, "gelu", (), (0,), dtype=BF),
           eu.op(abi.OP_LAYERNORM, "ln@eps1e-3", (), (3, 1, 2), dtype=BF),
           eu.op(abi.OP_OUTPUT, "y", (rows, D), (4,), dtype=BF)]
    out = oracle.bf16_to_f32(_run(ops, [x, g, be], [BF] * 3, (rows, D)))
    h = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.gelu_f64(oracle.bf16_to_f32(x).astype(np.float64))
                                              .astype(np.float32)))
    ref = oracle.layernorm_f64(h.astype(np.float64), oracle.bf16_to_f32(g), oracle.bf16_to_f32(be), 1e-3)
    # one bf16 rounding of the output (and of the GELU intermediate, identical here)
    assert np.all(np.abs(out - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)


def test_thread_count_does_not_change_results(monkeypatch):
    M, dims = 5, [128, 320, 64]
    ops, ins, dts, ref = _fp8_chain_module(M, dims, 6)
    for t in ("1", "3", "32"):
        monkeypatch.setenv("PYC_NUM_THREADS", t)
        assert np.array_equal(_run(ops, ins, dts, (M, dims[-1])), ref), t


def test_unsupported_kind_still_fails():
    ops = [eu.op(abi.OP_INPUT, "x", (4,)), eu.op(abi.OP_REDUCE_SUM, "r", (), (0,)), eu.op(abi.OP_OUTPUT, "o", (1,), (1,))]
    mdl = eu.Model(eu.mine(), ops, backend=abi.BACKEND_CPU)
    st, _, _ = mdl.run([np.ones(4, np.float32)], [(1,)])
    mdl.close()
    assert st == abi.STATUS_RUNTIME_FAILED

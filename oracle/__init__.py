"""CPU oracle for the MI355X backend — TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker. It wraps two native libraries:

* ``_build/liboracle.so`` — the C restatement in ``oracle.c`` of the
  reference CPU executor (reference src/compiler/compiler_api.c:1747-2092) and
  of fp32 reference attention / NHWC conv / fp8-weight GEMM.
* ``_ref/libpyc_ref.so`` — the reference's own C11 engine compiled from
  /root/reference by ``Makefile.ref`` (present only where it was built).

plus float64 numpy restatements of GELU and LayerNorm (ops the reference
executes nowhere), pinned against torch in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
REF_LIB_PATH = os.path.join(_HERE, "_ref", "libpyc_ref.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        Z = ctypes.c_size_t
        I = ctypes.c_int
        F = ctypes.c_float
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [F]
        L.orc_bf16_to_f32.restype = F
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_e4m3_to_f32.restype = F
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_f32_to_e4m3.restype = ctypes.c_uint8
        L.orc_f32_to_e4m3.argtypes = [F]
        L.orc_f32_to_bf16_array.argtypes = [P, P, Z]
        L.orc_bf16_to_f32_array.argtypes = [P, P, Z]
        L.orc_matmul_f32.argtypes = [P, P, P, Z, Z, Z, I]
        L.orc_add_epilogue.argtypes = [P, P, Z, Z, I]
        L.orc_relu.argtypes = [P, Z]
        L.orc_gemm_bf16.argtypes = [P, P, P, Z, Z, Z, I, Z, Z, I]
        L.orc_attention_f32.argtypes = [P, P, P, P, I, I, I, I, I, F, I, I]
        L.orc_conv2d_nhwc_f32.argtypes = [P, P, P, P] + [I] * 14
        L.orc_w8a16_layer.argtypes = [P, P, P, P, I, I, I, I]
        L.orc_w8a16_layer_mt.argtypes = [P, P, P, P, I, I, I, I, I]
        L.orc_quantize_e4m3_per_col.argtypes = [P, I, I, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_array(_p(h), _p(out), h.size)
    return out


def e4m3_table() -> np.ndarray:
    return np.array([lib().orc_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_e4m3
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.uint8).reshape(np.shape(x))


def matmul_f32(a: np.ndarray, b: np.ndarray, threads: int = 1) -> np.ndarray:
    """The CPU executor's GEMM: a[m,k] @ b[k,n], fp32, k ascending."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f32(_p(a), _p(b), _p(c), m, k, n, threads)
    return c


def add_epilogue(out: np.ndarray, addend: np.ndarray, mode: int) -> None:
    m, n = out.shape
    addend = np.ascontiguousarray(addend, dtype=np.float32)
    lib().orc_add_epilogue(_p(out), _p(addend), m, n, mode)


def relu_(out: np.ndarray) -> None:
    lib().orc_relu(_p(out), out.size)


def gemm_bias_relu_f32(a, b, bias, relu=True, threads=1):
    """The reference CUDA path's ROW_BIAS epilogue applied to the executor GEMM."""
    c = matmul_f32(a, b, threads)
    if bias is not None:
        add_epilogue(c, bias, 2)
    if relu:
        relu_(c)
    return c


def gemm_bf16(a_bits, b_bits, b_trans: bool, rows=None, threads=1) -> np.ndarray:
    """fp32 CPU GEMM of decoded bf16 operands for rows [r0, r1)."""
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16)
    b_bits = np.ascontiguousarray(b_bits, dtype=np.uint16)
    m, k = a_bits.shape
    n = b_bits.shape[0] if b_trans else b_bits.shape[1]
    r0, r1 = rows if rows is not None else (0, m)
    c = np.empty((r1 - r0, n), dtype=np.float32)
    lib().orc_gemm_bf16(_p(a_bits), _p(b_bits), _p(c), m, n, k, int(b_trans), r0, r1, threads)
    return c


def attention_f32(q, k, v, causal: bool, scale: float, bh=None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, H, S, D = q.shape
    bh0, bh1 = bh if bh is not None else (0, B * H)
    o = np.zeros_like(q)
    lib().orc_attention_f32(_p(q), _p(k), _p(v), _p(o), B, H, S, D, int(causal),
                            float(scale), bh0, bh1)
    return o


def conv2d_nhwc_f32(x, w, bias, pad, stride, relu: bool, images=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, H, W, C = x.shape
    K, R, S, C2 = w.shape
    assert C == C2
    ph, pw = pad
    sh, sw = stride
    P = (H + 2 * ph - R) // sh + 1
    Q = (W + 2 * pw - S) // sw + 1
    n0, n1 = images if images is not None else (0, N)
    y = np.zeros((N, P, Q, K), dtype=np.float32)
    bptr = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        bptr = _p(bias)
    lib().orc_conv2d_nhwc_f32(_p(x), _p(w), bptr, _p(y), N, H, W, C, K, R, S,
                              ph, pw, sh, sw, int(relu), n0, n1)
    return y


def w8a16_layer(x_bits, wq, scale, relu: bool, threads: int = 1) -> np.ndarray:
    """Output channels split over `threads` threads; the result does not
    depend on the thread count."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    M, K = x_bits.shape
    N = wq.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    if threads > 1:
        lib().orc_w8a16_layer_mt(_p(x_bits), _p(wq), _p(scale), _p(y), M, N, K, int(relu), int(threads))
    else:
        lib().orc_w8a16_layer(_p(x_bits), _p(wq), _p(scale), _p(y), M, N, K, int(relu))
    return y


def quantize_e4m3_per_col(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    K, N = w.shape
    wq = np.empty((N, K), dtype=np.uint8)
    scale = np.empty((N,), dtype=np.float32)
    lib().orc_quantize_e4m3_per_col(_p(w), K, N, _p(wq), _p(scale))
    return wq, scale


def w8a16_chain(x_bits, layers, threads: int = 1) -> np.ndarray:
    """layers: list of (wq_up [F,D], s_up [F], wq_down [D,F], s_down [D])."""
    h = x_bits
    for wq_up, s_up, wq_dn, s_dn in layers:
        t = w8a16_layer(h, wq_up, s_up, True, threads)
        h = w8a16_layer(t, wq_dn, s_dn, False, threads)
    return h


def gelu_f64(x: np.ndarray) -> np.ndarray:
    """GELU, exact form 0.5 x (1 + erf(x / sqrt(2))), in float64 (the
    reference defines no GELU: it is a graph break there; this is PyTorch's
    default definition)."""
    from scipy.special import erf
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def layernorm_f64(x: np.ndarray, gamma=None, beta=None, eps: float = 1e-5) -> np.ndarray:
    """LayerNorm over the last dimension in float64: (x - mean) / sqrt(var +
    eps) * gamma + beta, var the population variance (as PyTorch's
    layer_norm; the reference executes no LAYERNORM)."""
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, dtype=np.float64)
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)
    return y

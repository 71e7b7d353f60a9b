"""pyc_amd — MI355X (gfx950) backend for PyC's compiler-next run path.

The product is the C-ABI shared library ``pyc_amd/lib/libpyc_amd.so`` (HIP
kernels + C11 host engine, declared in ``include/pyc/*.h``). This package only
loads it and offers thin Python wrappers that pass device pointers of torch
tensors through that C-ABI; torch provides device memory and streams.

Loading fails loudly: there is no Python or CPU fallback for any kernel.
"""
from __future__ import annotations

import ctypes as C
import os

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libpyc_amd.so")

_lib = None


class PycError(RuntimeError):
    pass


def _declare(L: C.CDLL) -> None:
    P, I, F, Z = C.c_void_p, C.c_int, C.c_float, C.c_size_t
    S = C.c_char_p
    L.pyc_hip_gemm_dispatch.argtypes = [S, I, I, I, P, P, P, F, F, P, I, P]
    L.pyc_hip_gemm_dispatch.restype = I
    L.pyc_cutlass_gemm_dispatch.argtypes = [S, I, I, I, P, P, P, F, F, P]
    L.pyc_cutlass_gemm_dispatch.restype = I
    L.pyc_hip_attention_dispatch.argtypes = [S, I, I, I, I, I, P, P, P, P, F, P]
    L.pyc_hip_attention_dispatch.restype = I
    L.pyc_cutlass_attention_dispatch.argtypes = [S, I, I, P, P, P, P, F, P]
    L.pyc_cutlass_attention_dispatch.restype = I
    L.pyc_hip_conv2d_dispatch.argtypes = [S] + [I] * 11 + [P, P, P, I, P, P]
    L.pyc_hip_conv2d_dispatch.restype = I
    L.pyc_cutlass_conv2d_dispatch.argtypes = [S] + [I] * 11 + [P, P, P, P]
    L.pyc_cutlass_conv2d_dispatch.restype = I
    L.pyc_hip_w8a16_gemm_dispatch.argtypes = [S, I, I, I, P, P, P, I, P, P]
    L.pyc_hip_w8a16_gemm_dispatch.restype = I
    L.pyc_hip_w8a16_chain_dispatch.argtypes = [S, I, I, P, P, P, P, P, P, P, P]
    L.pyc_hip_w8a16_chain_dispatch.restype = I
    L.pyc_hip_w8a16_chain_dispatch_noalloc.argtypes = [S, I, I, P, P, P, P, P, P, P, P]
    L.pyc_hip_w8a16_chain_dispatch_noalloc.restype = I
    L.pyc_hip_w8a16_chain_reserve.argtypes = [I, I, P, P]
    L.pyc_hip_w8a16_chain_reserve.restype = I
    L.pyc_hip_w8a16_chain_error.argtypes = [I]
    L.pyc_hip_w8a16_chain_error.restype = I
    L.pyc_hip_w8a16_chain_supported.argtypes = [I, I, P, P]
    L.pyc_hip_w8a16_chain_supported.restype = I
    L.pyc_hip_w8a16_chain_error_raise.argtypes = []
    L.pyc_hip_w8a16_chain_error_raise.restype = I
    L.pyc_hip_gelu_dispatch.argtypes = [S, Z, P, P, P]
    L.pyc_hip_gelu_dispatch.restype = I
    L.pyc_hip_layernorm_dispatch.argtypes = [S, I, I, F, P, P, P, P, P]
    L.pyc_hip_layernorm_dispatch.restype = I
    L.pyc_hip_device_query.argtypes = [C.POINTER(abi.DeviceInfo)]
    L.pyc_hip_device_query.restype = I
    L.pyc_hip_kernel_resources_query.argtypes = [S, C.POINTER(abi.KernelResources)]
    L.pyc_hip_kernel_resources_query.restype = I
    L.pyc_hip_autotune_gemm.argtypes = [I, I, I, I, I, C.c_char_p, Z, C.POINTER(C.c_double), I]
    L.pyc_hip_autotune_gemm.restype = I
    L.pyc_hip_autotune_conv2d.argtypes = [I] + [I] * 11 + [I, C.c_char_p, Z, C.POINTER(C.c_double), I]
    L.pyc_hip_autotune_conv2d.restype = I
    L.pyc_hip_kernel_symbol_count.argtypes = [S]
    L.pyc_hip_kernel_symbol_count.restype = I
    L.pyc_cutlass_kernel_count.argtypes = [S]
    L.pyc_cutlass_kernel_count.restype = I
    L.pyc_cutlass_registry_init.argtypes = []
    L.pyc_cutlass_registry_init.restype = None
    L.pyc_cuda_dispatch_trace_init.argtypes = [C.POINTER(abi.DispatchTrace)]
    L.pyc_cuda_dispatch_trace_init.restype = None
    L.pyc_cuda_current_hardware_family.argtypes = []
    L.pyc_cuda_current_hardware_family.restype = I
    L.pyc_cuda_dispatch.argtypes = [C.POINTER(abi.IrModule), C.POINTER(abi.Tensor), Z,
                                    C.POINTER(abi.Tensor), Z, abi.CPU_EXECUTOR_FN, P,
                                    C.POINTER(abi.DispatchTrace)]
    L.pyc_cuda_dispatch.restype = I
    # registry
    L.pyc_kernel_registry_reset.argtypes = []
    L.pyc_kernel_register.argtypes = [C.POINTER(abi.KernelDesc)]
    L.pyc_kernel_register.restype = I
    L.pyc_kernel_select.argtypes = [S, I, C.POINTER(abi.KernelDesc)]
    L.pyc_kernel_select.restype = I
    L.pyc_kernel_select_with_policy.argtypes = [S, I, I, C.c_double, C.POINTER(abi.KernelDesc),
                                                C.POINTER(abi.KernelSelectionTrace)]
    L.pyc_kernel_select_with_policy.restype = I
    L.pyc_kernel_coselect_with_context.argtypes = [S, I, I, C.POINTER(abi.CoselectContext),
                                                   C.POINTER(abi.KernelDesc),
                                                   C.POINTER(abi.KernelSelectionTrace)]
    L.pyc_kernel_coselect_with_context.restype = I
    L.pyc_kernel_promote_symbol.argtypes = [S, I, S]
    L.pyc_kernel_promote_symbol.restype = I
    L.pyc_kernel_promoted_symbol.argtypes = [S, I, C.c_char_p, Z]
    L.pyc_kernel_promoted_symbol.restype = I
    L.pyc_kernel_benchmark_update_symbol.argtypes = [S, I, S, C.c_double]
    L.pyc_kernel_benchmark_update_symbol.restype = I
    L.pyc_kernel_benchmark_update.argtypes = [S, I, C.c_double]
    L.pyc_kernel_benchmark_update.restype = I
    L.pyc_kernel_benchmark_read.argtypes = [S, I, C.POINTER(abi.KernelBenchmark)]
    L.pyc_kernel_benchmark_read.restype = None
    L.pyc_kernel_collect.argtypes = [S, I, C.POINTER(abi.KernelDesc), Z]
    L.pyc_kernel_collect.restype = Z
    L.pyc_kernel_hardware_family_name.argtypes = [I]
    L.pyc_kernel_hardware_family_name.restype = C.c_char_p
    L.pyc_kernel_workload_family_name.argtypes = [I]
    L.pyc_kernel_workload_family_name.restype = C.c_char_p


def lib() -> C.CDLL:
    """The loaded product library; raises PycError when it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PycError(f"libpyc_amd.so is not built ({LIB_PATH}); run python -m pyc_amd.build")
        L = C.CDLL(LIB_PATH)  # RTLD_LOCAL: never interposes other libraries
        _declare(L)
        _lib = L
    return _lib


def _b(s: str) -> bytes:
    return s.encode()


def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _stream(stream) -> int:
    if stream is not None:
        return int(stream)
    import torch
    return int(torch.cuda.current_stream().cuda_stream)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise PycError(f"{what} failed with status {rc}")


def gemm(symbol: str, a, b, c, M: int, N: int, K: int, alpha: float = 1.0, beta: float = 0.0,
         bias=None, epilogue: int = 0, stream=None) -> None:
    """C = epi(alpha*A*op(B) + beta*C) through pyc_hip_gemm_dispatch (device tensors)."""
    _check(lib().pyc_hip_gemm_dispatch(_b(symbol), M, N, K, _ptr(a), _ptr(b), _ptr(c), alpha, beta,
                                       _ptr(bias), epilogue, _stream(stream)), f"gemm {symbol}")


def attention(symbol: str, q, k, v, o, causal: bool, scale: float, stream=None) -> None:
    B, H, S, D = q.shape
    _check(lib().pyc_hip_attention_dispatch(_b(symbol), B, H, S, D, int(causal), _ptr(q), _ptr(k),
                                            _ptr(v), _ptr(o), scale, _stream(stream)),
           f"attention {symbol}")


def conv2d(symbol: str, x, w, y, pad=(1, 1), stride=(1, 1), bias=None, relu: bool = False,
           stream=None) -> None:
    N, H, W, Cin = x.shape
    K, R, S, _ = w.shape
    _check(lib().pyc_hip_conv2d_dispatch(_b(symbol), N, H, W, Cin, K, R, S, pad[0], pad[1],
                                         stride[0], stride[1], _ptr(x), _ptr(w), _ptr(bias),
                                         int(relu), _ptr(y), _stream(stream)), f"conv2d {symbol}")


def w8a16_gemm(x, wq, scale, y, relu: bool, stream=None,
               symbol: str = "hip_gemm_w8a16_e4m3") -> None:
    M, K = x.shape
    N = wq.shape[0]
    _check(lib().pyc_hip_w8a16_gemm_dispatch(_b(symbol), M, N, K, _ptr(x), _ptr(wq), _ptr(scale),
                                             int(relu), _ptr(y), _stream(stream)), "w8a16 gemm")


def _chain_arrays(layers):
    n = len(layers)
    wq = (C.c_void_p * n)(*[_ptr(w) for w, _, _ in layers])
    sc = (C.c_void_p * n)(*[_ptr(s) for _, s, _ in layers])
    N = (C.c_int * n)(*[int(w.shape[0]) for w, _, _ in layers])
    K = (C.c_int * n)(*[int(w.shape[1]) for w, _, _ in layers])
    relu = (C.c_int * n)(*[int(bool(r)) for _, _, r in layers])
    return n, wq, sc, N, K, relu


def w8a16_chain(x, layers, y, stream=None, symbol: str = "hip_w8a16_chain_e4m3") -> None:
    """The whole chain x -> layers -> y in one launch. layers: [(wq [N,K] uint8
    e4m3, scale [N] fp32, relu bool), ...], each K equal to the previous N."""
    n, wq, sc, N, K, relu = _chain_arrays(layers)
    _check(lib().pyc_hip_w8a16_chain_dispatch(_b(symbol), int(x.shape[0]), n, _ptr(x), C.cast(wq, C.c_void_p),
                                              C.cast(sc, C.c_void_p), C.cast(N, C.c_void_p), C.cast(K, C.c_void_p),
                                              C.cast(relu, C.c_void_p), _ptr(y), _stream(stream)), "w8a16 chain")


def w8a16_chain_reserve(M: int, layers) -> None:
    """Allocates the chain workspace (call before capturing a chain launch)."""
    n, _, _, N, K, _ = _chain_arrays(layers)
    _check(lib().pyc_hip_w8a16_chain_reserve(M, n, C.cast(N, C.c_void_p), C.cast(K, C.c_void_p)),
           "w8a16 chain reserve")


def w8a16_chain_error(clear: bool = True) -> int:
    """1 if a chain launch timed out waiting (output invalid), else 0."""
    return lib().pyc_hip_w8a16_chain_error(int(clear))


def _elt_suffix(t) -> str:
    import torch
    return {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[t.dtype]


def gelu(x, y, stream=None) -> None:
    """y = GELU(x), exact erf form, elementwise (same dtype and element count)."""
    _check(lib().pyc_hip_gelu_dispatch(_b("hip_gelu_" + _elt_suffix(x)), x.numel(), _ptr(x), _ptr(y),
                                       _stream(stream)), "gelu")


def layernorm(x, y, gamma=None, beta=None, eps: float = 1e-5, stream=None) -> None:
    """y = LayerNorm(x) over the last dimension, optional gamma/beta [D] of x's type."""
    D = x.shape[-1]
    _check(lib().pyc_hip_layernorm_dispatch(_b("hip_layernorm_" + _elt_suffix(x)), x.numel() // D, D, eps,
                                            _ptr(x), _ptr(gamma) if gamma is not None else None,
                                            _ptr(beta) if beta is not None else None, _ptr(y),
                                            _stream(stream)), "layernorm")


def device_info() -> abi.DeviceInfo:
    info = abi.DeviceInfo()
    _check(lib().pyc_hip_device_query(C.byref(info)), "device query")
    return info


def kernel_resources(symbol: str) -> abi.KernelResources:
    """The registered LDS / waves-per-SIMD figures of the kernel a symbol
    launches, and (with a device) the loaded code object's own figures."""
    r = abi.KernelResources()
    _check(lib().pyc_hip_kernel_resources_query(_b(symbol), C.byref(r)), f"kernel resources {symbol}")
    return r


def _tune_out(n, names, ms):
    return [(names[i * 64:(i + 1) * 64].split(b"\0", 1)[0].decode(), ms[i]) for i in range(max(n, 0))]


def autotune_gemm(dtype: int, M: int, N: int, K: int, iters: int = 10):
    """pyc_hip_autotune_gemm: [(symbol, median ms)] of every timed variant."""
    names = C.create_string_buffer(64 * 16)
    ms = (C.c_double * 16)()
    n = lib().pyc_hip_autotune_gemm(dtype, M, N, K, iters, names, 64, ms, 16)
    if n < 0:
        raise PycError(f"autotune gemm failed with status {n}")
    return _tune_out(n, names.raw, ms)


def autotune_conv2d(dtype: int, N: int, H: int, W: int, C_in: int, K: int, R: int, S: int, pad=(1, 1),
                    stride=(1, 1), iters: int = 10):
    """pyc_hip_autotune_conv2d: [(symbol, median ms)] of every timed conv path."""
    names = C.create_string_buffer(64 * 16)
    ms = (C.c_double * 16)()
    n = lib().pyc_hip_autotune_conv2d(dtype, N, H, W, C_in, K, R, S, pad[0], pad[1], stride[0], stride[1], iters,
                                      names, 64, ms, 16)
    if n < 0:
        raise PycError(f"autotune conv2d failed with status {n}")
    return _tune_out(n, names.raw, ms)

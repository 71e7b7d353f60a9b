"""The compiler-next run path from Python: pyc_compile_model / pyc_run_model of
libpyc_amd.so over its C-ABI (include/pyc/compiler_api.h), with tensors in
host memory (numpy) or device memory (torch tensors on a HIP device).

This mirrors how the reference's own bench driver calls the engine
(reference benchmark/benchmarks/gpu/workloads/pyc_compiler_next_bench.c:
compile once, then pyc_run_model per iteration with pyc_run_stats), and
`run_stats_json` emits the same fields that driver prints (its lines
1166-1249), so a result can be compared with the reference's JSON field for
field.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import abi
from . import lib as _product_lib

P, Z = C.c_void_p, C.c_size_t


def _declare(L: C.CDLL) -> C.CDLL:
    L.pyc_compile_model.argtypes = [C.POINTER(abi.ModelDesc), C.POINTER(abi.CompileOptions), C.POINTER(P)]
    L.pyc_compile_model.restype = C.c_int
    L.pyc_run_model.argtypes = [P, C.POINTER(abi.Tensor), Z, C.POINTER(abi.Tensor), Z, C.POINTER(abi.RunStats)]
    L.pyc_run_model.restype = C.c_int
    L.pyc_destroy_model.argtypes = [P]
    L.pyc_destroy_model.restype = None
    L.pyc_model_last_decision_log.argtypes = [P]
    L.pyc_model_last_decision_log.restype = C.c_char_p
    L.pyc_runtime_rails_default.argtypes = [C.POINTER(abi.RuntimeRails)]
    L.pyc_runtime_rails_default.restype = None
    L.pyc_status_string.argtypes = [C.c_int]
    L.pyc_status_string.restype = C.c_char_p
    return L


def op(kind: int, name: str = "", dims=(), inputs=(), dtype: int = abi.DTYPE_F32) -> abi.IrOp:
    o = abi.IrOp()
    o.kind = kind
    o.name = name.encode()
    o.dtype = dtype
    o.shape = abi.make_shape(dims)
    for i, x in enumerate(inputs):
        o.input_ids[i] = x
    o.input_count = len(inputs)
    return o


def host_tensor(arr: np.ndarray, dtype: int) -> abi.Tensor:
    """pyc_tensor over a numpy array (the caller keeps the array alive)."""
    t = abi.Tensor()
    t.data = arr.ctypes.data
    t.size_bytes = arr.nbytes
    t.dtype = dtype
    t.shape = abi.make_shape(arr.shape)
    return t


def device_tensor(x, dtype: int) -> abi.Tensor:
    """pyc_tensor over a torch tensor in device memory (bound to the plan in
    place by the HIP backend: no staging copies)."""
    t = abi.Tensor()
    t.data = x.data_ptr()
    t.size_bytes = x.numel() * x.element_size()
    t.dtype = dtype
    t.shape = abi.make_shape(tuple(x.shape))
    return t


class Model:
    """One compiled module (pyc_compile_model) and its run calls."""

    def __init__(self, ops, backend: int = abi.BACKEND_CUDA, fusion: int = 0, **options):
        self.L = _declare(_product_lib())
        self.module = abi.IrModule()
        for i, o in enumerate(ops):
            self.module.ops[i] = o
        self.module.op_count = len(ops)
        desc = abi.ModelDesc()
        desc.module = C.pointer(self.module)
        desc.backend = backend
        self.options = abi.CompileOptions()
        self.options.enable_fusion = fusion
        self.options.enable_memory_reuse = 1
        self.options.objective_mode = abi.MODE_BALANCED
        self.options.target_utilization_floor = 0.70
        self.options.deterministic_strict = 1
        self.L.pyc_runtime_rails_default(C.byref(self.options.rails))
        for k, v in options.items():
            setattr(self.options, k, v)
        self.handle = P()
        self.status = self.L.pyc_compile_model(C.byref(desc), C.byref(self.options), C.byref(self.handle))

    def run(self, inputs, outputs):
        """pyc_run_model; inputs/outputs are abi.Tensor lists. Returns (status, RunStats)."""
        ins = (abi.Tensor * len(inputs))(*inputs)
        outs = (abi.Tensor * len(outputs))(*outputs)
        stats = abi.RunStats()
        rc = self.L.pyc_run_model(self.handle, ins, len(inputs), outs, len(outputs), C.byref(stats))
        return rc, stats

    def bind(self, inputs, outputs):
        """pyc_run_model on fixed tensor lists, with the argument arrays built
        once: returns a function that runs the model and returns
        (status, RunStats), as run() does."""
        ins = (abi.Tensor * len(inputs))(*inputs)
        outs = (abi.Tensor * len(outputs))(*outputs)
        n_in, n_out, fn, h = len(inputs), len(outputs), self.L.pyc_run_model, self.handle

        def call():
            stats = abi.RunStats()
            return fn(h, ins, n_in, outs, n_out, C.byref(stats)), stats

        return call

    def decision_log(self) -> str:
        return self.L.pyc_model_last_decision_log(self.handle).decode()

    def close(self) -> None:
        if self.handle:
            self.L.pyc_destroy_model(self.handle)
            self.handle = P()


def _s(b: bytes) -> str:
    return b.decode(errors="replace")


def _env_true(name: str, default: bool) -> bool:
    v = os.environ.get(name)
    if v is None or v == "":
        return default
    return v not in ("0", "false", "False", "off")


def run_stats_json(stats_list, wall_ms, model: Model) -> dict:
    """The reference bench driver's per-run fields (pyc_compiler_next_bench.c
    1166-1249) from a list of RunStats and the matching pyc_run_model wall
    times in ms: latency statistics, the per-phase profile means, controller
    state, execution path, kernel selection, compile options and
    reliability/phantom-graph counters of the last run."""
    w = np.asarray(wall_ms, dtype=np.float64)
    last = stats_list[-1]
    n = float(len(stats_list))
    mean = lambda f: float(sum(getattr(s, f) for s in stats_list) / n)  # noqa: E731
    o = model.options
    return {
        "latency_ms": {"mean": float(w.mean()), "p50": float(np.percentile(w, 50)), "p95": float(np.percentile(w, 95)),
                       "min": float(w.min()), "max": float(w.max())},
        "peak_memory_bytes": int(last.peak_bytes),
        "profile": {"dispatch_ms_mean": mean("dispatch_ms"), "graph_exec_ms_mean": mean("graph_exec_ms"),
                    "controller_ms_mean": mean("controller_ms"), "kernel_select_ms_mean": mean("kernel_select_ms"),
                    "cuda_copy_in_ms": mean("cuda_copy_in_ms"), "cuda_kernel_ms": mean("cuda_kernel_ms"),
                    "cuda_copy_out_ms": mean("cuda_copy_out_ms"), "cuda_sync_ms": mean("cuda_sync_ms")},
        "controller": {"active_mode": int(last.active_mode), "shadow_mode": int(last.shadow_mode),
                       "shadow_reason": int(last.shadow_reason), "rollback_reason": int(last.rollback_reason),
                       "rollback_count": int(last.rollback_count)},
        "execution_path": _s(last.execution_path),
        "kernel_selection": {"count": int(last.selected_kernel_count),
                             "candidates": int(last.selected_kernel_candidates),
                             "symbol": _s(last.selected_kernel_symbol)},
        "compile_options": {"enable_fusion": bool(o.enable_fusion), "enable_memory_reuse": bool(o.enable_memory_reuse),
                            "enable_autotune": bool(o.enable_autotune),
                            "objective_mode": int(o.objective_mode),
                            "deterministic_strict": bool(o.deterministic_strict)},
        "reliability": {"compile_cache_hit": int(last.compile_cache_hit),
                        "compile_budget_exceeded": int(last.compile_budget_exceeded),
                        "guard_miss_count": int(last.guard_miss_count), "fallback_count": int(last.fallback_count),
                        "graph_break_count": int(last.graph_break_count),
                        "compilability_score": float(last.compilability_score),
                        "autotune_loaded": int(last.autotune_loaded), "autotune_saved": int(last.autotune_saved),
                        "rematerialized_tensors": int(last.rematerialized_tensors),
                        "rematerialized_bytes": int(last.rematerialized_bytes)},
        "phantom_graph": {"enabled": bool(last.phantom_graph_enabled), "match": bool(last.phantom_graph_match),
                          "match_count": int(last.phantom_graph_match_count),
                          "mismatch_count": int(last.phantom_graph_mismatch_count)},
        "precision_policy": {"allow_tf32": _env_true("PYC_CUDA_ALLOW_TF32", True),
                             "assume_static_lhs": _env_true("PYC_CUDA_ASSUME_STATIC_LHS", False),
                             "assume_static_rhs": _env_true("PYC_CUDA_ASSUME_STATIC_RHS", False),
                             "skip_host_output_copy": _env_true("PYC_CUDA_SKIP_HOST_OUTPUT_COPY", False)},
    }

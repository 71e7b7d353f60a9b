"""ctypes helpers to drive either engine library through the same C-ABI:
libpyc_amd.so (the product) or oracle/_ref/libpyc_ref.so (the reference's
own engine, the checker). Both export the same names; each is loaded
RTLD_LOCAL and linked -Bsymbolic, so neither interposes the other."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from pyc_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libpyc_ref.so")

P, I, Z, D = C.c_void_p, C.c_int, C.c_size_t, C.c_double


def declare(L):
    L.pyc_ir_module_init.argtypes = [C.POINTER(abi.IrModule)]
    L.pyc_ir_add_op.argtypes = [C.POINTER(abi.IrModule), C.POINTER(abi.IrOp)]
    L.pyc_ir_verify.argtypes = [C.POINTER(abi.IrModule), C.POINTER(abi.IrDiagnostic)]
    L.pyc_ir_serialize.argtypes = [C.POINTER(abi.IrModule), C.c_char_p, Z]
    L.pyc_pass_pipeline_default.argtypes = [P]
    L.pyc_pass_pipeline_run.argtypes = [P, C.POINTER(abi.IrModule), P]
    L.pyc_alloc_plan_init.argtypes = [P]
    L.pyc_alloc_plan_add_request.argtypes = [P, AllocRequest]
    L.pyc_alloc_plan_build_with_mode.argtypes = [P, I, Z]
    L.pyc_alloc_plan_stats.argtypes = [P, P]
    L.pyc_runtime_rails_default.argtypes = [C.POINTER(abi.RuntimeRails)]
    L.pyc_runtime_controller_init.argtypes = [P, I]
    L.pyc_runtime_controller_observe.argtypes = [P, C.POINTER(abi.RuntimeRails), P, C.POINTER(C.c_int),
                                                 C.POINTER(C.c_int)]
    L.pyc_kernel_registry_reset.argtypes = []
    L.pyc_kernel_register.argtypes = [C.POINTER(abi.KernelDesc)]
    L.pyc_kernel_select.argtypes = [C.c_char_p, I, C.POINTER(abi.KernelDesc)]
    L.pyc_kernel_select_with_policy.argtypes = [C.c_char_p, I, I, D, C.POINTER(abi.KernelDesc),
                                                C.POINTER(abi.KernelSelectionTrace)]
    L.pyc_kernel_coselect_with_context.argtypes = [C.c_char_p, I, I, C.POINTER(abi.CoselectContext),
                                                   C.POINTER(abi.KernelDesc), C.POINTER(abi.KernelSelectionTrace)]
    L.pyc_kernel_promote_symbol.argtypes = [C.c_char_p, I, C.c_char_p]
    L.pyc_kernel_promoted_symbol.argtypes = [C.c_char_p, I, C.c_char_p, Z]
    L.pyc_kernel_benchmark_update.argtypes = [C.c_char_p, I, D]
    L.pyc_kernel_benchmark_update_symbol.argtypes = [C.c_char_p, I, C.c_char_p, D]
    L.pyc_kernel_benchmark_read.argtypes = [C.c_char_p, I, C.POINTER(abi.KernelBenchmark)]
    L.pyc_kernel_collect.argtypes = [C.c_char_p, I, C.POINTER(abi.KernelDesc), Z]
    L.pyc_kernel_collect.restype = Z
    L.pyc_compile_model.argtypes = [C.POINTER(abi.ModelDesc), C.POINTER(abi.CompileOptions), C.POINTER(P)]
    L.pyc_run_model.argtypes = [P, C.POINTER(abi.Tensor), Z, C.POINTER(abi.Tensor), Z, C.POINTER(abi.RunStats)]
    L.pyc_destroy_model.argtypes = [P]
    L.pyc_model_last_decision_log.argtypes = [P]
    L.pyc_model_last_decision_log.restype = C.c_char_p
    L.pyc_status_string.argtypes = [I]
    L.pyc_status_string.restype = C.c_char_p
    return L


class AllocRequest(C.Structure):
    _fields_ = [("tensor_id", C.c_int), ("size_bytes", C.c_size_t), ("alignment", C.c_size_t),
                ("start_step", C.c_int), ("end_step", C.c_int)]


class AllocPlan(C.Structure):
    _fields_ = [("requests", AllocRequest * 2048), ("request_count", C.c_size_t), ("offsets", C.c_size_t * 2048),
                ("peak_bytes", C.c_size_t), ("reused_allocations", C.c_size_t), ("allocation_events", C.c_size_t),
                ("overlap_pairs_observed", C.c_size_t), ("largest_allocation_bytes", C.c_size_t),
                ("rematerialized_tensors", C.c_size_t), ("rematerialized_bytes", C.c_size_t),
                ("pressure_events", C.c_size_t), ("pressure_score", C.c_double)]


class AllocStats(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in ("peak_bytes", "total_requested_bytes", "reused_allocations",
                                          "allocation_events", "overlap_pairs_observed", "largest_allocation_bytes",
                                          "rematerialized_tensors", "rematerialized_bytes", "pressure_events")] + \
               [("pressure_score", C.c_double)]


class WindowMetrics(C.Structure):
    _fields_ = [("baseline_p95_ms", D), ("observed_p95_ms", D), ("baseline_throughput", D),
                ("observed_throughput", D), ("pressure_score", D), ("pressure_events", Z),
                ("rematerialized_tensors", Z), ("runtime_error", I)]


class Controller(C.Structure):
    _fields_ = [("current_mode", I), ("recommended_mode", I), ("recommendation_reason", I),
                ("last_stable_mode", I), ("last_rollback_reason", I), ("rollback_count", Z),
                ("steps_in_mode", Z), ("cooldown_remaining", Z), ("consecutive_breaches", Z)]


class PassConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("canonicalize", "shape_inference", "layout_propagation", "fusion",
                                       "liveness", "allocation", "lowering")]


class PassReport(C.Structure):
    _fields_ = [("passes_run", I), ("warnings", I), ("errors", I), ("transformed_ops", I), ("fused_patterns", I),
                ("inferred_shapes", I), ("peak_live_values", Z), ("graph_break_count", Z),
                ("graph_break_const_count", Z), ("graph_break_gelu_count", Z), ("graph_break_reduce_sum_count", Z),
                ("graph_break_layernorm_count", Z), ("graph_break_unknown_count", Z),
                ("first_graph_break_op_id", I), ("first_graph_break_op_name", C.c_char * 64),
                ("compilability_score", D), ("graph_break_summary", C.c_char * 128),
                ("speculative_plan_count", Z), ("speculative_confidence", D),
                ("speculative_shape_bucket", C.c_char * 64), ("phantom_confidence", D),
                ("phantom_shape_bucket", C.c_char * 64), ("phantom_shape_signature", C.c_char * 128)]


_libs = {}


def mine():
    if "mine" not in _libs:
        import pyc_amd
        _libs["mine"] = declare(pyc_amd.lib())
    return _libs["mine"]


def ref():
    if "ref" not in _libs:
        _libs["ref"] = declare(C.CDLL(REF_LIB))
    return _libs["ref"]


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


# The reference's own engine driving this repository's backend: the
# reference's engine sources built into one library linked to
# libpyc_amd_backend.so (oracle/Makefile.ref), whose registry calls bind to
# the reference's registry.
REF_HIP_LIB = os.path.join(ROOT, "oracle", "_ref", "libpyc_ref_hip.so")
BACKEND_LIB = os.path.join(ROOT, "pyc_amd", "lib", "libpyc_amd_backend.so")


def ref_on_hip():
    if "ref_hip" not in _libs:
        _libs["ref_hip"] = declare(C.CDLL(REF_HIP_LIB))
    return _libs["ref_hip"]


def ref_on_hip_available() -> bool:
    return os.path.exists(REF_HIP_LIB) and os.path.exists(BACKEND_LIB)


def op(kind, name="", dims=(), inputs=(), dtype=abi.DTYPE_F32):
    o = abi.IrOp()
    o.kind = kind
    o.name = name.encode()
    o.dtype = dtype
    o.shape = abi.make_shape(dims)
    for i, x in enumerate(inputs):
        o.input_ids[i] = x
    o.input_count = len(inputs)
    return o


def module(ops):
    m = abi.IrModule()
    for i, o in enumerate(ops):
        m.ops[i] = o
    m.op_count = len(ops)
    return m


def serialize(L, m) -> str:
    buf = C.create_string_buffer(1 << 16)
    rc = L.pyc_ir_serialize(C.byref(m), buf, len(buf))
    return buf.value.decode() if rc == 0 else None


def tensor(arr, dtype=abi.DTYPE_F32):
    t = abi.Tensor()
    t.data = arr.ctypes.data
    t.size_bytes = arr.nbytes
    t.dtype = dtype
    t.shape = abi.make_shape(arr.shape)
    return t


def options(L, fusion=0, **kw):
    o = abi.CompileOptions()
    o.enable_fusion = fusion
    o.enable_memory_reuse = 1
    o.objective_mode = abi.MODE_BALANCED
    o.target_utilization_floor = 0.70
    o.deterministic_strict = 1
    L.pyc_runtime_rails_default(C.byref(o.rails))
    for k, v in kw.items():
        setattr(o, k, v)
    return o


class Model:
    def __init__(self, L, ops, backend=abi.BACKEND_CPU, **opt):
        self.L = L
        self.m = module(ops)
        desc = abi.ModelDesc()
        desc.module = C.pointer(self.m)
        desc.backend = backend
        self.opts = options(L, **opt)
        self.h = C.c_void_p()
        self.status = L.pyc_compile_model(C.byref(desc), C.byref(self.opts), C.byref(self.h))

    def run(self, inputs, out_shapes, in_dtypes=None, out_dtypes=None, out_np_dtype=np.float32):
        in_dtypes = in_dtypes or [abi.DTYPE_F32] * len(inputs)
        out_dtypes = out_dtypes or [abi.DTYPE_F32] * len(out_shapes)
        ins = (abi.Tensor * len(inputs))(*[tensor(a, d) for a, d in zip(inputs, in_dtypes)])
        self.outs = [np.zeros(s, out_np_dtype) for s in out_shapes]
        outs = (abi.Tensor * len(self.outs))(*[tensor(a, d) for a, d in zip(self.outs, out_dtypes)])
        stats = abi.RunStats()
        st = self.L.pyc_run_model(self.h, ins, len(inputs), outs, len(self.outs), C.byref(stats))
        return st, self.outs, stats

    def log(self):
        return self.L.pyc_model_last_decision_log(self.h).decode()

    def close(self):
        if self.h:
            self.L.pyc_destroy_model(self.h)
            self.h = C.c_void_p()


def log_fields(text: str) -> dict:
    out = {}
    for tok in text.split():
        if "=" in tok:
            k, v = tok.split("=", 1)
            out[k] = v
    return out

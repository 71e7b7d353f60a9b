"""ctypes mirrors of the C-ABI in include/pyc/*.h.

The struct layouts follow the headers field for field (which mirror the
reference's include/pyc/*.h); tests/test_abi.py checks their sizes against the
C compiler's view.
"""
from __future__ import annotations

import ctypes as C

IR_MAX_DIMS = 8
IR_MAX_OPS = 1024
IR_MAX_INPUTS = 8
IR_MAX_NAME = 64
KERNEL_OP_KEY_MAX = 64
KERNEL_SYMBOL_MAX = 128
CUDA_REASON_MAX = 128

# pyc_dtype (include/pyc/ir.h)
DTYPE_UNKNOWN, DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I32, DTYPE_I8, DTYPE_FP8_E4M3 = range(7)
DTYPE_BYTES = {DTYPE_F32: 4, DTYPE_F16: 2, DTYPE_BF16: 2, DTYPE_I32: 4, DTYPE_I8: 1, DTYPE_FP8_E4M3: 1}

# pyc_ir_op_kind
(OP_INPUT, OP_CONST, OP_MATMUL, OP_ADD, OP_RELU, OP_GELU, OP_REDUCE_SUM, OP_LAYERNORM,
 OP_OUTPUT, OP_CONV2D, OP_ATTENTION) = range(11)

# pyc_backend / families / modes / statuses
BACKEND_CPU, BACKEND_CUDA = 0, 1
HW_ANY, HW_GENERIC, HW_ADA, HW_HOPPER, HW_CDNA4 = range(5)
(WL_ANY, WL_SMALL, WL_SQUARE, WL_LARGE_SQUARE, WL_TALL_SKINNY, WL_WIDE_SKINNY) = range(6)
MODE_BALANCED, MODE_MEMORY_FIRST, MODE_UTILIZATION_FIRST = range(3)
STATUS_OK, STATUS_INVALID_ARGUMENT, STATUS_VERIFY_FAILED, STATUS_COMPILE_FAILED, STATUS_RUNTIME_FAILED = range(5)
DISPATCH_OK, DISPATCH_FALLBACK, DISPATCH_ERROR = range(3)
EPI_NONE, EPI_BIAS, EPI_RELU = 0, 1, 2


class Shape(C.Structure):
    _fields_ = [("rank", C.c_size_t), ("dims", C.c_int64 * IR_MAX_DIMS)]


class IrOp(C.Structure):
    _fields_ = [
        ("kind", C.c_int),
        ("name", C.c_char * IR_MAX_NAME),
        ("dtype", C.c_int),
        ("shape", Shape),
        ("input_ids", C.c_int * IR_MAX_INPUTS),
        ("input_count", C.c_size_t),
    ]


class IrModule(C.Structure):
    _fields_ = [("ops", IrOp * IR_MAX_OPS), ("op_count", C.c_size_t)]


class IrDiagnostic(C.Structure):
    _fields_ = [("code", C.c_int), ("message", C.c_char * 256)]


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("size_bytes", C.c_size_t), ("dtype", C.c_int), ("shape", Shape)]


class KernelDesc(C.Structure):
    _fields_ = [
        ("op_key", C.c_char * KERNEL_OP_KEY_MAX),
        ("backend", C.c_int),
        ("symbol", C.c_char * KERNEL_SYMBOL_MAX),
        ("priority", C.c_int),
        ("estimated_occupancy", C.c_double),
        ("tensor_core_eligible", C.c_int),
        ("shared_mem_bytes", C.c_size_t),
        ("reg_pressure_class", C.c_int),
        ("preferred_workload_family", C.c_int),
        ("preferred_hardware_family", C.c_int),
    ]


class KernelBenchmark(C.Structure):
    _fields_ = [("selected", C.c_int), ("considered", C.c_int), ("best_time_ms", C.c_double)]


class KernelSelectionTrace(C.Structure):
    _fields_ = [
        ("selected_score", C.c_double),
        ("selected_estimated_utilization", C.c_double),
        ("pressure_penalty", C.c_double),
        ("allocator_penalty", C.c_double),
        ("reuse_bonus", C.c_double),
        ("candidates_considered", C.c_size_t),
    ]


class CoselectContext(C.Structure):
    _fields_ = [
        ("pressure_score", C.c_double),
        ("pressure_events", C.c_size_t),
        ("rematerialized_tensors", C.c_size_t),
        ("reused_allocations", C.c_size_t),
        ("total_requested_bytes", C.c_size_t),
        ("peak_bytes", C.c_size_t),
        ("memory_budget_bytes", C.c_size_t),
        ("workload_family", C.c_int),
        ("hardware_family", C.c_int),
    ]


class RuntimeRails(C.Structure):
    _fields_ = [
        ("enable_auto_switch", C.c_int),
        ("enable_hard_rollback", C.c_int),
        ("dwell_steps", C.c_size_t),
        ("cooldown_steps", C.c_size_t),
        ("consecutive_breach_windows", C.c_size_t),
        ("latency_regression_threshold", C.c_double),
        ("throughput_regression_threshold", C.c_double),
        ("pressure_score_threshold", C.c_double),
        ("pressure_events_threshold", C.c_size_t),
        ("rematerialized_tensors_threshold", C.c_size_t),
    ]


class DistributedOptions(C.Structure):
    _fields_ = [
        ("enabled", C.c_int),
        ("backend", C.c_int),
        ("strategy", C.c_int),
        ("world_size", C.c_int),
        ("rank", C.c_int),
        ("local_rank", C.c_int),
        ("backend_path", C.c_char_p),
        ("config_json", C.c_char_p),
    ]


class CompileOptions(C.Structure):
    _fields_ = [
        ("enable_fusion", C.c_int),
        ("enable_memory_reuse", C.c_int),
        ("enable_autotune", C.c_int),
        ("enable_speculative_plans", C.c_int),
        ("enable_phantom_graph", C.c_int),
        ("max_speculative_plans", C.c_size_t),
        ("phantom_horizon_steps", C.c_size_t),
        ("objective_mode", C.c_int),
        ("memory_budget_bytes", C.c_size_t),
        ("target_utilization_floor", C.c_double),
        ("deterministic_strict", C.c_int),
        ("compile_budget_ms", C.c_double),
        ("cache_mode", C.c_int),
        ("autotune_db_path", C.c_char_p),
        ("rails", RuntimeRails),
        ("distributed", DistributedOptions),
    ]


class ModelDesc(C.Structure):
    _fields_ = [("module", C.POINTER(IrModule)), ("backend", C.c_int)]


class DispatchTrace(C.Structure):
    _fields_ = [
        ("cuda_requested", C.c_int),
        ("cuda_available", C.c_int),
        ("fallback_to_cpu", C.c_int),
        ("graph_replayed", C.c_int),
        ("copy_in_ms", C.c_double),
        ("kernel_ms", C.c_double),
        ("copy_out_ms", C.c_double),
        ("sync_ms", C.c_double),
        ("reason", C.c_char * CUDA_REASON_MAX),
    ]


class RunStats(C.Structure):
    _fields_ = [
        ("compile_ms", C.c_double),
        ("run_ms", C.c_double),
        ("peak_bytes", C.c_size_t),
        ("total_requested_bytes", C.c_size_t),
        ("reused_allocations", C.c_size_t),
        ("rematerialized_tensors", C.c_size_t),
        ("rematerialized_bytes", C.c_size_t),
        ("pressure_events", C.c_size_t),
        ("pressure_score", C.c_double),
        ("selected_kernel_score", C.c_double),
        ("selected_kernel_allocator_penalty", C.c_double),
        ("selected_kernel_reuse_bonus", C.c_double),
        ("estimated_utilization", C.c_double),
        ("active_mode", C.c_int),
        ("rollback_reason", C.c_int),
        ("rollback_count", C.c_size_t),
        ("shadow_mode", C.c_int),
        ("shadow_reason", C.c_int),
        ("workload_family", C.c_char * 32),
        ("hardware_family", C.c_char * 32),
        ("selected_kernel_count", C.c_int),
        ("selected_kernel_candidates", C.c_size_t),
        ("selected_kernel_symbol", C.c_char * KERNEL_SYMBOL_MAX),
        ("execution_path", C.c_char * 128),
        ("dispatch_ms", C.c_double),
        ("graph_exec_ms", C.c_double),
        ("controller_ms", C.c_double),
        ("kernel_select_ms", C.c_double),
        ("cuda_copy_in_ms", C.c_double),
        ("cuda_kernel_ms", C.c_double),
        ("cuda_copy_out_ms", C.c_double),
        ("cuda_sync_ms", C.c_double),
        ("deterministic_contract_enforced", C.c_int),
        ("deterministic_contract_ok", C.c_int),
        ("model_fingerprint", C.c_uint64),
        ("deterministic_contract_reason", C.c_char * 64),
        ("compile_cache_hit", C.c_int),
        ("compile_budget_exceeded", C.c_int),
        ("guard_miss_count", C.c_size_t),
        ("fallback_count", C.c_size_t),
        ("graph_break_count", C.c_size_t),
        ("graph_break_const_count", C.c_size_t),
        ("graph_break_gelu_count", C.c_size_t),
        ("graph_break_reduce_sum_count", C.c_size_t),
        ("graph_break_layernorm_count", C.c_size_t),
        ("graph_break_unknown_count", C.c_size_t),
        ("first_graph_break_op_id", C.c_int),
        ("first_graph_break_op_name", C.c_char * IR_MAX_NAME),
        ("compilability_score", C.c_double),
        ("autotune_loaded", C.c_int),
        ("autotune_saved", C.c_int),
        ("graph_break_summary", C.c_char * 128),
        ("speculative_plan_count", C.c_size_t),
        ("speculative_plan_hit", C.c_int),
        ("speculative_plan_miss_count", C.c_size_t),
        ("speculative_guard_miss_count", C.c_size_t),
        ("speculative_confidence", C.c_double),
        ("speculative_shape_bucket", C.c_char * 64),
        ("phantom_graph_enabled", C.c_int),
        ("phantom_graph_match", C.c_int),
        ("phantom_graph_match_count", C.c_size_t),
        ("phantom_graph_mismatch_count", C.c_size_t),
        ("phantom_graph_reshape_count", C.c_size_t),
        ("phantom_graph_confidence", C.c_double),
        ("phantom_graph_match_score", C.c_double),
        ("phantom_graph_expected_bucket", C.c_char * 64),
        ("phantom_graph_expected_signature", C.c_char * 128),
        ("phantom_graph_observed_signature", C.c_char * 128),
    ]


class DeviceInfo(C.Structure):
    _fields_ = [
        ("gcn_arch", C.c_char * 64),
        ("compute_units", C.c_int),
        ("clock_khz", C.c_int),
        ("memory_clock_khz", C.c_int),
        ("memory_bus_width", C.c_int),
        ("total_global_mem", C.c_size_t),
        ("lds_per_block", C.c_size_t),
        ("xcds", C.c_int),
    ]


class KernelResources(C.Structure):
    """pyc_hip_kernel_resources (pyc/hip_backend.h)."""
    _fields_ = [
        ("kernel", C.c_char * 64),
        ("lds_bytes", C.c_size_t),
        ("threads", C.c_int),
        ("waves_per_simd", C.c_int),
        ("device", C.c_int),
        ("attr_lds_bytes", C.c_size_t),
        ("attr_regs", C.c_int),
        ("attr_scratch_bytes", C.c_size_t),
        ("attr_max_threads", C.c_int),
        ("attr_blocks_per_cu", C.c_int),
    ]


CPU_EXECUTOR_FN = C.CFUNCTYPE(C.c_int, C.POINTER(IrModule), C.POINTER(Tensor), C.c_size_t,
                              C.POINTER(Tensor), C.c_size_t, C.c_void_p)


def make_shape(dims) -> Shape:
    s = Shape()
    s.rank = len(dims)
    for i, d in enumerate(dims):
        s.dims[i] = int(d)
    return s

"""Drive the reference's own C11 engine (oracle/_ref/libpyc_ref.so) through its
C-ABI. Test infrastructure: used to pin the oracle restatement against the
reference CPU executor. The library exists only where oracle/Makefile.ref was
run (it is built from /root/reference in the development container and travels
to the GPU box as a built file)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from pyc_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libpyc_ref.so")

_ref = None


def available() -> bool:
    return os.path.exists(REF_LIB)


def lib():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_LIB)
        L.pyc_compile_model.argtypes = [C.POINTER(abi.ModelDesc), C.POINTER(abi.CompileOptions),
                                        C.POINTER(C.c_void_p)]
        L.pyc_compile_model.restype = C.c_int
        L.pyc_run_model.argtypes = [C.c_void_p, C.POINTER(abi.Tensor), C.c_size_t,
                                    C.POINTER(abi.Tensor), C.c_size_t, C.POINTER(abi.RunStats)]
        L.pyc_run_model.restype = C.c_int
        L.pyc_destroy_model.argtypes = [C.c_void_p]
        L.pyc_runtime_rails_default.argtypes = [C.POINTER(abi.RuntimeRails)]
        L.pyc_model_last_decision_log.argtypes = [C.c_void_p]
        L.pyc_model_last_decision_log.restype = C.c_char_p
        _ref = L
    return _ref


def _op(kind, name, dims=(), inputs=(), dtype=abi.DTYPE_F32):
    op = abi.IrOp()
    op.kind = kind
    op.name = name.encode()
    op.dtype = dtype
    op.shape = abi.make_shape(dims)
    for i, x in enumerate(inputs):
        op.input_ids[i] = x
    op.input_count = len(inputs)
    return op


def module(ops):
    m = abi.IrModule()
    for i, op in enumerate(ops):
        m.ops[i] = op
    m.op_count = len(ops)
    return m


def tensor(arr: np.ndarray, dtype=abi.DTYPE_F32) -> abi.Tensor:
    t = abi.Tensor()
    t.data = arr.ctypes.data
    t.size_bytes = arr.nbytes
    t.dtype = dtype
    t.shape = abi.make_shape(arr.shape)
    return t


def options(fusion=0):
    o = abi.CompileOptions()
    o.enable_fusion = fusion
    o.enable_memory_reuse = 1
    o.objective_mode = abi.MODE_BALANCED
    o.target_utilization_floor = 0.70
    o.deterministic_strict = 1
    lib().pyc_runtime_rails_default(C.byref(o.rails))
    return o


class Model:
    """A compiled reference model; run() returns outputs and stats."""

    def __init__(self, ops, backend=abi.BACKEND_CPU, fusion=0):
        self.m = module(ops)
        desc = abi.ModelDesc()
        desc.module = C.pointer(self.m)
        desc.backend = backend
        self.opts = options(fusion)
        self.h = C.c_void_p()
        st = lib().pyc_compile_model(C.byref(desc), C.byref(self.opts), C.byref(self.h))
        assert st == abi.STATUS_OK, st

    def run(self, inputs, out_shapes):
        ins = (abi.Tensor * len(inputs))(*[tensor(a) for a in inputs])
        outs_np = [np.zeros(s, np.float32) for s in out_shapes]
        outs = (abi.Tensor * len(outs_np))(*[tensor(a) for a in outs_np])
        stats = abi.RunStats()
        st = lib().pyc_run_model(self.h, ins, len(inputs), outs, len(outs_np), C.byref(stats))
        return st, outs_np, stats

    def log(self) -> str:
        return lib().pyc_model_last_decision_log(self.h).decode()

    def close(self):
        if self.h:
            lib().pyc_destroy_model(self.h)
            self.h = C.c_void_p()


def matmul_model(m, k, n, bias=None, relu=False, backend=abi.BACKEND_CPU):
    ops = [_op(abi.OP_INPUT, "lhs", (m, k)), _op(abi.OP_INPUT, "rhs", (k, n))]
    cur = 2
    if bias is not None:
        ops.append(_op(abi.OP_INPUT, "bias", bias))
        cur = 3
    ops.append(_op(abi.OP_MATMUL, "matmul0", (), (0, 1)))
    mm = len(ops) - 1
    last = mm
    if bias is not None:
        ops.append(_op(abi.OP_ADD, "add0", (), (mm, 2)))
        last = len(ops) - 1
    if relu:
        ops.append(_op(abi.OP_RELU, "relu0", (), (last,)))
        last = len(ops) - 1
    ops.append(_op(abi.OP_OUTPUT, "out0", (m, n), (last,)))
    del cur
    return Model(ops, backend=backend)

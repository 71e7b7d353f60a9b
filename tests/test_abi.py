"""CPU checks of the C-ABI library: it loads, exports every function that
include/pyc/*.h declares, and its struct layouts match the ctypes mirrors."""
import ctypes as C
import os
import re
import subprocess

import pytest

import pyc_amd
from pyc_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include", "pyc")


# Headers whose every declaration the library implements.
HEADERS = sorted(f for f in os.listdir(INC) if f.endswith(".h"))


def declared_functions():
    names = set()
    for fn in HEADERS:
        text = open(os.path.join(INC, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text, flags=re.S)
        for mt in re.finditer(r"\b(pyc_\w+)\s*\(", text):
            names.add(mt.group(1))
    return sorted(names)


def test_library_loads():
    assert os.path.exists(pyc_amd.LIB_PATH)
    pyc_amd.lib()


def test_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", pyc_amd.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    assert len(declared_functions()) >= 45


STRUCTS = {
    "pyc_ir_op": abi.IrOp, "pyc_ir_module": abi.IrModule, "pyc_tensor": abi.Tensor,
    "pyc_kernel_desc": abi.KernelDesc, "pyc_compile_options": abi.CompileOptions,
    "pyc_run_stats": abi.RunStats, "pyc_cuda_dispatch_trace": abi.DispatchTrace,
    "pyc_kernel_coselect_context": abi.CoselectContext, "pyc_hip_device_info": abi.DeviceInfo,
}


def test_struct_layouts_match_headers(tmp_path):
    src = tmp_path / "sizes.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "pyc/cuda_backend.h"',
             '#include "pyc/hip_backend.h"', 'int main(void){']
    for name in STRUCTS:
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
    lines.append('printf("off_exec %zu\\n", offsetof(pyc_run_stats, execution_path));')
    lines.append('printf("off_phantom %zu\\n", offsetof(pyc_run_stats, phantom_graph_observed_signature));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for name, cls in STRUCTS.items():
        assert int(out[name]) == C.sizeof(cls), name
    assert int(out["off_exec"]) == abi.RunStats.execution_path.offset
    assert int(out["off_phantom"]) == abi.RunStats.phantom_graph_observed_signature.offset


def test_registry_registers_hip_variants():
    L = pyc_amd.lib()
    L.pyc_cutlass_registry_init()
    assert L.pyc_cutlass_kernel_count(b"matmul") >= pyc_amd.lib().pyc_hip_kernel_symbol_count(b"matmul")
    assert L.pyc_cutlass_kernel_count(b"attention") >= 4
    assert L.pyc_cutlass_kernel_count(b"conv2d") >= 4
    desc = abi.KernelDesc()
    assert L.pyc_kernel_select(b"matmul", abi.BACKEND_CUDA, C.byref(desc)) == 0
    assert desc.preferred_hardware_family == abi.HW_CDNA4 and desc.tensor_core_eligible == 1
    assert L.pyc_kernel_hardware_family_name(abi.HW_CDNA4) == b"cdna4"


def test_gpu_entry_points_refuse_without_device():
    """No HIP device here: argument errors still come back as -1 before any launch."""
    L = pyc_amd.lib()
    assert L.pyc_hip_gemm_dispatch(b"hip_gemm_bf16_nt", 0, 1, 1, None, None, None, 1.0, 0.0, None, 0, None) == -1
    assert L.pyc_hip_gemm_dispatch(b"unknown", 8, 8, 8, 1, 1, 1, 1.0, 0.0, None, 0, None) == -1
    assert L.pyc_hip_attention_dispatch(b"hip_attention_bf16", 1, 1, 16, 96, 1, 1, 1, 1, 1, 1.0, None) == -1
    assert L.pyc_hip_w8a16_gemm_dispatch(b"hip_gemm_w8a16_e4m3", 33, 8, 16, 1, 1, 1, 0, 1, None) == -1
    info = abi.DeviceInfo()
    if L.pyc_hip_device_query(C.byref(info)) != 0:
        pytest.skip("no device: device query reports -1 as documented")

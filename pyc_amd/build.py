"""Build recipe for libpyc_amd.so (gfx950 HIP kernels + C11 host engine).

Usage: ``python -m pyc_amd.build`` (or ``__graft_entry__.build()``).

* ``csrc/kernels/*.hip`` are compiled by hipcc for gfx950 only. Every HIP
  compile carries ``-Xclang -target-feature -Xclang -packed-fp32-ops`` so the
  compiler emits no packed-fp32 VALU instructions.
* ``csrc/host/*.c`` are compiled as C11 by gcc against the HIP runtime C API.
* Everything links into one in-tree shared library, ``pyc_amd/lib/libpyc_amd.so``,
  whose exported C-ABI is declared in ``include/pyc/*.h``.
* The same objects, without the engine (compiler_api, ir, pass_manager,
  runtime_allocator, runtime_control) and without the kernel registry, also
  link into ``pyc_amd/lib/libpyc_amd_backend.so``: the GPU backend alone, for
  a program that keeps its own engine (the reference's). Its registry calls
  (``pyc_kernel_register`` and the rest) are left undefined, so they bind to
  the registry of the program that loads it.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libpyc_amd.so")
BACKEND_LIB_PATH = os.path.join(LIB_DIR, "libpyc_amd_backend.so")
# host sources of the backend-only library: the dispatch, the kernel entry
# points and the op helpers the lowering uses
BACKEND_HOST = ("hip_backend.c", "hip_kernels.c", "cpu_ops.c")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wno-inline-asm",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]
C_FLAGS = [
    "-std=c11", "-O2", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Wno-stringop-truncation", "-Wno-format-truncation",
    "-D_POSIX_C_SOURCE=200809L", "-D_DEFAULT_SOURCE", "-D__HIP_PLATFORM_AMD__",
    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc", "host"),
    "-I", os.path.join(ROCM, "include"),
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _obj(src: str) -> str:
    base = os.path.relpath(src, os.path.join(HERE, "csrc")).replace(os.sep, "__")
    return os.path.join(OBJ_DIR, base + ".o")


def sources() -> tuple[list[str], list[str]]:
    hip = sorted(glob.glob(os.path.join(HERE, "csrc", "kernels", "*.hip")))
    c = sorted(glob.glob(os.path.join(HERE, "csrc", "host", "*.c")))
    return hip, c


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compile every source (always; this is the does-it-build check) and link."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    hip, c = sources()
    cmds = [[HIPCC, *HIP_FLAGS, "-c", s, "-o", _obj(s)] for s in hip]
    cmds += [["gcc", *C_FLAGS, "-c", s, "-o", _obj(s)] for s in c]
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH + ".tmp"
    # the full library resolves every symbol itself (-z defs: an entry point
    # missing from the sources fails the link, not a later load); the
    # backend-only one below takes the registry calls from the engine it is
    # loaded under
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
          *[_obj(s) for s in hip + c], "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
          "-lpthread", "-lm", "-Wl,-Bsymbolic", "-Wl,-z,defs", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    shutil.move(tmp, LIB_PATH)
    tmp = BACKEND_LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
          *[_obj(s) for s in hip + [x for x in c if os.path.basename(x) in BACKEND_HOST]],
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-lpthread", "-lm", "-Wl,-Bsymbolic",
          f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"])
    shutil.move(tmp, BACKEND_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} ({len(hip)} HIP + {len(c)} C sources) and {os.path.basename(BACKEND_LIB_PATH)}")
    return LIB_PATH


def build_asan(verbose: bool = True) -> str:
    """A host-sanitized copy of the library for checking the C11 host code:
    the host sources compiled by gcc with AddressSanitizer and
    UndefinedBehaviorSanitizer, linked by g++ (so gcc's runtimes) with the
    HIP kernel objects of the last build() unchanged, into
    pyc_amd/lib/asan/libpyc_amd.so. Host code only: nothing of the GPU side is
    instrumented. Programs linked to it, or a process started with the
    sanitizer runtimes in LD_PRELOAD, report the first error and stop."""
    hip, c = sources()
    missing = [_obj(s) for s in hip if not os.path.exists(_obj(s))]
    if missing:
        raise RuntimeError("build() first: the HIP objects are missing")
    adir = os.path.join(OBJ_DIR, "asan")
    os.makedirs(adir, exist_ok=True)
    san = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g", "-O1"]
    objs = []
    for src in c:
        o = os.path.join(adir, os.path.basename(src) + ".o")
        _run(["gcc", *[f for f in C_FLAGS if f != "-O2"], *san, "-c", src, "-o", o])
        objs.append(o)
    out_dir = os.path.join(LIB_DIR, "asan")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libpyc_amd.so")
    _run(["g++", "-shared", "-fPIC", "-o", out, *objs, *[_obj(s) for s in hip], "-L", os.path.join(ROCM, "lib"),
          "-lamdhip64", "-lpthread", "-lm", "-Wl,-Bsymbolic", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
          "-fsanitize=address,undefined"])
    if verbose:
        print(f"built {out} (host code with ASan + UBSan)")
    return out


if __name__ == "__main__":
    if "--asan" in sys.argv[1:]:
        build_asan()
    else:
        build()

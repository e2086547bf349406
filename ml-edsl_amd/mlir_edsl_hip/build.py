"""Build libedsl_hip.so (gfx950 kernels + C ABI) in-tree with hipcc.

``python -m mlir_edsl_hip.build`` (with ``ml-edsl_amd`` on ``sys.path``) or
``__graft_entry__.build()`` compiles every source in ``ml-edsl_amd/csrc`` for
gfx950 and links the shared library next to this file, where ``_native`` loads
it. The library is always rebuilt when asked (sources are few and compile in
seconds).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)  # ml-edsl_amd/
CSRC = os.path.join(ROOT, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_NAME = "libedsl_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

SOURCES = ["gemm_f32.hip", "gemm_f32_m16.hip", "gemm_f32_direct.hip", "gemv_f32.hip", "gemm_i8.hip", "runtime.cpp", "plan_f32.cpp",
           "program.cpp", "host_stage.cpp", "noalloc.hip", "unfused.hip"]
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled on purpose: the compiler would otherwise
# form v_pk_{add,mul,fma}_f32 from ordinary float2 code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
                "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int = 4, verbose: bool = False) -> str:
    """Compile all sources and link libedsl_hip.so. Returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    ext = build_launch_module()
    if verbose:
        print(f"built {LIB_PATH}")
        print(f"built {ext}")
    return LIB_PATH


def build_launch_module() -> str:
    """The CPython binding of the device launch entries (csrc/pylaunch.c),
    linked against libedsl_hip.so next to it (found through $ORIGIN, so the
    process maps the one library that _native also loads)."""
    import sysconfig
    out = os.path.join(PKG_DIR, "_launch" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out + ".tmp"
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    cmd = [cc, "-O2", "-fPIC", "-shared", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           os.path.join(CSRC, "pylaunch.c"), "-o", tmp, f"-L{PKG_DIR}", "-l:" + LIB_NAME,
           "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the launch module failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build(jobs=int(os.environ.get("MAX_JOBS", "4")), verbose=True)
    sys.exit(0)

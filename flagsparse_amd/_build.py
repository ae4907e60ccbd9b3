"""Build the gfx950 HIP library (``flagsparse_amd/_lib/libflagsparse_hip.so``) with hipcc.

Run ``python -m flagsparse_amd._build`` (or ``__graft_entry__.build()``).  The library is
built in-tree so that it travels with the source tree to the GPU host; nothing is JIT
compiled at run time.
"""

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libflagsparse_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

SOURCES = ("abi.cpp", "mtx.cpp", "plan.hip", "spmv.hip", "spmv_xcs.hip", "spmm.hip", "sddmm.hip",
           "index_stats.hip", "probe.hip")
ARCH = "gfx950"

# Packed-FP32 instructions (v_pk_*_f32) are disabled for all device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build flagsparse_amd")
    return exe


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + proc.stdout)
    return proc.stdout


def _scratch_kernels(log):
    """Kernels whose resource-usage remarks report scratch memory per lane."""
    found, name = set(), None
    for line in log.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            found.add(name)
    return found


def build(verbose=False):
    """Compile every source for gfx950 and link the shared library.  Always recompiles."""
    hipcc = _hipcc()
    obj_dir = os.path.join(PKG_DIR, "_lib", "obj")
    os.makedirs(obj_dir, exist_ok=True)
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]

    def compile_one(src):
        out = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
        # device sources also report each kernel's resources (checked below)
        lang = ["-x", "hip", "-Rpass-analysis=kernel-resource-usage"] if src.endswith(".hip") \
            else []
        cmd = [hipcc, *HIP_FLAGS, *includes, *lang, "-c", os.path.join(CSRC, src), "-o", out]
        log = _run(cmd)
        if verbose and log.strip():
            print(log)
        return out, _scratch_kernels(log)

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        done = list(ex.map(compile_one, SOURCES))
    objs = [o for o, _ in done]
    spills = sorted({k for _, ks in done for k in ks})
    if spills:
        # A kernel with per-lane scratch memory (spilled registers or a local array the compiler
        # could not keep in registers) pays a memory round trip for what should be a register.
        raise RuntimeError("kernels using scratch memory:\n  " + "\n  ".join(spills))
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)

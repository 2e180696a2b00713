"""Builds libsquirrel_hip.so (HIP kernels for gfx950 + C++ host + C ABI).

Run `python squirrel-rs_amd/build.py` (the repository's build entry point
calls it).  Objects go to squirrel-rs_amd/_build/, the library next to this
file.  Every HIP file is compiled with packed-FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsquirrel_hip.so")
ARCH = "gfx950"

HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]
# Per-file additions.  The prefill matmul converts every MFMA result on the
# VALU, so its results are placed straight in VGPRs (no AGPR copy-out).
FILE_FLAGS = {"k_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
CXX_FLAGS = ["-x", "c++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
             "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def host_cxx() -> str:
    c = "/opt/rocm/lib/llvm/bin/clang++"
    return c if os.path.exists(c) else "g++"


def _compile(src: str) -> tuple[str, str, int]:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src.endswith(".hip"):
        cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    else:
        cmd = [host_cxx(), *CXX_FLAGS, "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (p.stdout + p.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    return obj, out, p.returncode


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))
    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for obj, out, rc in ex.map(_compile, srcs):
            if out.strip() and (verbose or rc):
                print(out, file=sys.stderr)
            if rc:
                raise RuntimeError(f"compile failed: {obj}")
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, "-lpthread"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode:
        print(p.stdout + p.stderr, file=sys.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

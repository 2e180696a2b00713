"""Builds the CPU emulation of the squirrel-hip library (TEST INFRASTRUCTURE).

The HIP kernel sources of squirrel-rs_amd/csrc (all but the persistent
decode step) and the C++ host code are compiled for the host against the
emulated HIP device and runtime in tests/emu (one fiber per work-item,
wavefront collectives for cross-lane operations), with AddressSanitizer, and
linked with the oracle and the driver tests/emu/emu_model.cpp into
tests/emu/_build/emu_model.  An out-of-bounds access in a kernel or a host
launcher then stops the run with a sanitizer report naming the access.

Source rewrites, applied to copies under _build/src: dynamic
`extern __shared__` arrays become pointers to the launch's dynamic LDS,
`asm volatile` wait-count statements (no effect on the emulated memory
model) are dropped (the direct-to-LDS load helper's assembly becomes the
emulated load), and the library's refusals of the f32-activation
kernels (switched off on the device; see kA32Disabled) are removed so that
those kernels can be checked here.

    python tests/emu/build_emu.py [--no-asan]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
CSRC = os.environ.get("SQEMU_CSRC", os.path.join(REPO, "squirrel-rs_amd", "csrc"))
ORACLE = os.path.join(REPO, "oracle")
BUILD = os.environ.get("SQEMU_BUILD", os.path.join(HERE, "_build"))
EXE = os.path.join(BUILD, "emu_model")
SELFTEST = os.path.join(BUILD, "emu_selftest")
CLANG = "/opt/rocm/lib/llvm/bin/clang++"
CLANG_C = "/opt/rocm/lib/llvm/bin/clang"

SKIP = {"k_step.hip"}


def rewrite(text: str) -> str:
    text = re.sub(r"extern\s+__shared__\s+(\w+)\s+(\w+)\s*\[\s*\]\s*;",
                  r"\1* \2 = (\1*)::sqemu::dyn_lds();", text)
    # the direct-to-LDS load helper issues its load from inline assembly:
    # here the emulated load does the copy
    text = re.sub(r"(void dma_to_lds\(const void\* base, uint32_t off, lds_i8\* lds\) \{)",
                  r"\1\n    ::sqemu::global_load_lds((const char*)base + off, (void*)lds, SIZE, 0);", text)
    text = re.sub(r"asm\s+volatile\s*\((?:[^;]|\n)*?\)\s*;", ";", text)
    text = re.sub(r"^[ \t]*if \([^\n]*kA32Disabled\)+;[ \t]*\n", "", text, flags=re.M)
    return text


def sources(asan: bool):
    os.makedirs(os.path.join(BUILD, "src"), exist_ok=True)
    jobs = []
    for f in sorted(os.listdir(CSRC)):
        p = os.path.join(CSRC, f)
        if f in SKIP:
            continue
        if f.endswith((".hip", ".cpp")):
            dst = os.path.join(BUILD, "src", f.rsplit(".", 1)[0] + ".cpp")
            new = rewrite(open(p).read())
            if not os.path.exists(dst) or open(dst).read() != new:
                tmp = f"{dst}.{os.getpid()}.tmp"
                with open(tmp, "w") as fh:
                    fh.write(new)
                os.replace(tmp, dst)
            jobs.append(dst)
    jobs += [os.path.join(HERE, "emu.cpp"), os.path.join(HERE, "step_stub.cpp"),
             os.path.join(HERE, "emu_model.cpp"), os.path.join(HERE, "selftest.cpp")]
    return jobs


def flags(asan: bool):
    f = ["-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off"]
    if asan:
        f += ["-fsanitize=address"]
    return f


def compile_one(src: str, asan: bool):
    obj = os.path.join(BUILD, os.path.basename(src) + (".asan" if asan else "") + ".o")
    if src.endswith(".c"):
        cmd = [CLANG_C, "-std=c11", *flags(asan), "-c", src, "-o", obj]
    else:
        cmd = [CLANG, "-std=c++17", *flags(asan), "-D__HIPCC__", "-I", os.path.join(HERE, "include"),
               "-I", CSRC, "-Wno-unused-command-line-argument", "-c", src, "-o", obj]
    if os.path.exists(obj) and os.path.getmtime(obj) > max(
            os.path.getmtime(src), *(os.path.getmtime(os.path.join(CSRC, h)) for h in os.listdir(CSRC)
                                      if h.endswith(".h")),
            os.path.getmtime(os.path.join(HERE, "include", "hip", "hip_runtime.h"))):
        return obj, "", 0
    # written under a private name and renamed, so that concurrent builds
    # (parallel test workers) never see a partial object
    tmp = f"{obj}.{os.getpid()}.tmp"
    cmd[-1] = tmp
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode == 0:
        os.replace(tmp, obj)
    return obj, p.stdout + p.stderr, p.returncode


def build(asan: bool = True) -> str:
    srcs = sources(asan) + [os.path.join(ORACLE, "oracle.c")]
    objs = []
    with cf.ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        for obj, out, rc in ex.map(lambda s: compile_one(s, asan), srcs):
            if rc:
                print(out, file=sys.stderr)
                raise RuntimeError(f"compile failed: {obj}")
            objs.append(obj)
    emu = [o for o in objs if os.path.basename(o).startswith("emu.cpp")]
    lib = [o for o in objs if not os.path.basename(o).startswith(("emu", "selftest"))]
    drv = [o for o in objs if os.path.basename(o).startswith("emu_model")]
    st = [o for o in objs if os.path.basename(o).startswith("selftest")]
    for exe, parts in ((EXE, emu + lib + drv), (SELFTEST, emu + st)):
        tmp = f"{exe}.{os.getpid()}.tmp"
        cmd = [CLANG, *flags(asan), *parts, "-o", tmp, "-lm", "-lpthread"]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode:
            print(p.stdout + p.stderr, file=sys.stderr)
            raise RuntimeError("link failed")
        os.replace(tmp, exe)
    return EXE


if __name__ == "__main__":
    print(build(asan="--no-asan" not in sys.argv))

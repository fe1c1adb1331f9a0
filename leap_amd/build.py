"""Build recipe for libleap_hip_attention.so (gfx950), in-tree.

    python -m leap_amd.build [--no-timeline]

The RoPE table TU is compiled by the host C++ compiler with the reference's
release flags, the checkpoint reader by the host compiler, and the HIP TUs
(the host side and the three kernel tables, see csrc/kernels.hpp) by hipcc
for gfx950 only, in parallel.  Packed-fp32 VALU instructions are disabled for
device code (``-packed-fp32-ops``).
"""
from __future__ import annotations

import os
import shutil
from concurrent.futures import ThreadPoolExecutor
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libleap_hip_attention.so")
LIB_TL = os.path.join(PKG, "libleap_hip_attention_tl.so")  # the timeline build (-DLEAP_TIMELINE)
DEMO = os.path.join(PKG, "host", "engine_demo")
ARCH = "gfx950"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast-honor-pragmas",
    # the decode kernel's leading 14 argument words arrive preloaded in
    # scalar registers (kernels whose first argument is a struct preload
    # nothing)
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")
    return r


HIP_SOURCES = ("leap_hip_attention", "kernels_decode", "kernels_decode_64", "kernels_decode_64p",
               "kernels_decode_128", "kernels_decode_128p", "kernels_gemv", "kernels_q8")


def _hip_objects(build_dir: str, defines=()):
    """Compile steps of the HIP translation units into build_dir."""
    os.makedirs(build_dir, exist_ok=True)
    objs = [os.path.join(build_dir, f"{n}.o") for n in HIP_SOURCES]
    steps = [[_hipcc(), *HIPCC_FLAGS, *defines, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, f"{n}.hip"),
              "-o", o] for n, o in zip(HIP_SOURCES, objs)]
    return objs, steps


def build(verbose: bool = False, timeline: bool = True) -> str:
    """Build the library (and, with timeline, its timeline build
    libleap_hip_attention_tl.so, the same sources with -DLEAP_TIMELINE)."""
    os.makedirs(BUILD, exist_ok=True)
    rope_o = os.path.join(BUILD, "rope_table.o")
    ckpt_o = os.path.join(BUILD, "checkpoint.o")
    hip_os, hip_steps = _hip_objects(BUILD)
    compile_steps = [
        ["g++", "-std=c++17", "-O3", "-march=x86-64-v3", "-ffast-math", "-fPIC", "-c",
         os.path.join(CSRC, "rope_table.cpp"), "-o", rope_o],
        ["g++", "-std=c++17", "-O2", "-Wall", "-fPIC", "-I", INCLUDE, "-c",
         os.path.join(CSRC, "checkpoint.cpp"), "-o", ckpt_o],
    ] + hip_steps
    libs = [(LIB, hip_os)]
    if timeline:
        tl_os, tl_steps = _hip_objects(os.path.join(BUILD, "tl"), ("-DLEAP_TIMELINE",))
        compile_steps += tl_steps
        libs.append((LIB_TL, tl_os))
    if verbose:
        for cmd in compile_steps:
            print(" ".join(cmd))
    jobs = max(1, min(len(compile_steps), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, compile_steps))
    for lib, objs in libs:
        link = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib + ".tmp", *objs, rope_o, ckpt_o]
        if verbose:
            print(" ".join(link))
        _run(link)
        os.replace(lib + ".tmp", lib)
    # the C++20 engine-side wrapper and demo layer loop, linked against the
    # library in place
    demo = ["g++", "-std=c++20", "-O2", "-Wall", "-I", INCLUDE, "-I", os.path.join(PKG, "host"),
            "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
            os.path.join(PKG, "host", "engine_demo.cpp"), "-o", DEMO + ".tmp", "-L", PKG,
            "-lleap_hip_attention", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
            "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath," + os.path.join(ROCM, "lib")]
    if verbose:
        print(" ".join(demo))
    _run(demo)
    os.replace(DEMO + ".tmp", DEMO)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, timeline="--no-timeline" not in sys.argv[1:]))

"""Builds kadan_amd/libkadan_amd.so (gfx950 HIP kernels + the C ABI of include/kadan_amd.h)
and the host C++ layer kadan_amd/libkadan_amd_host.so in-tree with hipcc.

    python -m kadan_amd.build        # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures as futures
import os
import subprocess
import sys

PACKAGE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PACKAGE)
CSRC = os.path.join(PACKAGE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

DEVICE_SOURCES = ["capi.hip", "gguf_gemv.hip", "gguf_gemm.hip", "gguf_gemm_rows.hip",
                  "q4_0_gemm.hip", "moe_mxfp4.hip", "moe_gguf.hip", "hbm_read.hip"]
HOST_SOURCES = ["hip_dense_compute.cpp", "checkpoint.cpp"]
LIBRARY = os.path.join(PACKAGE, "libkadan_amd.so")
HOST_LIBRARY = os.path.join(PACKAGE, "libkadan_amd_host.so")
PROBE_SOURCE = os.path.join(ROOT, "tests", "cpp", "dense_compute_probe.cpp")
PROBE_LIBRARY = os.path.join(ROOT, "tests", "cpp", "libdense_compute_probe.so")

# gfx950 only.  Packed-fp32 instructions are disabled (the compiler would otherwise
# form v_pk_*_f32 from scalar float code).  No FMA contraction: every fused
# multiply-add in the kernels is written explicitly.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", INCLUDE, "-I", CSRC,
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line)
    if proc.returncode:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    """Compiles every HIP source (always, even when a library exists) and links."""
    os.makedirs(BUILD, exist_ok=True)
    objects = []
    jobs = []
    for src in DEVICE_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        objects.append(obj)
        jobs.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    workers = min(len(jobs), max(1, (os.cpu_count() or 2) // 2))
    with futures.ThreadPoolExecutor(workers) as pool:
        for out in pool.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    tmp = LIBRARY + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects])
    os.replace(tmp, LIBRARY)
    # host C++ layer (the DenseCompute-compatible class) over the C ABI
    host_objects = []
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src + ".o")
        _run([HIPCC, "-O2", "-std=c++20", "-fPIC", "-Wall", "-I", INCLUDE, "-I", CSRC,
              "-c", os.path.join(CSRC, src), "-o", obj])
        host_objects.append(obj)
    tmp = HOST_LIBRARY + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "-o", tmp, *host_objects, "-L", PACKAGE,
          "-lkadan_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_LIBRARY)
    # the tests' C shim over the host layer (tests/cpp), built here so no test compiles
    if os.path.exists(PROBE_SOURCE):
        tmp = PROBE_LIBRARY + ".tmp"
        _run([HIPCC, "-O2", "-std=c++20", "-fPIC", "-Wall", "-shared", "-I", INCLUDE,
              PROBE_SOURCE, "-o", tmp, "-L", PACKAGE, "-lkadan_amd_host", "-lkadan_amd",
              "-Wl,-rpath,$ORIGIN/../../kadan_amd"])
        os.replace(tmp, PROBE_LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

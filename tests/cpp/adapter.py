"""Builds tests/cpp/adapter_probe: the DenseCompute adapter of the integration guide's section 1
(extracted from the document as it stands), compiled with g++ -std=c++20 against the
reference's own headers, linked to libkadan_amd_host.so, plus adapter_probe.cpp, which
calls it through kadan::DenseCompute.  Test infrastructure; it needs the reference's
headers, so it builds only where /root/reference exists (the probe binary then travels
with the tree like the other built files).

    python tests/cpp/adapter.py
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REFERENCE_INCLUDE = "/root/reference/services/hikari/inference_worker/include"
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")
PROBE = os.path.join(HERE, "adapter_probe")
ADAPTER_SOURCE = os.path.join(HERE, "_adapter", "hip_dense_compute_adapter.cpp")
ROCM_LIB = "/opt/rocm/lib"


def available() -> bool:
    return os.path.isdir(REFERENCE_INCLUDE)


def adapter_source() -> str:
    """The first C++ block of the integration guide's section 1, verbatim."""
    text = open(INTEGRATION).read()
    section = text[text.index("## 1."):]
    match = re.search(r"```cpp\n(.*?)```", section, re.S)
    if not match:
        raise RuntimeError("INTEGRATION.md section 1 has no ```cpp block")
    return match.group(1)


def compile_adapter_only() -> None:
    """g++ -fsyntax-only of the adapter against the reference's header (no GPU needed)."""
    os.makedirs(os.path.dirname(ADAPTER_SOURCE), exist_ok=True)
    with open(ADAPTER_SOURCE, "w") as f:
        f.write(adapter_source())
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall",
                    "-I", REFERENCE_INCLUDE, "-I", os.path.join(ROOT, "include"),
                    ADAPTER_SOURCE], check=True, capture_output=True, text=True)


def build() -> str:
    compile_adapter_only()
    package = os.path.join(ROOT, "kadan_amd")
    tmp = PROBE + ".tmp"
    cmd = ["g++", "-std=c++20", "-O1", "-Wall", "-I", REFERENCE_INCLUDE,
           "-I", os.path.join(ROOT, "include"), ADAPTER_SOURCE,
           os.path.join(HERE, "adapter_probe.cpp"), "-o", tmp, "-L", package,
           "-lkadan_amd_host", "-lkadan_amd", f"-Wl,-rpath-link,{ROCM_LIB}",
           "-Wl,-rpath,$ORIGIN/../../kadan_amd"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"adapter probe build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, PROBE)
    return PROBE


if __name__ == "__main__":
    if not available():
        sys.exit("the reference's headers are not here")
    print(build())

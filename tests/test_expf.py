"""The device router's exponential (glibc_expf, kadan_amd/csrc/kdq_expf.hpp) against the
host C library's expf, which the reference's router calls through std::exp(float)
(IW/src/models/text/qwen_layers.cpp:404-408; IW = services/hikari/inference_worker).

tests/cpp/expf_check.cpp compiles the same header for the host and compares every one of
the 2^32 float bit patterns (about 12 s on 8 threads) bit for bit: the finite range, the
overflow and underflow ends, zeros, infinities and NaNs.  glibc's x86-64
build runs its FMA variant on CPUs with FMA and AVX2; the header restates that variant.
On a CPU without them the library takes the unfused variant, which differs on two of
those inputs, so the check is skipped there."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _cpu_flags():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def test_glibc_expf_restatement_exhaustive(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("no g++")
    if not {"fma", "avx2"} <= _cpu_flags():
        pytest.skip("the C library takes its unfused expf on this CPU")
    exe = str(tmp_path / "expf_check")
    subprocess.run(["g++", "-O2", "-std=c++20", "-ffp-contract=off", "-pthread", "-o", exe,
                    os.path.join(HERE, "cpp", "expf_check.cpp")], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 mismatches" in out.stdout

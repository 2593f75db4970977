"""The DenseCompute adapter published in the repository's integration guide (its section
1) compiles against the reference's
own interface (IW/include/kadan/dense_compute.hpp:60-345) and links to
libkadan_amd_host.so; the probe calls it through kadan::DenseCompute.  Without a GPU the
probe stops at construction with the library's kdq_hip error; the GPU test
(test_integration_gpu.py) runs the probe's products.  Skips where the reference's
headers are absent."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "cpp"))
import adapter  # noqa: E402

pytestmark = pytest.mark.skipif(not adapter.available(),
                                reason="the reference's headers are not here")


def test_adapter_compiles_against_reference_interface():
    adapter.compile_adapter_only()


def test_adapter_links_and_runs_through_dense_compute():
    probe = adapter.build()
    proc = subprocess.run([probe], capture_output=True, text=True, timeout=120)
    if proc.returncode == 3:  # no GPU here: the constructor's hipSetDevice failed, loudly
        assert "kdq_hip" in proc.stdout
    else:
        assert proc.returncode == 0, proc.stdout + proc.stderr
        assert "adapter probe passed" in proc.stdout

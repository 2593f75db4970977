"""The integration guide's DenseCompute adapter on the GPU, through the reference's interface
type: tests/cpp/adapter_probe (built by tests/cpp/adapter.py where the reference's
headers exist) runs a refused shape, a Q4_K dense_gguf_source with bias (and its bank
hit), a two-job Q8_0 dense_gguf_batch and an F32 dense, each against a double product of
the reference's own kadan::gguf::decode."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "adapter_probe")


@pytest.mark.skipif(not os.path.exists(PROBE),
                    reason="adapter_probe is built only where the reference's headers are")
def test_adapter_probe_on_gpu(device):
    proc = subprocess.run([PROBE], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "adapter probe passed" in proc.stdout

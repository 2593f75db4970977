"""CPU checks of the host layer's batch eligibility (HipDenseCompute::batch_supported,
the rule dense_gguf_batch applies before any source read), through the C shim
tests/cpp/dense_compute_probe.cpp.  No device is needed: the rule reads only the job
descriptions.

The cases follow IW/include/kadan/gguf_batch_partition.hpp:15-37 (IW =
services/hikari/inference_worker) and its tests IW/tests/gguf_batch_partition.cpp:18-100:
a job without an encoding is F32 rows and is admitted when in % 8 == 0 and a row fits the
16 MiB staging buffer; an encoded job needs whole blocks, in % 8 == 0 and a row of at most
16 MiB; every job needs rows <= 4096 and a non-empty input; one refused job refuses the
whole batch."""
import ctypes
import os

import pytest

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp",
                     "libdense_compute_probe.so")
F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
STAGING = 16 << 20


@pytest.fixture(scope="module")
def supported():
    if not os.path.exists(PROBE):
        pytest.skip("tests/cpp/libdense_compute_probe.so is not built (run build())")
    lib = ctypes.CDLL(PROBE)
    fn = lib.kdc_batch_supported
    fn.restype = ctypes.c_int
    sz = ctypes.c_size_t
    fn.argtypes = [sz, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]

    def call(jobs):
        """jobs: (ggml type, rows, in, out)"""
        n = len(jobs)
        arr = lambda t, k: (t * n)(*[j[k] for j in jobs])
        return fn(n, arr(ctypes.c_uint, 0), arr(sz, 1), arr(sz, 2), arr(sz, 3))
    return call


def test_f32_jobs_admitted(supported):
    assert supported([(F32, 1, 2048, 128)]) == 1
    assert supported([(F32, 8, 8, 1)]) == 1
    assert supported([(F32, 4096, 64, 4)]) == 1
    # the widest F32 row the staging holds
    assert supported([(F32, 1, STAGING // 4, 1)]) == 1


def test_f32_refusals(supported):
    assert supported([(F32, 1, 36, 4)]) == 0             # in % 8 != 0
    assert supported([(F32, 1, STAGING // 4 + 8, 1)]) == 0  # a row past 16 MiB
    assert supported([(F32, 4097, 64, 4)]) == 0          # more than gguf_batch_max_rows
    assert supported([(F32, 0, 64, 4)]) == 0             # empty input


def test_moe_first_batch_admitted(supported):
    # MoeLayer::forward's first batch (IW/src/models/text/qwen_layers.cpp:383-389): an F32
    # router and Q8_0 shared gate and up on the same rows
    assert supported([(F32, 4, 2048, 128), (Q8_0, 4, 2048, 768), (Q8_0, 4, 2048, 768)]) == 1


def test_encoded_refusals(supported):
    assert supported([(Q4_K, 1, 4096, 14336)]) == 1
    assert supported([(Q4_K, 1, 4000, 14336)]) == 0      # not whole super-blocks
    assert supported([(Q8_0, 1, 48, 16)]) == 0           # not whole blocks
    # a row of more than 16 MiB of blocks
    rows_of = STAGING // 210 + 1
    assert supported([(Q6_K, 1, rows_of * 256, 1)]) == 0
    assert supported([(Q6_K, 1, (rows_of - 1) * 256, 1)]) == 1


def test_one_refusal_refuses_the_batch(supported):
    assert supported([(Q8_0, 1, 256, 16), (F32, 1, 36, 4)]) == 0
    assert supported([]) == 0


def test_unknown_type(supported):
    assert supported([(3, 1, 256, 16)]) == -1  # GGML type 3 (Q4_1) has no kadan encoding

"""Comparison helpers shared by the parity tests."""
import numpy as np

# Tolerances of the quantized matmul path for fp32-accumulated outputs (rel-L2, and
# max-abs after normalising by the reference output RMS).
REL_L2 = 1e-3
MAX_ABS = 2e-2


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    denom = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (denom if denom else 1.0))


def normalized_max_abs(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    return float(np.max(np.abs(a - e)) / (rms if rms else 1.0)) if e.size else 0.0


def assert_close(actual, expected, rel=REL_L2, mabs=MAX_ABS, what=""):
    r = rel_l2(actual, expected)
    m = normalized_max_abs(actual, expected)
    assert r <= rel and m <= mabs, f"{what}: rel_l2={r:.3e} (<= {rel}) max_abs/rms={m:.3e} (<= {mabs})"
    return r, m


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and bool(np.array_equal(a, b))

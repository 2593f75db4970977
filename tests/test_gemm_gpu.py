"""GPU parity of the prefill Q4_0 GEMM (kdq_quantize_q8, kdq_gemm_q4_0, and
kdq_gemm_q4_0_packed over the tile-packed layout of kdq_gguf_pack).

The activation codes and scales must be bit-exact to the oracle's restatement of
ggml's x86 quantize_row_q8_0 (which tests/test_oracle.py pins to the compiled
reference).  The fp16 output must be within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the
output RMS of the oracle's Q4_0 x Q8 product over the same codes (double accumulation).
"""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


@pytest.mark.parametrize("m,k", [(1, 32), (3, 256), (64, 4096), (512, 4096), (7, 14336)])
def test_quantize_bit_exact(device, oracle, m, k):
    torch = _torch()
    x = synth.normal(0xC3 + m, 1, m * k).reshape(m, k).astype(np.float16)
    # exact half-way cases: values that land on .5 after scaling by 127/amax
    x[0, 0] = np.float16(127.0)
    if k >= 32:
        x[0, 1] = np.float16(0.5)   # 0.5 * 127/127 = 0.5 -> 0 (even)
        x[0, 2] = np.float16(1.5)   # -> 2
        x[0, 3] = np.float16(-2.5)  # -> -2
    if m > 1:
        x[1, :32] = 0  # all-zero block: d = 0, codes 0
    qs, d = oracle.quantize_q8_f16(x.view(np.uint16))
    from kadan_amd import ops
    gq, gd = ops.quantize_q8(torch.from_numpy(x).to(device))
    assert np.array_equal(gq.cpu().numpy(), qs)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), d.view(np.uint32))


SHAPES = [(1, 256, 1), (5, 256, 130), (128, 512, 128), (130, 1024, 300), (33, 4096, 256),
          (256, 4096, 1024), (512, 4096, 640)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_gemm_q4_0_parity(device, oracle, m, k, n):
    torch = _torch()
    seed = (m * 131 + k * 7 + n) & 0xFFFF
    w = synth.q4_0_weights(seed, n, k)
    x = synth.normal(seed, 9, m * k).reshape(m, k).astype(np.float16)
    xq, xd = oracle.quantize_q8_f16(x.view(np.uint16))
    expected = oracle.gemm_q4_0_q8(w, n, k, xq, xd)
    from kadan_amd import ops
    y = ops.gemm_q4_0(torch.from_numpy(w).to(device), torch.from_numpy(x).to(device), n)
    got = y.float().cpu().numpy()
    assert_close(got, expected, what=f"gemm m={m} k={k} n={n}")


def test_gemm_q4_0_baseline_shape_property(device, oracle):
    """C3 at full size (M=512, K=4096, N=14336): a column sample against the oracle, and
    linearity in the activations through the exact-code path (scaling x by 2 scales the
    codes' scale exactly, so the output doubles up to fp16 rounding)."""
    torch = _torch()
    m, k, n = 512, 4096, 14336
    w = synth.q4_0_weights(0xC3, n, k)
    x = synth.normal(0xC3, 9, m * k).reshape(m, k).astype(np.float16)
    from kadan_amd import ops
    wd = torch.from_numpy(w).to(device)
    xd_ = torch.from_numpy(x).to(device)
    y = ops.gemm_q4_0(wd, xd_, n).float().cpu().numpy()
    cols = np.arange(0, n, 97)
    xq, xs = oracle.quantize_q8_f16(x.view(np.uint16))
    expected = oracle.gemm_q4_0_q8(np.ascontiguousarray(w[cols]), cols.size, k, xq, xs)
    assert_close(y[:, cols], expected, what="C3 column sample")
    y2 = ops.gemm_q4_0(wd, xd_ * 2, n).float().cpu().numpy()
    assert_close(y2, 2 * y, rel=1e-6, mabs=1e-5, what="doubling")


# odd group counts (k / 256), ragged n (not a multiple of 16, 8 or 4), m below, at and
# above the 128-token tile
PACKED_SHAPES = SHAPES + [(1, 768, 16), (129, 1280, 250), (200, 768, 301), (64, 512, 514)]


def _packed(torch, device, w, k):
    from kadan_amd import ops
    return ops.gguf_pack(2, torch.from_numpy(w).to(device), k)


@pytest.mark.parametrize("m,k,n", PACKED_SHAPES)
def test_gemm_q4_0_packed_parity(device, oracle, m, k, n):
    torch = _torch()
    seed = (m * 131 + k * 7 + n) & 0xFFFF
    w = synth.q4_0_weights(seed, n, k)
    x = synth.normal(seed, 9, m * k).reshape(m, k).astype(np.float16)
    xq, xd = oracle.quantize_q8_f16(x.view(np.uint16))
    expected = oracle.gemm_q4_0_q8(w, n, k, xq, xd)
    from kadan_amd import ops
    packed = _packed(torch, device, w, k)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=device)
    ops.gemm_q4_0_packed(packed, torch.from_numpy(x).to(device), n, out=y)
    got = y.float().cpu().numpy()
    assert np.isfinite(got).all(), "an output element was not written"
    assert_close(got, expected, what=f"packed gemm m={m} k={k} n={n}")
    # same fp16 operands as the row-major kernel: only the fp32 summation order differs
    y_row = ops.gemm_q4_0(torch.from_numpy(w).to(device), torch.from_numpy(x).to(device), n)
    assert_close(got, y_row.float().cpu().numpy(), rel=1e-4, mabs=1e-2,
                 what=f"packed vs row-major m={m} k={k} n={n}")


def test_gemm_q4_0_packed_baseline_shape_property(device, oracle):
    """C3 at full size through the packed layout: a column sample against the oracle, the
    doubling property, and a second call with fewer tokens into the same output (rows
    past the new m stay untouched)."""
    torch = _torch()
    m, k, n = 512, 4096, 14336
    w = synth.q4_0_weights(0xC3, n, k)
    x = synth.normal(0xC3, 9, m * k).reshape(m, k).astype(np.float16)
    from kadan_amd import ops
    packed = _packed(torch, device, w, k)
    xd_ = torch.from_numpy(x).to(device)
    y = ops.gemm_q4_0_packed(packed, xd_, n).float().cpu().numpy()
    cols = np.arange(0, n, 97)
    xq, xs = oracle.quantize_q8_f16(x.view(np.uint16))
    expected = oracle.gemm_q4_0_q8(np.ascontiguousarray(w[cols]), cols.size, k, xq, xs)
    assert_close(y[:, cols], expected, what="C3 packed column sample")
    y2 = ops.gemm_q4_0_packed(packed, xd_ * 2, n).float().cpu().numpy()
    assert_close(y2, 2 * y, rel=1e-6, mabs=1e-5, what="doubling")
    out = torch.full((m, n), 7.0, dtype=torch.float16, device=device)
    ops.gemm_q4_0_packed(packed, xd_[:100].contiguous(), n, out=out[:100])
    got = out.float().cpu().numpy()
    assert_close(got[:100], y[:100], rel=1e-6, mabs=1e-5, what="first 100 tokens")
    assert (got[100:] == 7.0).all()

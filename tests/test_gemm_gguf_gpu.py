"""GPU parity of the prefill GEMM for the kadan encodings (kdq_gemm_packed over the
tile-packed bank copy of kdq_gguf_pack): Q4_K, Q8_0 and Q6_K.

The reference's prefill is the fp32 product of exactly decoded weights (decode tile +
cublasSgemm, IW/src/cuda/h3_compute.cu:2201-2218,2451); the oracle's kdo_gemv is that
product in double.  Outputs must be within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the
output RMS.  At the full prefill-chunk shapes (512 tokens, 4096 -> 14336 and
14336 -> 4096) the oracle runs on a sample of output columns (each output column depends
only on its own weight row).
"""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K = 8, 12, 14
ENCODINGS = [Q4_K, Q8_0, Q6_K]
NAMES = {Q4_K: "q4_k", Q8_0: "q8_0", Q6_K: "q6_k"}


def _torch():
    import torch
    return torch


def run(device, oracle, enc, m, k, n, seed, cols=None):
    torch = _torch()
    from kadan_amd import ops
    w = synth.gguf_weights(enc, seed, n, k)
    packed = ops.gguf_pack(enc, torch.from_numpy(w).to(device), k)
    x = synth.normal(seed, 7, m * k).reshape(m, k)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y = ops.gemm_packed(enc, packed, torch.from_numpy(x).to(device), n, status=status)
    y = y.cpu().numpy()
    assert int(status.item()) == 0
    if cols is None:
        want = oracle.gemv(enc, w, x, k, n)
        got = y
    else:
        pick = np.sort(np.random.default_rng(seed).choice(n, cols, replace=False))
        pick[-1] = n - 1  # the last row (a partial packed tile when n % 16 != 0)
        want = oracle.gemv(enc, w[pick], x, k, len(pick))
        got = y[:, pick]
    assert np.isfinite(y).all()
    assert_close(got, want, what=f"gemm {NAMES[enc]} m={m} k={k} n={n}")


@pytest.mark.parametrize("enc", ENCODINGS)
@pytest.mark.parametrize("m,k,n", [(1, 256, 16), (9, 512, 40), (130, 1024, 300),
                                   (129, 768, 257), (256, 2048, 512), (64, 6912, 520),
                                   (200, 4352, 96)])
def test_gemm_small_shapes(device, oracle, enc, m, k, n):
    """(64, 6912, 520) and (200, 4352, 96) have few output tiles: they run K slices (nine
    slices of 3 of the 27 groups; six slices of 3, 3, 3, 3, 3 and 2 of 17) and the ordered
    slice sum."""
    run(device, oracle, enc, m, k, n, seed=0x9E + m + n)


@pytest.mark.parametrize("enc", ENCODINGS)
@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 4096)])
def test_gemm_prefill_chunk(device, oracle, enc, k, n):
    """A 512-token prefill chunk (IW/src/models/text/gguf_engine.cpp:16) at Llama-3-8B's
    FFN shapes, checked on 64 sampled output columns."""
    run(device, oracle, enc, 512, k, n, seed=0xC2 + k, cols=64)


def test_gemm_status_flags(device):
    """A non-finite block scale sets bit 1; a scale whose dequantised weights could pass
    the fp16 range sets bit 2 (the caller then takes the decode-time product)."""
    torch = _torch()
    from kadan_amd import ops
    k, n = 512, 32
    for d_bits, flag in ((0x7C00, 1), (0x6000, 2)):  # +inf; 512.0 (128 * 512 > 65504)
        w = synth.gguf_weights(Q8_0, 3, n, k)
        w[5, 0], w[5, 1] = d_bits & 255, d_bits >> 8
        packed = ops.gguf_pack(Q8_0, torch.from_numpy(w).to(device), k)
        status = torch.zeros(1, dtype=torch.int32, device=device)
        ops.gemm_packed(Q8_0, packed, torch.ones(4, k, device=device), n, status=status)
        assert int(status.item()) & flag


D_AT = {Q8_0: 0, Q4_K: 0, Q6_K: 208}  # byte offset of the first block's fp16 d


@pytest.mark.parametrize("enc", ENCODINGS)
def test_gemm_check_matches_the_gemm_flags(device, enc):
    """kdq_gguf_gemm_check runs the GEMM's own scale checks over a packed matrix without
    the product: a clean matrix gives 0, a non-finite d bit 1, a d of 512 (every encoding's
    dequantised weights then pass the fp16 range) bit 2 -- the same bits the GEMM sets."""
    torch = _torch()
    from kadan_amd import ops
    k, n = 512, 40
    clean = synth.gguf_weights(enc, 5, n, k)
    packed = ops.gguf_pack(enc, torch.from_numpy(clean).to(device), k)
    assert ops.gguf_gemm_check(enc, packed, n, k) == 0
    for d_bits, flag in ((0x7C00, 1), (0x6000, 2)):
        w = clean.copy()
        w[33, D_AT[enc]], w[33, D_AT[enc] + 1] = d_bits & 255, d_bits >> 8
        packed = ops.gguf_pack(enc, torch.from_numpy(w).to(device), k)
        got = ops.gguf_gemm_check(enc, packed, n, k)
        assert got & flag
        status = torch.zeros(1, dtype=torch.int32, device=device)
        ops.gemm_packed(enc, packed, torch.ones(4, k, device=device), n, status=status)
        assert int(status.item()) == got


def test_gemm_nonfinite_input_poisons_its_row(device):
    torch = _torch()
    from kadan_amd import ops
    k, n, m = 512, 48, 6
    w = synth.gguf_weights(Q4_K, 4, n, k)
    packed = ops.gguf_pack(Q4_K, torch.from_numpy(w).to(device), k)
    x = synth.normal(4, 1, m * k).reshape(m, k)
    clean = ops.gemm_packed(Q4_K, packed, torch.from_numpy(x).to(device), n).cpu().numpy()
    x[2, 100] = np.inf
    got = ops.gemm_packed(Q4_K, packed, torch.from_numpy(x).to(device), n).cpu().numpy()
    assert not np.isfinite(got[2]).any()
    others = [t for t in range(m) if t != 2]
    assert np.array_equal(got[others], clean[others])

"""GPU parity of the decode and the products for the encodings beyond Q4_0 / Q8_0 / Q4_K
(Q3_K, Q6_K, IQ4_NL, IQ4_XS, IQ3_XXS, IQ2_S, IQ3_S, BF16;
IW/include/kadan/gguf_quantization.hpp:631-762).

Decoded weights must be bit-exact to the oracle (NaN matches NaN, as
IW/tests/gguf_quantization.cpp:21-29 compares), including the special fp16 block scales
of that test at each format's scale offset; products (kdq_gemv, which runs the MFMA
GEMV for Q3_K, Q6_K, IQ4_XS and IQ4_NL rows of whole 256-value groups and the exact
kernel otherwise, and
kdq_gemv_exact) within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the output RMS against the
oracle's double product of exactly decoded weights.
"""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16 = 11, 14, 20, 23, 30
IQ3_XXS, IQ3_S, IQ2_S = 18, 21, 22
ENCODINGS = [Q3_K, Q6_K, IQ4_NL, IQ4_XS, IQ3_XXS, IQ2_S, IQ3_S, BF16]
BV = {Q3_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256, BF16: 1, IQ3_XXS: 256, IQ2_S: 256,
      IQ3_S: 256}
BB = {Q3_K: 110, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136, BF16: 2, IQ3_XXS: 98, IQ2_S: 82,
      IQ3_S: 110}
SCALE_AT = {Q3_K: 108, Q6_K: 208, IQ4_NL: 0, IQ4_XS: 0, IQ3_XXS: 0, IQ2_S: 0, IQ3_S: 0}
SPECIAL_HALVES = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x83FF, 0x0400, 0x8400, 0x3C00,
                  0xBC00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E01, 0x7C01]


def _torch():
    import torch
    return torch


def same_bits_or_nan(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def special_rows(encoding, seed):
    """Random blocks, 8 per row for block formats (the first 16 carrying the special
    scales), or 4096 random bf16 values (the first 16 the special patterns)."""
    if encoding == BF16:
        raw = synth.random_bytes(seed, 7, 2 * 4096)
        raw.view(np.uint16)[:16] = SPECIAL_HALVES
        return raw.reshape(8, -1), 512
    count = 2048
    blocks = synth.random_bytes(seed, 7, count * BB[encoding]).reshape(count, BB[encoding])
    at = SCALE_AT[encoding]
    for i, h in enumerate(SPECIAL_HALVES):
        blocks[i, at], blocks[i, at + 1] = h & 0xFF, h >> 8
    return blocks.reshape(count // 8, 8 * BB[encoding]), 8 * BV[encoding]


def test_iq_grids_every_entry(device, oracle, golden_iq):
    """Blocks whose grid indices enumerate each IQ grid: every device table entry decodes
    as the oracle's (itself pinned to ggml on the same blocks)."""
    torch = _torch()
    from kadan_amd import ops
    for encoding, blocks in golden_iq.items():
        expected = oracle.dequantize(encoding, blocks, 256)
        got = ops.dequantize(encoding, torch.from_numpy(blocks).to(device), 256)
        assert same_bits_or_nan(got.cpu().numpy(), expected), encoding


@pytest.fixture(scope="module")
def golden_iq():
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "reference_vectors.npz")
    with np.load(path, allow_pickle=False) as f:
        return {IQ3_XXS: f["decode_iq3_xxs_blocks"], IQ2_S: f["decode_iq2_s_blocks"],
                IQ3_S: f["decode_iq3_s_blocks"]}


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_dequantize_bit_exact(device, oracle, encoding):
    torch = _torch()
    rows, n_in = special_rows(encoding, 0x2718 + encoding)
    expected = oracle.dequantize(encoding, rows, n_in)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.dequantize(encoding, torch.from_numpy(rows).to(device), n_in, status=status)
    assert same_bits_or_nan(got.cpu().numpy(), expected)
    assert int(status.item()) == 1  # inf / NaN scales (bf16: patterns) decode non-finite


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_dequantize_finite_status_clear(device, oracle, encoding):
    torch = _torch()
    w = synth.gguf_weights(encoding, 11, 64, 1024)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.dequantize(encoding, torch.from_numpy(w).to(device), 1024, status=status)
    assert same_bits_or_nan(got.cpu().numpy(), oracle.dequantize(encoding, w, 1024))
    assert int(status.item()) == 0


SHAPES = [(1, 256, 1), (1, 512, 64), (3, 2048, 100), (8, 4096, 33), (1, 14336, 17),
          (2, 768, 257)]


@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemv_parity(device, oracle, encoding, exact, shape):
    torch = _torch()
    rows, n_in, n_out = shape
    seed = (encoding * 1009 + rows * 131 + n_in * 7 + n_out) & 0xFFFF
    w = synth.gguf_weights(encoding, seed, n_out, n_in)
    x = synth.normal(seed, 50, rows * n_in).reshape(rows, n_in)
    expected = oracle.gemv(encoding, w, x, n_in, n_out)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.gemv(encoding, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device),
                   n_out, status=status, exact=exact)
    assert_close(got.cpu().numpy(), expected, what=f"enc={encoding} exact={exact} {shape}")
    assert int(status.item()) == 0


@pytest.mark.parametrize("encoding", [Q3_K, Q6_K, IQ4_NL, IQ4_XS, IQ3_XXS, IQ2_S, IQ3_S])
def test_gemv_nonfinite_scale_status(device, encoding):
    torch = _torch()
    w = synth.gguf_weights(encoding, 3, 16, 512)
    at = SCALE_AT[encoding]
    w[5, at], w[5, at + 1] = 0x00, 0x7C  # +inf scale in the first block of row 5
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y = ops.gemv(encoding, torch.from_numpy(w).to(device), torch.ones(1, 512, device=device),
                 16, status=status)
    assert int(status.item()) == 1
    assert not np.isfinite(y.cpu().numpy()[0, 5])


def test_batch_mixes_streamed_and_exact_encodings(device, oracle):
    """One submission over every encoding: streamed ones fuse, the others run exact."""
    torch = _torch()
    shared = synth.normal(19, 1, 2 * 1024).reshape(2, 1024)
    xs = torch.from_numpy(shared).to(device)
    jobs, expected = [], []
    for i, enc in enumerate([12, Q6_K, 8, Q3_K, IQ4_XS, 2, IQ4_NL, BF16, IQ3_XXS, IQ2_S, IQ3_S]):
        n_out = 40 + 8 * i
        w = synth.gguf_weights(enc, 60 + i, n_out, 1024)
        jobs.append({"encoding": enc, "weights": torch.from_numpy(w).to(device), "input": xs,
                     "output": torch.empty(2, n_out, device=device)})
        expected.append(oracle.gemv(enc, w, shared, 1024, n_out))
    from kadan_amd import ops
    ops.gemv_batch(jobs)
    for j, e in zip(jobs, expected):
        assert_close(j["output"].cpu().numpy(), e, what=f"enc={j['encoding']}")


@pytest.mark.parametrize("shift", [0, 1])
def test_q6_k_mfma_two_byte_aligned_rows(device, oracle, shift):
    """Q6_K rows start 210 bytes apart, so super-blocks and whole rows alternate between
    dword and half-dword alignment; a base two bytes past a dword flips every one of
    them.  Rows of 3 super-blocks (630 bytes), batch 1, 2 and 5."""
    torch = _torch()
    from kadan_amd import ops
    n_in, n_out = 768, 77
    w = synth.gguf_weights(Q6_K, 41 + shift, n_out + 1, n_in)
    dev = torch.from_numpy(w).to(device)
    view = dev[shift:shift + n_out]  # shift 1: the base moves by 630 bytes
    assert (view.data_ptr() % 4) == (2 if shift else 0)
    for rows in (1, 2, 5):
        x = synth.normal(7 + rows, 3, rows * n_in).reshape(rows, n_in)
        expected = oracle.gemv(Q6_K, w[shift:shift + n_out], x, n_in, n_out)
        got = ops.gemv(Q6_K, view, torch.from_numpy(x).to(device), n_out)
        assert_close(got.cpu().numpy(), expected, what=f"shift={shift} rows={rows}")

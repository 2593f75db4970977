"""GPU parity of the GGUF decode and decode-time products (kdq_dequantize, kdq_gemv,
kdq_gemv_exact, kdq_gemv_batch) against the CPU oracle on identical seeded inputs.

Decoded weights must be bit-exact (NaN matches NaN, as IW/tests/gguf_quantization.cpp:21-29
compares); products within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the output RMS against
the oracle's double-accumulated product of exactly decoded weights.
"""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K = 2, 8, 12
BV = {Q4_0: 32, Q8_0: 32, Q4_K: 256}
BB = {Q4_0: 18, Q8_0: 34, Q4_K: 144}
ENCODINGS = [Q8_0, Q4_0, Q4_K]

# special fp16 scales: signed zeros, subnormals, normals, max, inf, NaNs
SPECIAL_HALVES = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x83FF, 0x0400, 0x8400, 0x3C00,
                  0xBC00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E01, 0x7C01]


def _torch():
    import torch
    return torch


def random_blocks(encoding, count, seed, specials=True):
    blocks = synth.random_bytes(seed, 7, count * BB[encoding]).reshape(count, BB[encoding])
    if specials:
        for i, h in enumerate(SPECIAL_HALVES[: count]):
            blocks[i, 0] = h & 0xFF
            blocks[i, 1] = h >> 8
            if encoding == Q4_K:
                h2 = SPECIAL_HALVES[len(SPECIAL_HALVES) - 1 - i]
                blocks[i, 2] = h2 & 0xFF
                blocks[i, 3] = h2 >> 8
    return blocks


def same_bits_or_nan(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    eq = a.view(np.uint32) == b.view(np.uint32)
    return bool(np.all(eq | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_dequantize_bit_exact(device, oracle, encoding):
    torch = _torch()
    count = 2048
    blocks = random_blocks(encoding, count, seed=0x31415926 + encoding)
    n_in = 8 * BV[encoding]  # 8 blocks per row
    rows = blocks.reshape(count // 8, 8 * BB[encoding])
    expected = oracle.dequantize(encoding, rows, n_in)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.dequantize(encoding, torch.from_numpy(rows).to(device), n_in, status=status)
    assert same_bits_or_nan(got.cpu().numpy(), expected)
    # the special scales include inf/NaN: the nonfinite flag must be raised
    assert int(status.item()) == 1


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_dequantize_finite_status_clear(device, oracle, encoding):
    torch = _torch()
    w = synth.gguf_weights(encoding, 11, 64, 1024)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.dequantize(encoding, torch.from_numpy(w).to(device), 1024, status=status)
    assert same_bits_or_nan(got.cpu().numpy(), oracle.dequantize(encoding, w, 1024))
    assert int(status.item()) == 0


SHAPES = [  # (rows, n_in, n_out)
    (1, 256, 1), (1, 256, 7), (1, 512, 64), (2, 1024, 33), (3, 2048, 100), (1, 4096, 257),
    (8, 4096, 64), (5, 14336, 40), (1, 14336, 130), (4, 8192, 96), (1, 12288, 17),
]


@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_gemv_parity(device, oracle, encoding, exact, shape):
    torch = _torch()
    rows, n_in, n_out = shape
    seed = hash((encoding, rows, n_in, n_out)) & 0xFFFF
    w = synth.gguf_weights(encoding, seed, n_out, n_in)
    x = synth.normal(seed, 50, rows * n_in).reshape(rows, n_in)
    expected = oracle.gemv(encoding, w, x, n_in, n_out)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.gemv(encoding, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device),
                   n_out, status=status, exact=exact)
    assert_close(got.cpu().numpy(), expected, what=f"enc={encoding} exact={exact} {shape}")
    assert int(status.item()) == 0


@pytest.mark.parametrize("encoding,n_in,n_out", [(Q8_0, 4096, 4096), (Q4_K, 4096, 14336),
                                                 (Q4_K, 14336, 4096), (Q4_0, 4096, 14336)])
def test_gemv_baseline_shapes(device, oracle, encoding, n_in, n_out):
    """The benchmark configurations' GEMV shapes (C1 Q8_0 4096x4096, C2 Q4_K 4096->14336 and
    14336->4096, and Q4_0 at C2's size) at full size, batch 1."""
    torch = _torch()
    w = synth.gguf_weights(encoding, 0xC2, n_out, n_in)
    x = synth.normal(0xC2, 50, n_in).reshape(1, n_in)
    expected = oracle.gemv(encoding, w, x, n_in, n_out)
    from kadan_amd import ops
    got = ops.gemv(encoding, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device),
                   n_out)
    assert_close(got.cpu().numpy(), expected, what=f"enc={encoding} {n_in}->{n_out}")


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_gemv_nonfinite_weight_status(device, encoding):
    torch = _torch()
    w = synth.gguf_weights(encoding, 3, 16, 512)
    w[5, 0], w[5, 1] = 0x00, 0x7C  # +inf scale in the first block of row 5
    from kadan_amd import ops
    for exact in (False, True):
        status = torch.zeros(1, dtype=torch.int32, device=device)
        y = ops.gemv(encoding, torch.from_numpy(w).to(device),
                     torch.ones(1, 512, device=device), 16, status=status, exact=exact)
        assert int(status.item()) == 1
        assert not np.isfinite(y.cpu().numpy()[0, 5])


def test_gemv_nonfinite_input_propagates(device):
    torch = _torch()
    w = synth.gguf_weights(Q4_K, 4, 8, 512)
    x = synth.normal(4, 1, 512).reshape(1, 512)
    x[0, 100] = np.inf
    from kadan_amd import ops
    y = ops.gemv(Q4_K, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device), 8)
    assert not np.isfinite(y.cpu().numpy()).any()


def test_gemv_zero_input(device):
    torch = _torch()
    w = synth.gguf_weights(Q8_0, 5, 8, 512)
    from kadan_amd import ops
    y = ops.gemv(Q8_0, torch.from_numpy(w).to(device), torch.zeros(2, 512, device=device), 8)
    assert np.all(y.cpu().numpy() == 0)


def test_gemv_output_stride(device, oracle):
    """Output rows land at r*stride, untouched columns stay as they were."""
    torch = _torch()
    w = synth.gguf_weights(Q4_K, 6, 20, 1024)
    x = synth.normal(6, 1, 3 * 1024).reshape(3, 1024)
    out = torch.full((3, 32), -7.0, device=device)
    from kadan_amd import ops
    ops.gemv(Q4_K, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device), 20, out=out)
    got = out.cpu().numpy()
    assert np.all(got[:, 20:] == -7.0)
    assert_close(got[:, :20], oracle.gemv(Q4_K, w, x, 1024, 20))


def test_gemv_batch_matches_single_calls(device, oracle):
    torch = _torch()
    jobs, expected = [], []
    shared = synth.normal(9, 1, 2 * 4096).reshape(2, 4096)
    xs = torch.from_numpy(shared).to(device)
    for i, (enc, n_out) in enumerate([(Q4_K, 100), (Q8_0, 64), (Q4_0, 33), (Q4_K, 7)]):
        w = synth.gguf_weights(enc, 20 + i, n_out, 4096)
        jobs.append({"encoding": enc, "weights": torch.from_numpy(w).to(device), "input": xs,
                     "output": torch.empty(2, n_out, device=device)})
        expected.append(oracle.gemv(enc, w, shared, 4096, n_out))
    from kadan_amd import ops
    ops.gemv_batch(jobs)
    for j, e in zip(jobs, expected):
        assert_close(j["output"].cpu().numpy(), e)


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_gemv_batch_fused_bit_identical(device, oracle, rows):
    """Jobs of one shape run as one fused launch (the reference runs a submission as one
    launch per format); every output must equal its own single kdq_gemv bit for bit.
    Mixed submission: 9 Q4_K gate/up-like jobs (over the 8-job launch limit) sharing one
    input, two Q8_0 jobs, a Q4_K job with another input, and a Q4_K job with in=4352
    (a different shape)."""
    torch = _torch()
    from kadan_amd import ops
    x = synth.normal(31, 1, rows * 4096).reshape(rows, 4096)
    x2 = synth.normal(32, 1, rows * 4096).reshape(rows, 4096)
    x3 = synth.normal(33, 1, rows * 4352).reshape(rows, 4352)
    xs, xs2, xs3 = (torch.from_numpy(a).to(device) for a in (x, x2, x3))
    specs = [(Q4_K, 1000 + 37 * i, xs, 40 + i) for i in range(9)]
    specs += [(Q8_0, 513, xs, 60), (Q8_0, 77, xs2, 61), (Q4_K, 300, xs2, 62),
              (Q4_K, 129, xs3, 63)]
    jobs, singles = [], []
    for enc, n_out, inp, seed in specs:
        n_in = inp.shape[1]
        w = torch.from_numpy(synth.gguf_weights(enc, seed, n_out, n_in)).to(device)
        jobs.append({"encoding": enc, "weights": w, "input": inp,
                     "output": torch.full((rows, n_out), -3.0, device=device)})
        singles.append(ops.gemv(enc, w, inp, n_out))
    ops.gemv_batch(jobs)
    for j, single in zip(jobs, singles):
        assert np.array_equal(j["output"].cpu().numpy().view(np.uint32),
                              single.cpu().numpy().view(np.uint32))
    # and one of them against the oracle
    w0 = synth.gguf_weights(Q4_K, 40, 1000, 4096)
    assert_close(jobs[0]["output"].cpu().numpy(), oracle.gemv(Q4_K, w0, x, 4096, 1000))


def test_gemv_rejects_alias_and_shape(device):
    torch = _torch()
    import kadan_amd
    from kadan_amd import ops
    w = torch.zeros(4, 144, dtype=torch.uint8, device=device)
    x = torch.zeros(1, 256, device=device)
    with pytest.raises(kadan_amd.KdqError, match="shape"):
        ops.gemv(Q4_K, w, torch.zeros(1, 200, device=device), 4)
    y = x[:, :4]  # output inside the input
    with pytest.raises(kadan_amd.KdqError, match="alias"):
        ops.gemv(Q4_K, w, x, 4, out=y)

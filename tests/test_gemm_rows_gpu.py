"""GPU parity of the prefill GEMM over row-major GGUF rows (kdq_gemm_rows): every encoding
through the one exact decoder, the weights rounded once to fp16 and the activations once
(after a per-row power-of-two scale), fp32 accumulation.

The reference's prefill is the fp32 product of exactly decoded weights (decode tile +
cublasSgemm, IW/src/cuda/h3_compute.cu:2201-2218,2451; IW =
services/hikari/inference_worker); the oracle's kdo_gemv is that product in double.
Outputs must be within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the output RMS.  At the
full prefill-chunk shape (512 tokens, 4096 -> 14336) the oracle runs on a sample of output
columns (each output column depends only on its own weight row)."""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q3_K, Q4_K, Q6_K = 2, 8, 11, 12, 14
IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, BF16 = 18, 20, 21, 22, 23, 30
ALL = [Q3_K, IQ4_XS, IQ4_NL, IQ3_XXS, IQ3_S, IQ2_S, BF16, Q4_0, Q4_K, Q8_0, Q6_K]


def run(device, oracle, enc, m, k, n, seed, cols=None):
    import torch
    from kadan_amd import ops
    w = synth.gguf_weights(enc, seed, n, k)
    x = synth.normal(seed, 7, m * k).reshape(m, k)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y = ops.gemm_rows(enc, torch.from_numpy(w).to(device), torch.from_numpy(x).to(device), n,
                      status=status).cpu().numpy()
    assert int(status.item()) == 0
    assert np.isfinite(y).all()
    if cols is None:
        want, got = oracle.gemv(enc, w, x, k, n), y
    else:
        pick = np.sort(np.random.default_rng(seed).choice(n, cols, replace=False))
        pick[-1] = n - 1
        want, got = oracle.gemv(enc, w[pick], x, k, len(pick)), y[:, pick]
    assert_close(got, want, what=f"gemm_rows enc={enc} m={m} k={k} n={n}")
    return y


@pytest.mark.parametrize("enc", ALL)
@pytest.mark.parametrize("m,k,n", [(9, 256, 40), (130, 1024, 300), (129, 768, 257),
                                   (200, 512, 302), (256, 2048, 128)])
def test_gemm_rows_shapes(device, oracle, enc, m, k, n):
    """Partial token and weight tiles (m, n not multiples of 128), n not a multiple of 4
    (scalar stores), one and several K groups."""
    run(device, oracle, enc, m, k, n, seed=0xA0 + enc + m + n)


def test_gemm_rows_bf16_k64(device, oracle):
    """BF16 stages 64-value groups: a k that is a multiple of 64 but not of 256."""
    run(device, oracle, BF16, 40, 192, 96, seed=0xA7)


@pytest.mark.parametrize("enc", [IQ4_XS, Q3_K, IQ2_S, BF16])
def test_gemm_rows_prefill_chunk(device, oracle, enc):
    """512 tokens, 4096 -> 14336 (a Llama-3-8B FFN prefill chunk), sampled columns."""
    run(device, oracle, enc, 512, 4096, 14336, seed=0xA8 + enc, cols=48)


def test_gemm_rows_matches_rows_run_apart(device):
    """Each token's output depends only on its own row (the tiles never mix rows): the
    first 9 rows of a 200-row product equal those rows run on their own."""
    import torch
    from kadan_amd import ops
    w = torch.from_numpy(synth.gguf_weights(IQ4_XS, 0xA9, 256, 1024)).to(device)
    x = torch.from_numpy(synth.normal(0xA9, 1, 200 * 1024).reshape(200, 1024)).to(device)
    a = ops.gemm_rows(IQ4_XS, w, x, 256).cpu().numpy()
    b = ops.gemm_rows(IQ4_XS, w, x[:9].contiguous(), 256).cpu().numpy()
    assert np.array_equal(a[:9], b)


def test_gemm_rows_flags(device):
    """A non-finite decoded weight sets bit 1, a weight past the fp16 range bit 2."""
    import torch
    from kadan_amd import ops
    x = torch.ones(16, 256, device=device)
    w = synth.gguf_weights(Q8_0, 0xAA, 32, 256).copy()
    w[5, 0], w[5, 1] = 0x00, 0x7C  # block 0 of row 5: d = +inf
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.gemm_rows(Q8_0, torch.from_numpy(w).to(device), x, 32, status=status)
    assert int(status.item()) & 1
    w = synth.gguf_weights(Q8_0, 0xAB, 32, 256).copy()
    w[7, 0], w[7, 1] = 0x00, 0x7B  # d = 57344: 57344 * |q| passes 65504 for |q| >= 2
    w[7, 2] = 100
    status.zero_()
    ops.gemm_rows(Q8_0, torch.from_numpy(w).to(device), x, 32, status=status)
    assert int(status.item()) == 2


def test_gemm_rows_rejections(device):
    import torch
    from kadan_amd import KdqError, KdqUnsupported, ops
    x = torch.ones(16, 256, device=device)
    w = torch.zeros(32, 110, dtype=torch.uint8, device=device)
    with pytest.raises(KdqUnsupported):
        ops.gemm_rows(0, torch.zeros(32, 1024, dtype=torch.uint8, device=device), x, 32)
    with pytest.raises(KdqError):  # k = 200 is not a whole number of groups
        ops.gemm_rows(Q3_K, w, torch.ones(16, 200, device=device), 32)
    with pytest.raises(KdqError):  # rows shorter than k needs
        ops.gemm_rows(Q3_K, torch.zeros(32, 100, dtype=torch.uint8, device=device), x, 32)


@pytest.mark.parametrize("enc", [Q3_K, IQ2_S, BF16, Q6_K])
def test_gemm_rows_padded_rows(device, oracle, enc):
    """Rows held with a stride longer than their data (row_bytes > the encoding's row),
    and K split into slices (few output tiles): the final row's last group comes from the
    staged tail copy, the other rows' from the weights in place."""
    import torch
    from kadan_amd import ops
    m, k, n = 64, 2048, 200
    w = synth.gguf_weights(enc, 0xAC + enc, n, k)
    padded = np.full((n, w.shape[1] + 6), 0xFF, dtype=np.uint8)
    padded[:, :w.shape[1]] = w
    x = synth.normal(0xAC, 3, m * k).reshape(m, k)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y = ops.gemm_rows(enc, torch.from_numpy(padded).to(device), torch.from_numpy(x).to(device),
                      n, status=status).cpu().numpy()
    assert int(status.item()) == 0
    assert_close(y, oracle.gemv(enc, w, x, k, n), what=f"gemm_rows padded enc={enc}")

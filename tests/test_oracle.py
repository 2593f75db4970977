"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against something other than itself:
  * the reference's own known answers, restated as data (IW/tests/gguf_quantization.cpp:
    36-91, IW/tests/quantization.cpp:97-351; IW = services/hikari/inference_worker);
  * vectors of the reference's compiled code (tests/golden/reference_vectors.npz, made by
    tests/golden/make_golden.py from oracle/_ref), and oracle/_ref itself when built here;
  * closed forms and independent formulations (numpy's IEEE conversions, vectorised
    decodes, float64 brute-force products, stable argsort) chosen so that a dropped
    term, a wrong sign or index, or a transposed operand fails.
"""
import os

import numpy as np
import pytest

from kadan_amd import synth

Q4_0, Q8_0, Q4_K = 2, 8, 12
Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16 = 11, 14, 20, 23, 30
IQ3_XXS, IQ3_S, IQ2_S = 18, 21, 22
NEW = [Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16, IQ3_XXS, IQ2_S, IQ3_S]
BV = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q3_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256, BF16: 1,
      IQ3_XXS: 256, IQ2_S: 256, IQ3_S: 256}
BB = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q3_K: 110, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136, BF16: 2,
      IQ3_XXS: 98, IQ2_S: 82, IQ3_S: 110}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q3_K: "q3_k", Q6_K: "q6_k",
         IQ4_NL: "iq4_nl", IQ4_XS: "iq4_xs", BF16: "bf16", IQ3_XXS: "iq3_xxs",
         IQ2_S: "iq2_s", IQ3_S: "iq3_s"}
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_vectors.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


# ---------------------------------------------------------------- fp16 / bf16

def test_half_to_float_exhaustive_vs_ieee(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.halves_to_float(bits)
    want = bits.view(np.float16).astype(np.float32)  # IEEE binary16 -> binary32, exact
    finite = ~np.isnan(want)
    assert np.array_equal(got.view(np.uint32)[finite], want.view(np.uint32)[finite])
    # NaN patterns decode to NaN of the same sign (the vectorised route multiplies by a
    # code of 1, which quiets signalling NaNs, as the reference decode does)
    assert np.isnan(got[~finite]).all()
    assert np.array_equal(np.signbit(got[~finite]), (bits[~finite] & 0x8000) != 0)


def test_half_to_float_vs_compiled_reference(oracle, reference):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.halves_to_float(bits)
    want = np.array([reference.half_to_float(int(b)) for b in bits], np.float32)
    assert same_bits(got, want)


def test_float_to_half_round_to_nearest_even(oracle):
    g = np.random.default_rng(1)
    x = np.concatenate([g.standard_normal(4000) * 10.0 ** g.integers(-8, 5, 4000),
                        [65504.0, 65519.9, 65520.0, 6.0e-8, 2.98e-8, 1.0 + 2.0 ** -11,
                         1.0 + 3 * 2.0 ** -11, -0.0]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)  # numpy: IEEE RNE
    got = np.array([oracle.float_to_half(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- GGUF decode

def half_bits(block, offset, bits):
    block[offset] = bits & 0xFF
    block[offset + 1] = bits >> 8


def test_q8_0_literal_block(oracle):
    """IW/tests/gguf_quantization.cpp:37-44: d = 0.5, codes 0..15 then -16..-31."""
    block = np.zeros(34, np.uint8)
    half_bits(block, 0, 0x3800)
    for i in range(32):
        block[2 + i] = i if i < 16 else 256 - i
    want = np.array([0.5 * (i if i < 16 else -i) for i in range(32)], np.float32)
    assert same_bits(oracle.dequantize(Q8_0, block[None], 32)[0], want)


def test_q4_k_literal_block(oracle):
    """IW/tests/gguf_quantization.cpp:61-78: d = 2, dmin = 0.5, packed scales 1..8 and
    mins 8..1, every code byte 0xc3 (low nibble 3, high nibble 12)."""
    block = np.zeros(144, np.uint8)
    half_bits(block, 0, 0x4000)
    half_bits(block, 2, 0x3800)
    block[4:16] = [1, 2, 3, 4, 8, 7, 6, 5, 0x45, 0x36, 0x27, 0x18]
    block[16:] = 0xC3
    g = np.arange(256) // 32
    want = (2.0 * (g + 1) * np.where(g % 2, 12.0, 3.0) - 0.5 * (8 - g)).astype(np.float32)
    assert same_bits(oracle.dequantize(Q4_K, block[None], 256)[0], want)


def test_q4_0_literal_block(oracle):
    """G/src/ggml-quants.c:459-476: value j is the low nibble of byte j, value j+16 its
    high nibble, w = (q - 8) * d."""
    block = np.zeros(18, np.uint8)
    half_bits(block, 0, 0xC000)  # d = -2
    block[2:] = [(15 - j) << 4 | j for j in range(16)]
    q = np.concatenate([np.arange(16), 15 - np.arange(16)])
    assert same_bits(oracle.dequantize(Q4_0, block[None], 32)[0],
                     ((q - 8) * -2.0).astype(np.float32))


def test_q3_k_literal_block(oracle):
    """IW/tests/gguf_quantization.cpp:46-59: high-bit bytes 0x55 (bit j set for even j),
    code bytes 0xe4 (fields 0, 1, 2, 3 in consecutive 32-value groups), scale nibbles 1
    and high scale bits 2 (every 6-bit scale 33 - 32 = +1), d = -2."""
    block = np.zeros(110, np.uint8)
    block[0:32] = 0x55
    block[32:96] = 0xE4
    block[96:104] = 0x11
    block[104:108] = 0xAA
    half_bits(block, 108, 0xC000)
    g = np.arange(256) // 32
    code = g % 4 - np.where(g % 2, 4, 0)
    assert same_bits(oracle.dequantize(Q3_K, block[None], 256)[0],
                     (-2.0 * code).astype(np.float32))


def test_q6_k_literal_block(oracle):
    """Closed form of the Q6_K layout: low nibbles 5 / high nibbles 9 (ql bytes 0x95),
    high pairs 0b11100100 (fields 0, 1, 2, 3 for quarters 0..3), int8 scales s = 1..16
    alternating in sign, d = 0.25: value v of half k, quarter q, lane l has code
    (nibble | field << 4) - 32 and scale s[8k + l/16 + 2q]."""
    block = np.zeros(210, np.uint8)
    block[0:128] = 0x95
    block[128:192] = 0xE4
    scales = np.array([(i + 1) * (-1) ** i for i in range(16)], np.int8)
    block[192:208] = scales.view(np.uint8)
    half_bits(block, 208, 0x3400)
    v = np.arange(256)
    k, q, l = v // 128, (v % 128) // 32, v % 32
    nibble = np.where(q < 2, 5, 9)
    code = (nibble | (q << 4)) - 32
    s = scales[8 * k + l // 16 + 2 * q].astype(np.float32)
    assert same_bits(oracle.dequantize(Q6_K, block[None], 256)[0],
                     ((0.25 * s) * code).astype(np.float32))


def test_iq4_literal_blocks(oracle):
    """IQ4_NL / IQ4_XS code points are ggml's kvalues_iq4nl (G/src/ggml-common.h:1120-1122):
    index i in byte 2 + i (low nibble) and its high nibble decode to d * grid."""
    grid = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89,
                     113], np.float32)
    block = np.zeros(18, np.uint8)
    half_bits(block, 0, 0x3C00)  # d = 1
    block[2:] = [(15 - j) << 4 | j for j in range(16)]
    want = np.concatenate([grid, grid[::-1]])
    assert same_bits(oracle.dequantize(IQ4_NL, block[None], 32)[0], want)
    # IQ4_XS: sub-block s has scale (low nibble s % 16) | (high bits 2) << 4 minus 32 =
    # s + 0; d = 0.5; every index byte 0x70 (low 0, high 7)
    xs = np.zeros(136, np.uint8)
    half_bits(xs, 0, 0x3800)
    xs[2], xs[3] = 0xAA, 0xAA  # high bits 2 for every sub-block: +32
    xs[4:8] = [0x10, 0x32, 0x54, 0x76]  # low nibbles 0..7
    xs[8:] = 0x70
    s = np.repeat(np.arange(8), 32).astype(np.float32)
    idx = np.tile(np.concatenate([np.zeros(16, int), np.full(16, 7)]), 8)
    assert same_bits(oracle.dequantize(IQ4_XS, xs[None], 256)[0],
                     ((0.5 * s) * grid[idx]).astype(np.float32))


def test_bf16_is_the_upper_half_of_binary32(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.dequantize(BF16, bits.view(np.uint8)[None], 65536)[0]
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    assert same_bits(got, want)


@pytest.mark.parametrize("encoding", NEW)
def test_new_formats_vs_reference_vectors(oracle, golden, encoding):
    """ggml to_float of the same blocks (specials included; kadan::gguf::decode equal to
    it on every block, checked when the fixture was made).  For the IQ grid formats the
    256 blocks draw every grid entry, pinning the re-encoded grid tables."""
    blocks = golden[f"decode_{NAMES[encoding]}_blocks"]
    got = oracle.dequantize(encoding, blocks, BV[encoding])
    assert same_bits(got, golden[f"decode_{NAMES[encoding]}_values"])


def test_iq_grid_fixture_draws_every_entry(golden):
    """The golden IQ blocks index every entry of each grid at least once (so a wrong
    entry of a re-encoded table cannot pass test_new_formats_vs_reference_vectors)."""
    b = golden["decode_iq2_s_blocks"].astype(np.int64)
    q = np.arange(4)
    idx = b[:, 2:34].reshape(-1, 8, 4) | ((b[:, 66:74, None] << (8 - 2 * q)) & 0x300)
    assert np.unique(idx).size == 1024
    b = golden["decode_iq3_xxs_blocks"]
    assert np.unique(b[:, 2:66]).size == 256
    b = golden["decode_iq3_s_blocks"].astype(np.int64)
    lo = b[:, 2:66].reshape(-1, 8, 4, 2)
    shift = (8 - 2 * q[:, None] - np.arange(2)[None, :])
    idx = lo | ((b[:, 66:74, None, None] << shift) & 256)
    assert np.unique(idx).size == 512


@pytest.mark.parametrize("encoding", NEW)
def test_new_formats_vs_compiled_reference(oracle, reference, encoding):
    count = 2048 if encoding != BF16 else 65536
    raw = synth.random_bytes(13, encoding, count * BB[encoding])
    if encoding in (Q3_K, Q6_K):  # finite scales at the format's offset
        at = 108 if encoding == Q3_K else 208
        raw.reshape(count, -1)[:, at + 1] = 0x10 + (raw.reshape(count, -1)[:, at + 1] & 0x1F)
    got = oracle.dequantize(encoding, raw[None], count * BV[encoding])
    assert same_bits(got, reference.to_float(encoding, raw[None], count * BV[encoding]))
    step = BB[encoding]
    for b in range(0, 64):
        blk = raw[b * step:(b + 1) * step]
        mine = oracle.dequantize(encoding, blk[None], BV[encoding])[0]
        assert same_bits(mine, reference.kadan_decode_block(encoding, blk))


def numpy_decode(encoding, blocks):
    """Independent vectorised decode (float32 numpy ops, each one rounded)."""
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    if encoding == Q8_0:
        return blocks[:, 2:].view(np.int8).astype(np.float32) * d[:, None]
    if encoding == Q4_0:
        qs = blocks[:, 2:]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int32) - 8
        return q.astype(np.float32) * d[:, None]
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = blocks[:, 4:16].astype(np.int32)
    sc = np.empty((len(blocks), 8), np.int32)
    mn = np.empty((len(blocks), 8), np.int32)
    sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = blocks[:, 16:].reshape(-1, 4, 32).astype(np.int32)
    codes = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block g
    scaled = (d[:, None] * sc.astype(np.float32))[:, :, None]
    offset = (dmin[:, None] * mn.astype(np.float32))[:, :, None]
    return (scaled * codes.astype(np.float32) - offset).reshape(-1, 256)


@pytest.mark.parametrize("encoding", [Q4_0, Q8_0, Q4_K])
def test_decode_vs_independent_numpy(oracle, encoding):
    raw = synth.random_bytes(7, encoding, 512 * BB[encoding]).reshape(512, BB[encoding])
    raw[:, 1] = 0x10 + (raw[:, 1] & 0x1F)  # finite scales of many magnitudes
    if encoding == Q4_K:
        raw[:, 3] = 0x10 + (raw[:, 3] & 0x1F)
    with np.errstate(over="ignore", invalid="ignore"):
        want = numpy_decode(encoding, raw)
    got = oracle.dequantize(encoding, raw.reshape(64, -1), 8 * BV[encoding]).reshape(512, -1)
    assert same_bits(got, want)


@pytest.mark.parametrize("encoding", [Q4_0, Q8_0, Q4_K])
def test_decode_vs_reference_vectors(oracle, golden, encoding):
    blocks = golden[f"decode_{NAMES[encoding]}_blocks"]
    want = golden[f"decode_{NAMES[encoding]}_values"]
    got = oracle.dequantize(encoding, blocks, BV[encoding])
    assert same_bits(got, want)


@pytest.mark.parametrize("encoding", [Q4_0, Q8_0, Q4_K])
def test_decode_vs_compiled_reference(oracle, reference, encoding):
    raw = synth.random_bytes(11, encoding, 2048 * BB[encoding])
    got = oracle.dequantize(encoding, raw[None], 2048 * BV[encoding])
    want = reference.to_float(encoding, raw[None], 2048 * BV[encoding])
    assert same_bits(got, want)
    if encoding != Q4_0:  # kadan's own decode (no Q4_0 encoding in the reference)
        for b in range(0, 64):
            blk = raw[b * BB[encoding]:(b + 1) * BB[encoding]]
            mine = oracle.dequantize(encoding, blk[None], BV[encoding])[0]
            assert same_bits(mine, reference.kadan_decode_block(encoding, blk))


# ---------------------------------------------------------------- quantizers

def test_quantize_q8_0_vs_reference_vectors(oracle, golden):
    x = golden["q8_0_x"]
    ref = golden["q8_0_bytes"].reshape(-1, 34)
    qs, d = oracle.quantize_row_q8_0(x)
    assert np.array_equal(qs, ref[:, 2:].view(np.int8).ravel())
    assert np.array_equal(d, ref[:, :2].copy().view(np.uint16).ravel())


def test_quantize_q8_0_ties_round_to_even(oracle):
    x = np.zeros(32, np.float32)
    x[:5] = [127.0, 0.5, 1.5, -2.5, 3.5]  # amax 127: id = 1, codes = RNE(x)
    qs, d = oracle.quantize_row_q8_0(x)
    assert list(qs[:5]) == [127, 0, 2, -2, 4]
    assert d[0] == np.float16(1.0).view(np.uint16)
    qs, d = oracle.quantize_row_q8_0(np.zeros(32, np.float32))
    assert not qs.any() and d[0] == 0


def test_quantize_q8_K_vs_reference_vectors(oracle, golden):
    x = golden["q8_K_x"]
    ref = golden["q8_K_bytes"].reshape(2, -1)
    qs, d, bsums = oracle.quantize_row_q8_K(x)
    assert np.array_equal(d, ref[:, :4].copy().view(np.float32).ravel())
    assert np.array_equal(qs, ref[:, 4:260].view(np.int8).ravel())
    assert np.array_equal(bsums, ref[:, 260:].copy().view(np.int16).ravel())
    # bsums are sums of 16 codes (a closed form the reference states)
    assert np.array_equal(bsums, qs.reshape(-1, 16).astype(np.int32).sum(1))


def test_quantize_q8_f16_is_x86_q8_0_with_fp32_scale(oracle):
    """The prefill quantizer: x86 quantize_row_q8_0 codes on fp32(x_half), d = amax/127
    kept in fp32 (not rounded to fp16)."""
    xh = (synth.normal(3, 1, 4 * 256) * 3).astype(np.float16).reshape(4, 256)
    xh[0, :32] = 0
    qs, d = oracle.quantize_q8_f16(xh.view(np.uint16))
    for r in range(4):
        q_row, _ = oracle.quantize_row_q8_0(xh[r].astype(np.float32))
        assert np.array_equal(qs[r], q_row)
    amax = np.abs(xh.astype(np.float32)).reshape(4, -1, 32).max(2)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))


# ---------------------------------------------------------------- dots and products

@pytest.mark.parametrize("encoding", [Q8_0, Q4_0, Q4_K])
def test_vec_dot_vs_reference_vectors_and_closed_form(oracle, golden, encoding):
    w = golden[f"dot_{NAMES[encoding]}_w"]
    xq = golden[f"dot_{NAMES[encoding]}_x"]
    want = golden[f"dot_{NAMES[encoding]}_out"]
    n = 512
    for r in range(4):
        if encoding == Q4_K:
            blk = xq[r].reshape(2, 292)
            d = blk[:, :4].copy().view(np.float32).ravel()
            qs = blk[:, 4:260].view(np.int8).ravel()
            bs = blk[:, 260:].copy().view(np.int16).ravel()
            got = oracle.vec_dot(encoding, w[r], qs, d, bs)
            xs = np.repeat(d.astype(np.float64), 256) * qs
        else:
            blk = xq[r].reshape(-1, 34)
            d = blk[:, :2].copy().view(np.uint16).ravel()
            qs = blk[:, 2:].view(np.int8).ravel()
            got = oracle.vec_dot(encoding, w[r], qs, d)
            xs = np.repeat(d.view(np.float16).astype(np.float64), 32) * qs
        # AVX2 summation order differs from the scalar restatement: fp32 tolerance
        assert abs(got - want[r]) <= 1e-5 * max(1.0, abs(want[r])), (r, got, want[r])
        exact = float(oracle.dequantize(encoding, w[r][None], n)[0].astype(np.float64) @ xs)
        assert abs(got - exact) <= 1e-4 * max(1.0, abs(exact))


@pytest.mark.parametrize("encoding", [Q8_0, Q4_0, Q4_K])
def test_cpu_matvec_port_vs_reference_vectors(oracle, golden, encoding):
    w = golden[f"matvec_{NAMES[encoding]}_w"]
    x = golden[f"matvec_{NAMES[encoding]}_x"]
    want = golden[f"matvec_{NAMES[encoding]}_y"]
    got = oracle.cpu_matvec(encoding, w, x, 512, 96, threads=2)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


@pytest.mark.parametrize("encoding", [Q8_0, Q4_0, Q4_K])
def test_gemv_is_float64_product_of_decoded_weights(oracle, encoding):
    n_in, n_out = 512, 48
    w = synth.gguf_weights(encoding, 5, n_out, n_in)
    x = synth.normal(5, 9, 3 * n_in).reshape(3, n_in)
    decoded = oracle.dequantize(encoding, w, n_in).astype(np.float64)
    want = x.astype(np.float64) @ decoded.T
    got = oracle.gemv(encoding, w, x, n_in, n_out)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    # a transposed or shifted operand is far off
    assert np.abs(got - x.astype(np.float64) @ np.roll(decoded, 1, axis=0).T).max() > 1e-3


def test_gemm_q4_0_q8_is_float64_product(oracle):
    m, k, n = 5, 256, 40
    w = synth.q4_0_weights(6, n, k)
    xh = synth.normal(6, 1, m * k).reshape(m, k).astype(np.float16)
    qs, d = oracle.quantize_q8_f16(xh.view(np.uint16))
    xdeq = qs.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)
    want = xdeq @ oracle.dequantize(Q4_0, w, k).astype(np.float64).T
    got = oracle.gemm_q4_0_q8(w, n, k, qs, d)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


# ---------------------------------------------------------------- MXFP4

def test_e2m1_golden_table(oracle):
    """IW/tests/quantization.cpp:97-105."""
    table = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    for code, v in enumerate(table):
        got = oracle.e2m1(code)
        assert got == v and np.signbit(got) == (code >= 8)


def test_mxfp4_two_by_sixty_four_fixture(oracle):
    """IW/tests/quantization.cpp:250-270: low nibble first, one exponent per 32."""
    packed = np.full(64, 0xA2, np.uint8)
    packed[0] = 0x71
    scales = np.array([127, 128, 126, 129], np.uint8)
    factor = np.repeat([1.0, 2.0, 0.5, 4.0], 32)
    want = np.where(np.arange(128) % 2, -factor, factor).astype(np.float32)
    want[0], want[1] = 0.5, 6.0
    rc, got = oracle.mxfp4_decode_rows(packed.reshape(2, 32), scales.reshape(2, 2), 2, 64)
    assert rc == 0 and np.array_equal(got.ravel(), want)
    bad = scales.copy()
    bad[3] = 255  # invalid E8M0
    rc, _ = oracle.mxfp4_decode_rows(packed.reshape(2, 32), bad.reshape(2, 2), 2, 64)
    assert rc != 0


def test_mxfp4_extremes(oracle):
    """IW/tests/quantization.cpp:293-317."""
    packed = np.full(16, 0xA2, np.uint8)

    def decode(p, s):
        return oracle.mxfp4_decode_rows(p.reshape(1, 16), np.array([[s]], np.uint8), 1, 32)

    rc, v = decode(packed, 0)
    assert rc == 0 and v[0, 0] == 2.0 ** -127 and v[0, 1] == -(2.0 ** -127)
    rc, v = decode(packed, 254)
    assert rc == 0 and v[0, 0] == 2.0 ** 127 and v[0, 1] == -(2.0 ** 127)
    p = packed.copy()
    p[0] = 0x11
    rc, v = decode(p, 0)
    assert rc == 0 and v[0, 0] == 2.0 ** -128
    zeros = np.full(16, 0x80, np.uint8)
    for s in (0, 127, 254):
        rc, v = decode(zeros, s)
        assert rc == 0 and v[0, 0] == 0 and not np.signbit(v[0, 0]) and np.signbit(v[0, 1])
    p = packed.copy()
    p[0] = 0x77
    rc, _ = decode(p, 253)  # 6 * 2^126 overflows: the reference refuses it
    assert rc != 0


def test_mxfp4_matvec_known_answer(oracle):
    """IW/tests/quantization.cpp:319-330: 2x32, x = (3, 1, 0...), y = {2, 8}."""
    packed = np.full(32, 0xA2, np.uint8).reshape(2, 16)
    scales = np.array([[127], [129]], np.uint8)
    x = np.zeros(32, np.float32)
    x[0], x[1] = 3, 1
    rc, y = oracle.mxfp4_matvec(packed, scales, 2, 32, x)
    assert rc == 0 and list(y) == [2.0, 8.0]


def test_mxfp4_vs_reference_vectors(oracle, golden):
    rc, v = oracle.mxfp4_decode_rows(golden["mxfp4_blocks"], golden["mxfp4_scales"], 8, 128)
    assert rc == 0 and np.array_equal(v.view(np.uint32), golden["mxfp4_values"].view(np.uint32))
    rc, y = oracle.mxfp4_matvec(golden["mxfp4_blocks"], golden["mxfp4_mv_scales"], 8, 128,
                                golden["mxfp4_x"])
    assert rc == 0 and np.array_equal(y.view(np.uint32), golden["mxfp4_y"].view(np.uint32))


def test_mxfp4_vs_compiled_reference(oracle, reference):
    blocks = synth.random_bytes(8, 1, 16 * 128).reshape(16, 128)
    scales = (synth.random_bytes(8, 2, 16 * 8) % 24 + 116).astype(np.uint8).reshape(16, 8)
    x = synth.normal(8, 3, 256)
    a, b = oracle.mxfp4_decode_rows(blocks, scales, 16, 256), reference.mxfp4_decode_rows(
        blocks, scales, 16, 256)
    assert a[0] == b[0] == 0 and np.array_equal(a[1], b[1])
    a, b = oracle.mxfp4_matvec(blocks, scales, 16, 256, x), reference.mxfp4_matvec(
        blocks, scales, 16, 256, x)
    assert a[0] == b[0] == 0 and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


# ---------------------------------------------------------------- MoE routing

def brute_route(logits, top_k):
    """Router of IW/src/models/text/qwen_layers.cpp:403-425 restated with numpy."""
    idx = np.empty((len(logits), top_k), np.int32)
    w = np.empty((len(logits), top_k), np.float32)
    for t, row in enumerate(logits.astype(np.float32)):
        e = np.exp(row - row.max()).astype(np.float32)
        p = (e.astype(np.float64) / e.astype(np.float64).sum()).astype(np.float32)
        order = np.argsort(-p, kind="stable")[:top_k]  # callers keep ties out
        idx[t] = order
        s = np.float32(0)
        for v in p[order]:
            s = np.float32(s + v)
        w[t] = p[order] / max(s, np.float32(6.103515625e-5))
    return idx, w


def test_route_hand_case(oracle):
    # probabilities proportional to 1, 2, 3, 4: top-2 = experts 3, 2 with weights 4/7, 3/7
    logits = np.log(np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float64)).astype(np.float32)
    idx, w = oracle.moe_route(logits, 2)
    assert idx.tolist() == [[3, 2], [0, 1]]
    np.testing.assert_allclose(w, [[4 / 7, 3 / 7], [4 / 7, 3 / 7]], rtol=1e-6)


def test_route_ties_follow_the_library_heap(oracle):
    """Equal probabilities come out in the order of libstdc++'s std::partial_sort (heap
    selection, then sort_heap), not by expert number.  Worked by hand through the heap
    steps: with 16 equal probabilities make_heap turns order [0, 1, 2, 3] into
    [2, 3, 0, 1] and sort_heap pops it as [1, 3, 0, 2]."""
    logits = np.zeros((2, 16), np.float32)
    logits[1] = [1, 0, 0, 0, -5, 1, 0, 0, -5, 1, 0, 0, 1, 0, 0, 0]
    idx, w = oracle.moe_route(logits[:1], 4)
    assert idx.tolist() == [[1, 3, 0, 2]]
    np.testing.assert_allclose(w, 0.25, rtol=1e-6)
    idx, _ = oracle.moe_route(logits[1:, :13], 8)
    # the four logits of 1 first (heap order), then four of the zeros: expert 7, not 6
    assert idx.tolist() == [[12, 0, 5, 9, 3, 7, 1, 2]]


def test_route_masked_experts(oracle):
    logits = np.full((1, 6), -np.inf, np.float32)
    logits[0, 3] = 0.0
    idx, w = oracle.moe_route(logits, 3)
    assert idx[0, 0] == 3 and w[0].tolist() == [1.0, 0.0, 0.0]


ROUTE_CASES = [(4, 4), (6, 3), (13, 8), (16, 4), (32, 4), (128, 4), (256, 8)]


@pytest.mark.parametrize("experts,top_k", ROUTE_CASES)
def test_route_ties_vs_reference_vectors(oracle, golden, experts, top_k):
    """Tie-heavy logits (NaN and +-inf in some rows) against std::partial_sort's output
    recorded from the compiled reference bindings: indices and weights bit for bit."""
    key = f"route_{experts}_{top_k}"
    idx, w = oracle.moe_route(golden[f"{key}_logits"], top_k)
    assert np.array_equal(idx, golden[f"{key}_idx"])
    assert same_bits(w, golden[f"{key}_w"])


def test_route_ties_vs_compiled_library(oracle, reference):
    """Random tie patterns against std::partial_sort itself, over every expert count
    from 1 to 140 and top_k up to 8."""
    rng = np.random.default_rng(77)
    values = np.array([0, 1, 2, -1, -np.inf, np.nan, np.inf], np.float32)
    for trial in range(3000):
        experts = int(rng.integers(1, 141))
        top_k = int(rng.integers(1, min(experts, 8) + 1))
        p = [.3, .3, .2, .1, .05, .03, .02] if trial % 3 == 0 else [.4, .3, .2, .1, 0, 0, 0]
        logits = rng.choice(values, size=(2, experts), p=p).astype(np.float32)
        a, b = oracle.moe_route(logits, top_k), reference.moe_route(logits, top_k)
        assert np.array_equal(a[0], b[0]), (logits, top_k)
        assert same_bits(a[1], b[1])


@pytest.mark.parametrize("experts,top_k", [(32, 4), (128, 8)])
def test_route_near_ties_vs_reference_vectors(oracle, golden, experts, top_k):
    """Logits a few ulps apart at the top-k boundary (tests/util.py near_tie_logits):
    indices and weights bit for bit against the compiled reference's router.  The order
    rests on the last bits of expf, of the double total and of the division."""
    key = f"route_near_{experts}_{top_k}"
    idx, w = oracle.moe_route(golden[f"{key}_logits"], top_k)
    assert np.array_equal(idx, golden[f"{key}_idx"])
    assert same_bits(w, golden[f"{key}_w"])


def test_route_near_ties_vs_compiled_library(oracle, reference):
    """20000 fresh near-tie rows per configuration against the compiled reference."""
    from tests.util import near_tie_logits
    for experts, top_k, seed in ((32, 4, 0x7138), (128, 8, 0x7139), (256, 8, 0x713A)):
        logits = near_tie_logits(seed, 20000, experts, top_k)
        a, b = oracle.moe_route(logits, top_k), reference.moe_route(logits, top_k)
        assert np.array_equal(a[0], b[0])
        assert same_bits(a[1], b[1])


def test_route_orders_by_probability_not_logit(oracle):
    # logits 0 and 1e-8 differ, their float probabilities do not (expf(-1e-8) rounds to
    # 1): they tie, and the heap order decides (std::partial_sort over 8 experts, top 3)
    assert np.float32(np.exp(np.float32(-1e-8))) == np.float32(1.0)
    logits = np.full((1, 8), -5.0, np.float32)
    logits[0, [2, 5]] = [0.0, 1e-8]
    logits[0, 6] = 1e-8
    idx, _ = oracle.moe_route(logits, 3)
    assert sorted(idx[0].tolist()) == [2, 5, 6]


@pytest.mark.parametrize("tokens,experts,top_k", [(64, 8, 2), (50, 32, 4), (20, 128, 8)])
def test_route_vs_numpy(oracle, tokens, experts, top_k):
    _, logits = synth.moe_inputs(9 + experts, tokens, 32, experts, hot=4 if experts > 8 else 0)
    idx, w = oracle.moe_route(logits, top_k)
    bi, bw = brute_route(logits, top_k)
    assert np.array_equal(idx, bi)
    # numpy's float32 exp may differ from the C library's expf by an ulp
    np.testing.assert_allclose(w, bw, rtol=5e-7, atol=0)
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


@pytest.mark.parametrize("tokens,experts,top_k", [(1, 4, 2), (37, 8, 4), (300, 64, 8)])
def test_permute_is_stable_sort_by_expert(oracle, tokens, experts, top_k):
    _, logits = synth.moe_inputs(10, tokens, 32, experts)
    idx, _ = oracle.moe_route(logits, top_k)
    offsets, perm = oracle.moe_permute(idx, experts)
    assert np.array_equal(perm, np.argsort(idx.ravel(), kind="stable"))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(idx.ravel(),
                                                                              minlength=experts))]))


def test_moe_forward_known_answer(oracle):
    """The composed layer against a case worked out by hand from MoeLayer::forward's
    definition (tests/util.py known_answer_moe: 2 tokens x 4 experts, closed form)."""
    from tests.util import known_answer_moe
    x, logits, ((gb, gs), (ub, us), (db, ds)), y, idx = known_answer_moe()
    got, gi, gw, _, _ = oracle.moe_forward(x, logits, 2, gb, gs, ub, us, db, ds)
    assert np.array_equal(gi, idx)
    np.testing.assert_allclose(got, y, rtol=1e-6, atol=0)


def test_moe_forward_vs_numpy_composition(oracle):
    """MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:378-492) composed in float64
    from pinned parts.  The reference never runs MXFP4 weights through MoeLayer, so the
    whole is pinned by the closed-form case above, and this checks the composition at a
    size that case does not reach."""
    tokens, hidden, inter, experts, top_k = 6, 64, 96, 4, 2
    x, logits = synth.moe_inputs(12, tokens, hidden, experts)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(12, experts, hidden, inter)
    y, idx, w, _, _ = oracle.moe_forward(x, logits, top_k, gb, gs, ub, us, db, ds)
    xf = synth.bf16_bits_to_float(x).astype(np.float64)

    def dec(b, s, rows, cols, e):
        rc, v = oracle.mxfp4_decode_rows(b[e].reshape(rows, -1), s[e].reshape(rows, -1), rows,
                                         cols)
        assert rc == 0
        return v.astype(np.float64)

    want = np.zeros((tokens, hidden))
    for t in range(tokens):
        for i in range(top_k):
            e = idx[t, i]
            g = dec(gb, gs, inter, hidden, e) @ xf[t]
            u = dec(ub, us, inter, hidden, e) @ xf[t]
            h = g / (1 + np.exp(-g)) * u
            want[t] += (dec(db, ds, hidden, inter, e) @ h) * w[t, i]
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    # dropping the routing weight, or the up projection, is far off
    assert np.abs(y - want / np.maximum(w.max(), 1e-9)).max() > 1e-4 * np.abs(want).max()


# ---------------------------------------------------------------- GGUF MoE layer

def _moe_numpy(spec_f32, x):
    """Independent float64 restatement of MoeLayer::forward (IW/src/models/text/
    qwen_layers.cpp:378-492) over already-decoded weights."""
    r, ge, ue, de, gs, us, ds, sg = (spec_f32[k].astype(np.float64) for k in
                                     ("router", "gate_exps", "up_exps", "down_exps",
                                      "gate_shexp", "up_shexp", "down_shexp", "shared_gate"))
    K = spec_f32["top_k"]
    X = x.astype(np.float64)
    silu = lambda v: v / (1 + np.exp(-v))
    logits = X @ r.T
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sel = np.argsort(-p, axis=1, kind="stable")[:, :K]
    pw = np.take_along_axis(p, sel, 1)
    pw /= np.maximum(pw.sum(1, keepdims=True), 6.103515625e-5)
    Y = np.zeros((x.shape[0], r.shape[1]))
    for t in range(x.shape[0]):
        for i in range(K):
            e = sel[t, i]
            Y[t] += (de[e] @ (silu(ge[e] @ X[t]) * (ue[e] @ X[t]))) * pw[t, i]
        gate = 1 / (1 + np.exp(-(sg @ X[t])))
        Y[t] += (ds @ (silu(gs @ X[t]) * (us @ X[t]))) * gate
    return Y, sel, pw


def test_moe_gguf_forward_vs_numpy(oracle):
    """The composition (routing, SwiGLU, selection weights, the sigmoid-gated shared
    expert) against an independent numpy restatement, with F32 weights and with Q4_K / Q6_K /
    Q8_0 weights decoded by the (separately pinned) oracle decode."""
    H, E, K, F, S = 256, 6, 2, 256, 256
    g = np.random.default_rng(5)
    x = g.standard_normal((3, H)).astype(np.float32)
    f32 = {"router": g.standard_normal((E, H)).astype(np.float32),
           "gate_exps": (g.standard_normal((E, F, H)) * 0.05).astype(np.float32),
           "up_exps": (g.standard_normal((E, F, H)) * 0.05).astype(np.float32),
           "down_exps": (g.standard_normal((E, H, F)) * 0.05).astype(np.float32),
           "gate_shexp": (g.standard_normal((S, H)) * 0.05).astype(np.float32),
           "up_shexp": (g.standard_normal((S, H)) * 0.05).astype(np.float32),
           "down_shexp": (g.standard_normal((H, S)) * 0.05).astype(np.float32)}
    sg = (g.standard_normal(H) * 0.05).astype(np.float32)
    spec = dict(hidden=H, experts=E, top_k=K, ff=F, shared_ff=S, shared_gate=sg,
                **{k: (0, v.view(np.uint8).reshape(*v.shape[:-1], -1)) for k, v in f32.items()})
    y, idx, w = oracle.moe_gguf_forward(spec, x)
    Y, sel, pw = _moe_numpy(dict(f32, shared_gate=sg, top_k=K), x)
    assert np.array_equal(idx, sel)
    assert np.abs(w - pw).max() < 1e-6
    assert np.abs(y - Y).max() <= 1e-5 * np.abs(Y).max()
    # quantized tensors: the same composition over the oracle's decode of them
    encs = {"router": Q8_0, "gate_exps": Q4_K, "up_exps": Q4_K, "down_exps": Q6_K,
            "gate_shexp": Q8_0, "up_shexp": Q8_0, "down_shexp": Q4_K}
    qspec = dict(hidden=H, experts=E, top_k=K, ff=F, shared_ff=S, shared_gate=sg)
    decoded = {}
    for i, (name, enc) in enumerate(encs.items()):
        shape = f32[name].shape
        rows = int(np.prod(shape[:-1]))
        packed = synth.gguf_weights(enc, 40 + i, rows, shape[-1])
        qspec[name] = (enc, packed.reshape(*shape[:-1], -1))
        decoded[name] = oracle.dequantize(enc, packed, shape[-1]).reshape(shape)
    decoded["router"] *= 300.0  # well-separated routing logits
    qspec["router"] = (0, decoded["router"].astype(np.float32).view(np.uint8).reshape(E, -1))
    y, idx, w = oracle.moe_gguf_forward(qspec, x)
    Y, sel, pw = _moe_numpy(dict(decoded, shared_gate=sg, top_k=K), x)
    assert np.array_equal(idx, sel)
    assert np.abs(y - Y).max() <= 1e-5 * np.abs(Y).max()


def test_moe_gguf_forward_known_answer(oracle):
    """The oracle's GGUF MoE composition against the closed form of MoeLayer::forward with
    its sigmoid-gated shared expert (tests/util.py known_answer_moe_gguf), which no oracle
    code computes; the shared term is a large part of y, so dropping it, or its gate,
    would fail."""
    from tests.util import known_answer_moe_gguf
    spec, x, want, idx = known_answer_moe_gguf()
    y, got_idx, w = oracle.moe_gguf_forward(spec, x)
    assert np.array_equal(got_idx, idx)
    assert np.abs(y - want).max() <= 1e-6 * np.abs(want).max()
    # the closed form's parts are each large against that tolerance: the shared term
    silu = lambda a: a / (1 + np.exp(-a))
    for t, v in enumerate((1.0 / 16, -1.0 / 32)):
        shared = 8 * (1 + np.arange(64) % 5) * silu(32 * v) * 64 * v / (1 + np.exp(-8 * v))
        assert np.abs(shared).max() > 0.05 * np.abs(want[t]).max()
        # a sigmoid swapped for silu (or no gate at all) moves y far past the tolerance
        assert np.abs(shared * (1 - 1 / (1 + np.exp(-8 * v)))).max() > 1e-3 * np.abs(want[t]).max()


def test_moe_forward_f32_baseline_agrees(oracle):
    """The AVX2 fp32 MoE baseline (timed by bench.py beside the exact flow) computes the
    same layer: within fp32 rounding of the exact double-accumulation flow, any thread
    count."""
    from kadan_amd import synth
    x, logits = synth.moe_inputs(0x51, 7, 128, 8)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(0x51, 8, 128, 192)
    want = oracle.moe_forward(x, logits, 2, gb, gs, ub, us, db, ds)[0]
    for threads in (1, 3):
        got = oracle.moe_forward_f32(x, logits, 2, gb, gs, ub, us, db, ds, threads=threads)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()

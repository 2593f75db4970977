"""Writes tests/golden/reference_vectors.npz: input/output vectors of the reference's own
compiled code (oracle/_ref, built from /root/reference by oracle/Makefile), so that the
oracle stays pinned where the reference is absent (the GPU box, later rounds).

    python tests/golden/make_golden.py      # needs oracle/_ref/libkadan_ref.so

Contents (all little-endian, plain arrays, no pickles):
  decode_<fmt>_blocks / decode_<fmt>_values   ggml to_float of 64 blocks per format
      (Q4_0, Q8_0, Q4_K), random bytes from xorshift32 seeded 0x31415926 as
      IW/tests/gguf_quantization.cpp:93-147 seeds its own; the first 16 blocks carry
      the special fp16 scales of that test (zeros, subnormals, max, inf, NaN).
      Q3_K, Q6_K, IQ4_NL, IQ4_XS the same way from a second generator (seed
      0x27182818, so the arrays above keep their bytes), the scale at the format's
      offset (108 for Q3_K, 208 for Q6_K) as that test places it; BF16 as 256 values
      (512 random bytes, the first 16 values the special patterns); IQ3_XXS, IQ2_S,
      IQ3_S as 256 random blocks each from a third generator (seed 0x14142135) plus
      blocks whose grid indices enumerate the whole grid.
  (for these formats the script also checks kadan::gguf::decode, the reference's own
  device decode, IW/include/kadan/gguf_quantization.hpp:631-762, equal to ggml on every
  block, and stores the values once)
  q8_0_x / q8_0_bytes        ggml x86 quantize_row_q8_0 (G/src/ggml-cpu/arch/x86/quants.c:302-398)
  q8_K_x / q8_K_bytes        ggml quantize_row_q8_K (G/src/ggml-quants.c:2769-2806)
  dot_<fmt>_w / dot_<fmt>_x / dot_<fmt>_out   ggml AVX2 vec_dot against the dot type
  matvec_<fmt>_w / _x / _y   kadan::text::CpuMatvec (IW/src/models/text/cpu_matvec.cpp:28-66)
  mxfp4_blocks / mxfp4_scales / mxfp4_values / mxfp4_x / mxfp4_y
                             kadan quantization::decode_rows / matvec
                             (IW/src/weights/quantization.cpp:193-247)
  route_<E>_<k>_logits / _idx / _w
                             the router of MoeLayer::forward (IW/src/models/text/
                             qwen_layers.cpp:397-425) with the C++ library's
                             std::partial_sort, on logits drawn from a few values
                             (0, 1, 2, -1, -inf, and NaN / +inf in some rows) so that
                             equal probabilities are the rule: the order the library's
                             heap selection gives ties
  route_near_<E>_<k>_logits / _idx / _w
                             the same router on 256 rows whose top-k boundary sits among
                             logits a few ulps apart (tests/util.py near_tie_logits):
                             the order comes from the last bits of the library's expf,
                             the double total and the division
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import (BF16, BLOCK_BYTES, BLOCK_VALUES, IQ2_S, IQ3_S, IQ3_XXS, IQ4_NL,  # noqa: E402
                    IQ4_XS, Q3_K, Q4_0, Q4_K, Q6_K, Q8_0, Reference)

OUT = os.path.join(HERE, "reference_vectors.npz")
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q3_K: "q3_k", Q6_K: "q6_k",
         IQ4_NL: "iq4_nl", IQ4_XS: "iq4_xs", BF16: "bf16", IQ3_XXS: "iq3_xxs",
         IQ2_S: "iq2_s", IQ3_S: "iq3_s"}
SCALE_OFFSET = {Q3_K: 108, Q6_K: 208}
SPECIAL_HALVES = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x83FF, 0x0400, 0x8400, 0x3C00,
                  0xBC00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E01, 0x7C01]


class XorShift32:
    def __init__(self, state=0x31415926):
        self.s = state

    def __call__(self):
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        self.s = s
        return s


def random_blocks(encoding, count, rng):
    size = BLOCK_BYTES[encoding]
    blocks = np.zeros((count, size), np.uint8)
    for t in range(count):
        for i in range(size):
            blocks[t, i] = rng() & 255
        scale = (SPECIAL_HALVES[t] if t < 16
                 else (rng() & 0x83FF) | ((rng() % 31) << 10))
        at = SCALE_OFFSET.get(encoding, 0)
        blocks[t, at], blocks[t, at + 1] = scale & 255, scale >> 8
        if encoding == Q4_K:
            minimum = (SPECIAL_HALVES[15 - t] if t < 16
                       else (rng() & 0x83FF) | ((rng() % 31) << 10))
            blocks[t, 2], blocks[t, 3] = minimum & 255, minimum >> 8
    return blocks


def finite_weights(encoding, n_out, n_in, rng):
    """Packed rows with finite, modest scales (every code byte random)."""
    blocks = random_blocks(encoding, n_out * n_in // BLOCK_VALUES[encoding], rng)
    for b in blocks:
        b[1] = 0x18 + (b[1] & 7)  # fp16 exponent 6..7: scales ~1e-3
        if encoding == Q4_K:
            b[3] = 0x14 + (b[3] & 7)
    return blocks.reshape(n_out, -1)


def grid_blocks(enc, rng):
    """Random blocks whose grid indices enumerate every entry of the format's grid (32
    IQ2_S blocks, 4 IQ3_XXS, 8 IQ3_S), so the fixture pins each table entry."""
    entries = {IQ2_S: 1024, IQ3_XXS: 256, IQ3_S: 512}[enc]
    per_block = {IQ2_S: 32, IQ3_XXS: 64, IQ3_S: 64}[enc]
    blocks = random_blocks(enc, entries // per_block, rng)
    for t, block in enumerate(blocks):
        index = np.arange(t * per_block, (t + 1) * per_block)
        if enc == IQ3_XXS:
            block[2:66] = index
        elif enc == IQ2_S:  # slot 4g + q: low byte, bits 8..9 in byte 66 + g at 2q
            block[2:34] = index & 255
            high = (index >> 8).reshape(8, 4)
            block[66:74] = (high << (2 * np.arange(4))).sum(axis=1)
        else:  # IQ3_S slot 8g + 2q + h: low byte, bit 8 in byte 66 + g at 2q + h
            block[2:66] = index & 255
            high = (index >> 8).reshape(8, 8)
            block[66:74] = (high << np.arange(8)).sum(axis=1)
    return blocks


def check_kadan_equals_ggml(ref, enc, blocks, ggml_values):
    """kadan::gguf::decode (the reference's device decode) must equal ggml to_float on
    every block, bit for bit (NaN matches NaN), as IW/tests/gguf_quantization.cpp:93-147
    requires; the fixture then stores the ggml values once."""
    for b, want in zip(blocks, ggml_values):
        got = ref.kadan_decode_block(enc, b)
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), NAMES[enc]


def main():
    if not Reference.available():
        raise SystemExit("oracle/_ref/libkadan_ref.so is not built (make -C oracle ref)")
    ref = Reference()
    rng = XorShift32()
    data = {}
    for enc in (Q4_0, Q8_0, Q4_K):
        blocks = random_blocks(enc, 64, rng)
        data[f"decode_{NAMES[enc]}_blocks"] = blocks
        data[f"decode_{NAMES[enc]}_values"] = ref.to_float(enc, blocks.reshape(1, -1),
                                                           64 * BLOCK_VALUES[enc]).reshape(64, -1)
    rng2 = XorShift32(0x27182818)
    for enc in (Q3_K, Q6_K, IQ4_NL, IQ4_XS):
        blocks = random_blocks(enc, 64, rng2)
        data[f"decode_{NAMES[enc]}_blocks"] = blocks
        data[f"decode_{NAMES[enc]}_values"] = ref.to_float(enc, blocks.reshape(1, -1),
                                                           64 * BLOCK_VALUES[enc]).reshape(64, -1)
        check_kadan_equals_ggml(ref, enc, blocks, data[f"decode_{NAMES[enc]}_values"])
    bf = np.array([rng2() & 255 for _ in range(512)], np.uint8)
    bf.view(np.uint16)[:16] = SPECIAL_HALVES  # 0, -0, subnormals, max, inf, NaNs as bf16 bits
    data["decode_bf16_blocks"] = bf.reshape(256, 2)
    data["decode_bf16_values"] = ref.to_float(BF16, bf.reshape(1, -1), 256).reshape(256, 1)
    check_kadan_equals_ggml(ref, BF16, bf.reshape(256, 2), data["decode_bf16_values"])
    rng3 = XorShift32(0x14142135)
    for enc in (IQ3_XXS, IQ2_S, IQ3_S):
        blocks = np.concatenate([random_blocks(enc, 256, rng3), grid_blocks(enc, rng3)])
        data[f"decode_{NAMES[enc]}_blocks"] = blocks
        data[f"decode_{NAMES[enc]}_values"] = ref.to_float(
            enc, blocks.reshape(1, -1), len(blocks) * BLOCK_VALUES[enc]).reshape(len(blocks), -1)
        check_kadan_equals_ggml(ref, enc, blocks, data[f"decode_{NAMES[enc]}_values"])
    # activation quantizers: N(0,1) values plus exact half-way cases after scaling
    g = np.random.default_rng(0x5EED)
    x = g.standard_normal(512).astype(np.float32)
    x[:32] = np.arange(32, dtype=np.float32) - 15.5  # amax 15.5: id = 127/15.5
    x[32:64] = 0.0
    x[64] = 127.0
    x[65:68] = [0.5, 1.5, -2.5]  # id = 1: ties to even
    x[68:96] = 0.25
    data["q8_0_x"] = x
    data["q8_0_bytes"] = ref.quantize_row(Q8_0, x, 512 // 32 * 34)
    xk = g.standard_normal(512).astype(np.float32) * 3
    xk[256:512] = -np.abs(xk[256:512])  # negative signed max
    data["q8_K_x"] = xk
    data["q8_K_bytes"] = ref.quantize_row(15, xk, 2 * (4 + 256 + 32))
    # AVX2 vec_dot against the quantized activations
    for enc, dot_type, xbytes in ((Q8_0, Q8_0, 34), (Q4_0, Q8_0, 34), (Q4_K, 15, 292)):
        n = 512
        w = finite_weights(enc, 4, n, rng)
        xv = g.standard_normal((4, n)).astype(np.float32)
        per_block = 32 if dot_type == Q8_0 else 256
        xq = np.stack([ref.quantize_row(dot_type, xv[r], n // per_block * xbytes)
                       for r in range(4)])
        out = np.array([ref.vec_dot(enc, n, w[r], xq[r]) for r in range(4)], np.float32)
        data[f"dot_{NAMES[enc]}_w"] = w
        data[f"dot_{NAMES[enc]}_x"] = xq
        data[f"dot_{NAMES[enc]}_out"] = out
    # CpuMatvec over 64-column units (the CPU baseline path)
    for enc in (Q8_0, Q4_0, Q4_K):
        n_in, n_out = 512, 96
        w = finite_weights(enc, n_out, n_in, rng)
        xv = g.standard_normal((2, n_in)).astype(np.float32)
        data[f"matvec_{NAMES[enc]}_w"] = w
        data[f"matvec_{NAMES[enc]}_x"] = xv
        data[f"matvec_{NAMES[enc]}_y"] = ref.cpu_matvec(enc, w, xv, n_in, n_out, 2)
    # MXFP4 decode and exact matvec
    rows, cols = 8, 128
    blocks = np.array([rng() & 255 for _ in range(rows * cols // 2)], np.uint8).reshape(rows, -1)
    scales = np.array([110 + rng() % 30 for _ in range(rows * cols // 32)], np.uint8).reshape(rows, -1)
    scales[0, 0], scales[1, 1] = 0, 254  # 2^-127 and 2^127 block scales
    blocks[1, 16:32] = 0x9A  # codes -0.5 and -1.0 stay finite at 2^127
    rc, values = ref.mxfp4_decode_rows(blocks, scales, rows, cols)
    assert rc == 0, rc
    xm = g.standard_normal(cols).astype(np.float32)
    scales_mv = scales.copy()
    scales_mv[1, 1] = 130  # the matvec needs finite products
    rc, ym = ref.mxfp4_matvec(blocks, scales_mv, rows, cols, xm)
    assert rc == 0, rc
    data.update(mxfp4_blocks=blocks, mxfp4_scales=scales, mxfp4_values=values,
                mxfp4_mv_scales=scales_mv, mxfp4_x=xm, mxfp4_y=ym)
    # routing with ties: logits from a small set of values, std::partial_sort's order
    gr = np.random.default_rng(0x7135)
    values = np.array([0, 1, 2, -1, -np.inf, np.nan, np.inf], np.float32)
    finite = np.array([.4, .3, .2, .07, .03, 0, 0])
    special = np.array([.3, .3, .2, .1, .05, .03, .02])
    for experts, top_k in ((4, 4), (6, 3), (13, 8), (16, 4), (32, 4), (128, 4), (256, 8)):
        rows = [gr.choice(values, size=experts, p=special if t % 4 == 3 else finite)
                for t in range(48)]
        logits = np.stack(rows).astype(np.float32)
        logits[0] = 0.0  # every probability equal
        idx, w = ref.moe_route(logits, top_k)
        key = f"route_{experts}_{top_k}"
        data[f"{key}_logits"], data[f"{key}_idx"], data[f"{key}_w"] = logits, idx, w
    # routing near ties: values a few ulps apart at the top-k boundary
    from tests.util import near_tie_logits
    for experts, top_k, seed in ((32, 4, 0x7136), (128, 8, 0x7137)):
        logits = near_tie_logits(seed, 256, experts, top_k)
        idx, w = ref.moe_route(logits, top_k)
        key = f"route_near_{experts}_{top_k}"
        data[f"{key}_logits"], data[f"{key}_idx"], data[f"{key}_w"] = logits, idx, w
    np.savez_compressed(OUT, **data)
    print(OUT, os.path.getsize(OUT), "bytes,", len(data), "arrays")


if __name__ == "__main__":
    main()

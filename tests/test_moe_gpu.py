"""GPU parity of the MXFP4 MoE layer (kdq_moe_route, kdq_mxfp4_dequantize, kdq_moe_mxfp4).

Top-k indices and the permutation must be bit-exact (ties included: the reference's
std::partial_sort order, recorded in tests/golden from the C++ library); routing weights
and the layer output within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the output RMS (the
MoE outputs are far from unit scale at these distributions, so max-abs is normalised)
against the oracle's composition of the reference pieces (double-accumulated MXFP4
products).  The full-size C4 T=256 and C5 layers are compared on sampled tokens: a
token's output depends only on its own routing, so the oracle runs on the sample.
"""
import os

import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_vectors.npz")
ROUTE_CASES = [(4, 4), (6, 3), (13, 8), (16, 4), (32, 4), (128, 4), (256, 8)]


@pytest.mark.parametrize("tokens,experts,top_k", [(1, 32, 4), (7, 8, 2), (256, 32, 4),
                                                  (2048, 128, 4), (300, 256, 8), (5, 4, 4),
                                                  (3000, 128, 4), (700, 256, 8)])
def test_route_and_permutation_bit_exact(device, oracle, tokens, experts, top_k):
    torch = _torch()
    _, logits = synth.moe_inputs(0xC4 + tokens, tokens, 64, experts,
                                 hot=8 if experts >= 128 else 0)
    idx, w = oracle.moe_route(logits, top_k)
    offsets, perm = oracle.moe_permute(idx, experts)
    from kadan_amd import ops
    gi, gw, go, gp = ops.moe_route(torch.from_numpy(logits).to(device), top_k)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert np.array_equal(go.cpu().numpy(), offsets)
    assert np.array_equal(gp.cpu().numpy(), perm)
    assert_close(gw.cpu().numpy(), w, rel=1e-6, mabs=1e-5, what="routing weights")


@pytest.mark.parametrize("experts,top_k", ROUTE_CASES)
def test_route_ties_in_library_order(device, experts, top_k):
    """Logits drawn from a few values (and NaN / +-inf in some rows), so equal
    probabilities are the rule: indices bit-exact to std::partial_sort's output recorded
    from the compiled C++ library, weights bit-exact too (NaN matches NaN)."""
    torch = _torch()
    with np.load(GOLDEN, allow_pickle=False) as f:
        key = f"route_{experts}_{top_k}"
        logits, idx, w = f[f"{key}_logits"], f[f"{key}_idx"], f[f"{key}_w"]
    from kadan_amd import ops
    gi, gw, _, _ = ops.moe_route(torch.from_numpy(logits).to(device), top_k)
    assert np.array_equal(gi.cpu().numpy(), idx)
    gw = gw.cpu().numpy()
    assert np.all((gw.view(np.uint32) == w.view(np.uint32)) | (np.isnan(gw) & np.isnan(w)))


@pytest.mark.parametrize("experts,top_k", [(32, 4), (128, 8)])
def test_route_near_ties_golden(device, experts, top_k):
    """Logits a few ulps apart at the top-k boundary, recorded through the compiled
    reference's router: indices and weights bit-exact."""
    torch = _torch()
    with np.load(GOLDEN, allow_pickle=False) as f:
        key = f"route_near_{experts}_{top_k}"
        logits, idx, w = f[f"{key}_logits"], f[f"{key}_idx"], f[f"{key}_w"]
    from kadan_amd import ops
    gi, gw, _, _ = ops.moe_route(torch.from_numpy(logits).to(device), top_k)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert np.array_equal(gw.cpu().numpy().view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("experts,top_k,seed", [(32, 4, 0x713B), (128, 8, 0x713C),
                                                (256, 8, 0x713D)])
def test_route_near_ties_bit_exact(device, oracle, experts, top_k, seed):
    """100000 near-tie rows (tests/util.py near_tie_logits; a third of them with
    probabilities below 2^-22, where the double total's order matters): the device's
    indices and weights bit for bit equal to the oracle's router (the host C library's
    expf, the total summed in expert order), which tests/test_oracle.py pins to the
    compiled reference on the same kind of rows."""
    torch = _torch()
    from kadan_amd import ops
    from tests.util import near_tie_logits
    logits = near_tie_logits(seed, 100000, experts, top_k)
    idx, w = oracle.moe_route(logits, top_k)
    gi, gw, _, _ = ops.moe_route(torch.from_numpy(logits).to(device), top_k)
    gi, gw = gi.cpu().numpy(), gw.cpu().numpy()
    bad = np.flatnonzero((gi != idx).any(1) | (gw.view(np.uint32) != w.view(np.uint32)).any(1))
    assert bad.size == 0, (bad.size, bad[:5])


@pytest.mark.parametrize("experts,top_k,seed", [(32, 4, 0x714B), (128, 8, 0x714C),
                                                (256, 8, 0x714D), (100, 6, 0x714E)])
def test_route_few_tokens_near_ties_bit_exact(device, oracle, experts, top_k, seed):
    """Calls of at most 64 tokens route one token per workgroup (route_wg_kernel: the
    probabilities ranked by counting, the in-order total by one thread): 8192 near-tie
    rows in calls of 64, 17 and 1 tokens, bit for bit equal to the oracle's router."""
    torch = _torch()
    from kadan_amd import ops
    from tests.util import near_tie_logits
    logits = near_tie_logits(seed, 8192, experts, top_k)
    idx, w = oracle.moe_route(logits, top_k)
    cuts = list(range(0, 8192 - 18, 64)) + [8192 - 18, 8192 - 1, 8192]
    dev = torch.from_numpy(logits).to(device)
    gi = np.zeros_like(idx)
    gw = np.zeros_like(w)
    for a, b in zip(cuts[:-1], cuts[1:]):
        ci, cw, _, _ = ops.moe_route(dev[a:b].contiguous(), top_k)
        gi[a:b], gw[a:b] = ci.cpu().numpy(), cw.cpu().numpy()
    bad = np.flatnonzero((gi != idx).any(1) | (gw.view(np.uint32) != w.view(np.uint32)).any(1))
    assert bad.size == 0, (bad.size, bad[:5])


def test_route_equal_logits_heap_order(device):
    """16 equal probabilities, top-4: std::partial_sort gives [1, 3, 0, 2] (worked through
    the heap steps in tests/test_oracle.py)."""
    torch = _torch()
    logits = np.zeros((2, 16), np.float32)
    logits[1, :13] = [1, 0, 0, 0, -5, 1, 0, 0, -5, 1, 0, 0, 1]
    logits[1, 13:] = -5
    from kadan_amd import ops
    gi, gw, _, _ = ops.moe_route(torch.from_numpy(logits).to(device), 4)
    assert gi.cpu().numpy()[0].tolist() == [1, 3, 0, 2]
    np.testing.assert_allclose(gw.cpu().numpy()[0], 0.25, rtol=1e-6)


def test_route_equal_probabilities_from_different_logits(device, oracle):
    """Logits 0 and 1e-8 both give p = 1 after the float exp: they tie, and the device
    follows the oracle's (the library's) heap order."""
    torch = _torch()
    logits = np.full((3, 16), -5.0, np.float32)
    logits[0, :2] = [0.0, 1e-8]
    logits[1, [4, 7]] = [1e-8, 0.0]
    logits[2, [2, 9, 11]] = [1e-8, 0.0, 1e-8]
    idx, w = oracle.moe_route(logits, 3)
    from kadan_amd import ops
    gi, gw, _, _ = ops.moe_route(torch.from_numpy(logits).to(device), 3)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert_close(gw.cpu().numpy(), w, rel=1e-6, mabs=1e-6, what="routing weights")


def test_mxfp4_dequantize_bit_exact(device, oracle):
    torch = _torch()
    rows, cols = 64, 256
    blocks = synth.random_bytes(5, 1, rows * cols // 2).reshape(rows, cols // 2)
    scales = (synth.random_bytes(5, 2, rows * cols // 32) % 200 + 20).astype(np.uint8)
    scales = scales.reshape(rows, cols // 32)
    scales[0, 0], scales[1, 0], scales[2, 0] = 0, 254, 1  # extremes that stay finite
    blocks[1, :16] = 0x11  # 0.5 * 2^127 values
    rc, expected = oracle.mxfp4_decode_rows(blocks, scales, rows, cols)
    assert rc == 0
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.mxfp4_dequantize(torch.from_numpy(blocks).to(device),
                               torch.from_numpy(scales).to(device), rows, cols, status=status)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), expected.view(np.uint32))
    assert int(status.item()) == 0
    bad = scales.copy()
    bad[3, 1] = 255
    status.zero_()
    ops.mxfp4_dequantize(torch.from_numpy(blocks).to(device), torch.from_numpy(bad).to(device),
                         rows, cols, status=status)
    assert int(status.item()) & 1


def run_layer(device, oracle, tokens, hidden, inter, experts, top_k, seed, hot=0, threads=8):
    torch = _torch()
    x, logits = synth.moe_inputs(seed, tokens, hidden, experts, hot=hot)
    weights = synth.moe_weights_torch(seed, experts, hidden, inter, device)
    (gb, gs), (ub, us), (db, ds) = [(b.cpu().numpy(), s.cpu().numpy()) for b, s in weights]
    y, idx, w, offsets, perm = oracle.moe_forward(x, logits, top_k, gb, gs, ub, us, db, ds,
                                                  threads=threads)
    from kadan_amd import ops
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    gy, gi, gw, go, gp = ops.moe_mxfp4(dev(x).view(torch.bfloat16), dev(logits), top_k,
                                       dev(gb), dev(gs), dev(ub), dev(us), dev(db), dev(ds),
                                       routing=True)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert np.array_equal(gp.cpu().numpy(), perm)
    assert np.array_equal(go.cpu().numpy(), offsets)
    assert_close(gy.cpu().numpy(), y, what=f"moe T={tokens} H={hidden} I={inter} E={experts}")


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k", [
    (1, 64, 64, 4, 2), (3, 128, 192, 8, 2), (37, 256, 128, 8, 4), (130, 128, 128, 4, 4),
    (16, 2880, 2880, 32, 4),
    # more than 4096 slots (the chunked permutation): heavy items first, and experts of
    # several work items each
    (1100, 64, 64, 256, 4), (1300, 64, 64, 16, 4),
])
def test_moe_layer_parity(device, oracle, tokens, hidden, inter, experts, top_k):
    run_layer(device, oracle, tokens, hidden, inter, experts, top_k, seed=0xC4 + tokens)


def test_moe_layer_decode_shape(device, oracle):
    """C4 decode: gpt-oss-20b-like layer at 1 token."""
    run_layer(device, oracle, 1, 2880, 2880, 32, 4, seed=0xC4)


@pytest.mark.parametrize("hidden,inter,experts,top_k", [
    (192, 320, 8, 3),     # partial quads in both products
    (4480, 448, 16, 8),   # gate/up runs of 3 quads taken in batches of 2
    (256, 1856, 8, 3),    # down runs of 2 quads, 4 runs per slot
    (128, 3520, 16, 8),   # down runs of 7 quads in batches of 3, the last step partial
    (1024, 1024, 256, 1), # the most experts, one slot
])
def test_moe_single_token_path(device, oracle, hidden, inter, experts, top_k):
    """One token runs the two-launch decode (routing in every gate/up workgroup, gate/up
    and down split into runs of whole quads over the K dimension)."""
    run_layer(device, oracle, 1, hidden, inter, experts, top_k, seed=0x1D + hidden + top_k)


def test_moe_layer_skewed_routing(device, oracle):
    """C5-like skew (25% of tokens favour 8 hot experts) at a size the oracle finishes."""
    run_layer(device, oracle, 64, 256, 256, 128, 4, seed=0xC5, hot=8)


def test_moe_known_answer(device):
    """The hand-derived 2-token x 4-expert case (tests/util.py known_answer_moe) on the
    device: routing exact, output within the tolerance of the closed form."""
    torch = _torch()
    from tests.util import known_answer_moe
    x, logits, ((gb, gs), (ub, us), (db, ds)), y, idx = known_answer_moe()
    from kadan_amd import ops
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    gy, gi, _, _, _ = ops.moe_mxfp4(dev(x).view(torch.bfloat16), dev(logits), 2, dev(gb),
                                    dev(gs), dev(ub), dev(us), dev(db), dev(ds), routing=True)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert_close(gy.cpu().numpy(), y, what="moe known answer")


def sampled_tokens(offsets, perm, top_k, tokens, hot=8, extra=16, seed=5):
    """Tokens to check at full size: for the `hot` experts with the most rows, the token of
    their first slot and of their last (the last work item of a multi-item expert), plus
    `extra` seeded random tokens."""
    counts = np.diff(offsets)
    chosen = set()
    for e in np.argsort(-counts, kind="stable")[:hot]:
        if counts[e]:
            chosen.add(int(perm[offsets[e]]) // top_k)
            chosen.add(int(perm[offsets[e + 1] - 1]) // top_k)
    rng = np.random.default_rng(seed)
    chosen |= set(int(t) for t in rng.choice(tokens, min(extra, tokens), replace=False))
    return np.array(sorted(chosen))


def run_full_size(device, oracle, tokens, experts, hot, seed, what):
    """The packed (resident-bank) entry point at a benchmark configuration: the whole
    batch's routing bit-exact, sampled tokens' outputs against the oracle."""
    torch = _torch()
    hidden = inter = 2880
    top_k = 4
    x, logits = synth.moe_inputs(seed, tokens, hidden, experts, hot=hot)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights_torch(seed, experts, hidden, inter,
                                                           device)
    from kadan_amd import ops
    packed = [ops.moe_mxfp4_pack(gb, gs, experts, inter, hidden),
              ops.moe_mxfp4_pack(ub, us, experts, inter, hidden),
              ops.moe_mxfp4_pack(db, ds, experts, hidden, inter)]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    gy, gi, gw, go, gp = ops.moe_mxfp4_packed(dev(x).view(torch.bfloat16), dev(logits), top_k,
                                              inter, *packed, routing=True)
    idx, w = oracle.moe_route(logits, top_k)
    offsets, perm = oracle.moe_permute(idx, experts)
    assert np.array_equal(gi.cpu().numpy(), idx)
    assert np.array_equal(go.cpu().numpy(), offsets)
    assert np.array_equal(gp.cpu().numpy(), perm)
    assert_close(gw.cpu().numpy(), w, rel=1e-6, mabs=1e-5, what=f"{what} routing weights")
    sample = sampled_tokens(offsets, perm, top_k, tokens)
    host = [a.cpu().numpy() for a in (gb, gs, ub, us, db, ds)]
    del packed
    y, _, _, _, _ = oracle.moe_forward(x[sample], logits[sample], top_k, *host,
                                       threads=min(16, os.cpu_count() or 1))
    assert_close(gy.cpu().numpy()[sample], y, what=f"{what} ({len(sample)} sampled tokens)")
    return np.diff(offsets)


def test_moe_c5_full_size_sampled(device, oracle):
    """C5 at its own size: 128 experts, H = I = 2880, T = 2048, 25 % of tokens favouring
    8 hot experts (about 300 rows each, five work items)."""
    counts = run_full_size(device, oracle, 2048, 128, 8, 0xC5, "moe C5 T=2048")
    assert counts.max() > 4 * 64  # the hot experts do span several work items


def test_moe_c4_prefill_full_size_sampled(device, oracle):
    """C4 prefill at its own size: 32 experts, H = I = 2880, T = 256."""
    run_full_size(device, oracle, 256, 32, 0, 0xC4, "moe C4 T=256")


def test_moe_prefill_256_properties(device):
    """C4 prefill (256 tokens) at full size: determinism across calls, and permutation
    invariance (reversing the token order reverses the output rows)."""
    torch = _torch()
    x, logits = synth.moe_inputs(0xC4, 256, 2880, 32)
    from kadan_amd import ops
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    wts = [a for pair in synth.moe_weights_torch(0xC4, 32, 2880, 2880, device) for a in pair]
    xb = dev(x).view(torch.bfloat16)
    y1 = ops.moe_mxfp4(xb, dev(logits), 4, *wts).cpu().numpy()
    y2 = ops.moe_mxfp4(xb, dev(logits), 4, *wts).cpu().numpy()
    assert np.array_equal(y1, y2)
    yr = ops.moe_mxfp4(dev(x[::-1]).view(torch.bfloat16), dev(logits[::-1]), 4, *wts)
    assert_close(yr.cpu().numpy()[::-1], y1, rel=1e-6, mabs=1e-5, what="token order")


def unpack_reference(packed, experts, rows, cols):
    """The GPT-OSS layout back from the packed one (the layout as include/kadan_amd.h states
    it): codes [E][R/32][C/64][lane i + 32h][16 B], scales [E][R/32][ceil(C/256)][lane][4 B]."""
    groups, steps = rows // 32, cols // 64
    sgroups = (steps + 3) // 4
    code_bytes = experts * rows * cols // 2
    codes = packed[:code_bytes].reshape(experts, groups, steps, 2, 32, 16)
    blocks = codes.transpose(0, 1, 4, 2, 3, 5).reshape(experts, rows, cols // 2)
    sc = packed[code_bytes:].reshape(experts, groups, sgroups, 2, 32, 4)
    sc = sc.transpose(0, 1, 4, 2, 5, 3).reshape(experts, rows, sgroups * 4 * 2)
    return blocks, sc[:, :, :cols // 32], sc[:, :, cols // 32:]


@pytest.mark.parametrize("experts,rows,cols", [(3, 64, 2880), (2, 96, 192), (1, 32, 256)])
def test_moe_pack_layout(device, experts, rows, cols):
    """kdq_moe_mxfp4_pack moves every code and scale byte to its stated place and zero-fills
    the scale slots past the last step."""
    torch = _torch()
    blocks = synth.random_bytes(7, 1, experts * rows * cols // 2).reshape(experts, rows, -1)
    scales = synth.random_bytes(7, 2, experts * rows * cols // 32).reshape(experts, rows, -1)
    from kadan_amd import ops
    packed = ops.moe_mxfp4_pack(torch.from_numpy(blocks).to(device),
                                torch.from_numpy(scales).to(device), experts, rows, cols)
    packed = packed.cpu().numpy()
    import kadan_amd
    assert packed.size == kadan_amd.lib().kdq_moe_mxfp4_packed_bytes(experts, rows, cols)
    b, s, pad = unpack_reference(packed, experts, rows, cols)
    assert np.array_equal(b, blocks)
    assert np.array_equal(s, scales)
    assert not pad.any()


@pytest.mark.parametrize("tokens,hidden,inter,experts,top_k", [
    (1, 2880, 2880, 32, 4), (256, 2880, 2880, 32, 4), (37, 256, 192, 8, 4), (1, 64, 64, 4, 2),
])
def test_moe_packed_matches_reference_layout(device, tokens, hidden, inter, experts, top_k):
    """The packed entry point over resident packed weights gives the reference-layout
    entry point's output and routing bit for bit."""
    torch = _torch()
    x, logits = synth.moe_inputs(0xAB + tokens, tokens, hidden, experts)
    from kadan_amd import ops
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    wts = [a for pair in synth.moe_weights_torch(0xAB, experts, hidden, inter, device)
           for a in pair]
    xb, lg = dev(x).view(torch.bfloat16), dev(logits)
    ref = ops.moe_mxfp4(xb, lg, top_k, *wts, routing=True)
    packed = [ops.moe_mxfp4_pack(wts[0], wts[1], experts, inter, hidden),
              ops.moe_mxfp4_pack(wts[2], wts[3], experts, inter, hidden),
              ops.moe_mxfp4_pack(wts[4], wts[5], experts, hidden, inter)]
    got = ops.moe_mxfp4_packed(xb, lg, top_k, inter, *packed, routing=True)
    for a, b in zip(got, ref):
        assert np.array_equal(a.cpu().numpy().view(np.uint8), b.cpu().numpy().view(np.uint8))


@pytest.mark.parametrize("tokens", [1, 3, 40])  # single-token, one-workgroup prologue, large
@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_moe_nonfinite_activation(device, tokens, bad):
    """A non-finite activation poisons its own token's outputs and nothing else: the FP8
    terms of its 32-value block carry NaN codes and the NaN block scale, so every product
    that touches it is NaN (as an fp32 product would be); the other tokens' outputs are
    bit-identical to a run without it."""
    torch = _torch()
    from kadan_amd import ops
    hidden = inter = 256
    experts, top_k = 8, 4
    x, logits = synth.moe_inputs(0xBAD, tokens, hidden, experts)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(0xBAD, experts, hidden, inter)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    wts = [dev(a) for a in (gb, gs, ub, us, db, ds)]
    clean = ops.moe_mxfp4(dev(x).view(torch.bfloat16), dev(logits), top_k, *wts).cpu().numpy()
    poisoned = x.copy()
    bits = np.array([bad], np.float32).view(np.uint32)[0] >> 16
    bad_row = min(1, tokens - 1)
    poisoned[bad_row, 37] = np.uint16(bits)
    got = ops.moe_mxfp4(dev(poisoned).view(torch.bfloat16), dev(logits), top_k,
                        *wts).cpu().numpy()
    assert not np.isfinite(got[bad_row]).any()
    others = [t for t in range(tokens) if t != bad_row]
    assert np.array_equal(got[others], clean[others])


def test_moe_alignment_rejected(device):
    torch = _torch()
    import kadan_amd
    from kadan_amd import ops
    tokens, hidden, inter, experts = 2, 64, 64, 4
    x, logits = synth.moe_inputs(1, tokens, hidden, experts)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(1, experts, hidden, inter)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    wts = [dev(a) for a in (gb, gs, ub, us, db, ds)]
    xs = torch.zeros(tokens * hidden + 8, dtype=torch.bfloat16, device=device)
    shifted = xs[1:1 + tokens * hidden].view(tokens, hidden)  # 2-byte offset
    with pytest.raises(kadan_amd.KdqError, match="align"):
        ops.moe_mxfp4(shifted, dev(logits), 2, *wts)
    packed = [ops.moe_mxfp4_pack(wts[0], wts[1], experts, inter, hidden),
              ops.moe_mxfp4_pack(wts[2], wts[3], experts, inter, hidden),
              ops.moe_mxfp4_pack(wts[4], wts[5], experts, hidden, inter)]
    with pytest.raises(kadan_amd.KdqError, match="align"):
        ops.moe_mxfp4_packed(dev(x).view(torch.bfloat16), dev(logits), 2, inter,
                             packed[0][16:], packed[1], packed[2])
    with pytest.raises(kadan_amd.KdqError, match="shape"):
        kadan_amd.call("kdq_moe_mxfp4_pack", wts[0].data_ptr(), wts[1].data_ptr(), experts,
                       48, hidden, packed[0].data_ptr(), None)

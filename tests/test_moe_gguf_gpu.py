"""GPU parity of the GGUF MoE layer (kdq_moe_gguf) against the oracle's restatement of
MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:378-492): the routing (selected
experts bit-exact, weights to 1e-6) and y within rel-L2 <= 1e-3, max-abs <= 2e-2 of its
RMS.  Expert projections of the block encodings (Q4_0 / Q8_0 / Q4_K / Q3_K / Q6_K /
IQ4_XS / IQ4_NL and the lattice encodings IQ3_XXS / IQ3_S / IQ2_S) run on the MFMA
kernel with the expert slice chosen on the device, BF16 on the exact kernel.  The
encoding mixes cover each launch form: gate and up stored alike run as one paired launch
that applies the swiglu (MIXED: experts and shared expert; EXACT and LATTICE: IQ3_S /
IQ2_S experts and the shared expert), gate and up stored differently as two launches and
the swiglu kernel (SPLIT), and the exact kernel's slot-affine launch (EXACT: BF16
down experts)."""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

F32, Q4_0, Q8_0, Q3_K, Q4_K, Q6_K, IQ4_XS = 0, 2, 8, 11, 12, 14, 23
IQ3_XXS, IQ3_S, IQ2_S, BF16 = 18, 21, 22, 30
NAMES = ("router", "gate_exps", "up_exps", "down_exps", "gate_shexp", "up_shexp", "down_shexp")


def make_layer(seed, H, E, K, F, S, encs):
    """Host spec: F32 router with logits of a few units (well separated top-k), the rest
    synthetic GGUF tensors of the given encodings, and the shared gate vector."""
    g = np.random.default_rng(seed)
    shapes = {"router": (E, H), "gate_exps": (E, F, H), "up_exps": (E, F, H),
              "down_exps": (E, H, F), "gate_shexp": (S, H), "up_shexp": (S, H),
              "down_shexp": (H, S)}
    spec = dict(hidden=H, experts=E, top_k=K, ff=F, shared_ff=S,
                shared_gate=(g.standard_normal(H) * 0.05).astype(np.float32))
    router = (g.standard_normal((E, H)) * 0.1).astype(np.float32)
    spec["router"] = (F32, router.view(np.uint8).reshape(E, -1))
    for i, name in enumerate(NAMES[1:]):
        shape = shapes[name]
        rows = int(np.prod(shape[:-1]))
        packed = synth.gguf_weights(encs[name], seed * 16 + i, rows, shape[-1])
        spec[name] = (encs[name], packed.reshape(*shape[:-1], -1))
    return spec


def to_device(torch, device, spec):
    dev = dict(spec)
    for name in NAMES:
        enc, arr = spec[name]
        dev[name] = (enc, torch.from_numpy(np.ascontiguousarray(arr)).to(device))
    dev["shared_gate"] = torch.from_numpy(spec["shared_gate"]).to(device)
    return dev


MIXED = {"gate_exps": Q4_K, "up_exps": Q4_K, "down_exps": Q6_K, "gate_shexp": Q8_0,
         "up_shexp": Q8_0, "down_shexp": Q4_K}
EXACT = {"gate_exps": IQ3_S, "up_exps": IQ3_S, "down_exps": BF16, "gate_shexp": Q4_0,
         "up_shexp": Q4_0, "down_shexp": Q6_K}
LATTICE = {"gate_exps": IQ2_S, "up_exps": IQ2_S, "down_exps": IQ3_XXS, "gate_shexp": IQ3_S,
           "up_shexp": IQ3_S, "down_shexp": IQ3_XXS}
SPLIT = {"gate_exps": Q4_K, "up_exps": Q8_0, "down_exps": Q4_0, "gate_shexp": Q8_0,
         "up_shexp": Q4_K, "down_shexp": Q8_0}


@pytest.mark.parametrize("rows", [1, 3, 8])
@pytest.mark.parametrize("encs", [MIXED, EXACT, SPLIT, LATTICE],
                         ids=["mixed", "exact", "split", "lattice"])
def test_moe_gguf_parity(device, oracle, rows, encs):
    import torch
    H, E, K, F, S = 512, 16, 4, 256, 512
    spec = make_layer(7 + rows, H, E, K, F, S, encs)
    x = synth.normal(11 + rows, 1, rows * H).reshape(rows, H)
    want, idx, w = oracle.moe_gguf_forward(spec, x)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, ws = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device),
                              status=status)
    assert np.array_equal(sel.cpu().numpy(), idx)
    assert np.abs(ws.cpu().numpy() - w).max() < 1e-6
    assert_close(y.cpu().numpy(), want, what=f"moe_gguf rows={rows}")
    assert int(status.item()) == 0


@pytest.mark.parametrize("rows,top_k", [(9, 4), (16, 4), (64, 8), (200, 8)])
@pytest.mark.parametrize("encs", [MIXED, EXACT, SPLIT], ids=["mixed", "exact", "split"])
def test_moe_gguf_more_rows(device, oracle, rows, top_k, encs):
    """Past 8 rows the slots are grouped by expert into padded segments: 9 and 16 rows (two
    passes of the router / shared batch), 64 rows x top-8 = 512 slots, and 200 rows x
    top-8 (100 slots per expert).  MIXED runs gate, up and down on the grouped prefill
    GEMM (64-row token tiles of one expert each) once the experts average 4 rows (from 16
    rows here; 9 rows run 8-row items); SPLIT runs gate / up on the GEMM and
    its Q4_0 down on 8-row GEMV items over the same tiles; EXACT runs its IQ3_S gate / up
    on 8-row MFMA items and its BF16 down on the exact kernel's 8-row items."""
    import torch
    H, E, F, S = 512, 16, 256, 512
    spec = make_layer(40 + rows, H, E, top_k, F, S, encs)
    x = synth.normal(50 + rows, 1, rows * H).reshape(rows, H)
    want, idx, w = oracle.moe_gguf_forward(spec, x)
    from kadan_amd import ops
    y, sel, ws = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device))
    assert np.array_equal(sel.cpu().numpy(), idx)
    assert np.abs(ws.cpu().numpy() - w).max() < 1e-6
    assert_close(y.cpu().numpy(), want, what=f"moe_gguf rows={rows} top_k={top_k}")


def test_moe_gguf_qwen3_shape(device, oracle):
    """Qwen3-30B-A3B's expert geometry (hidden 2048, 128 experts, top-8, expert ff 768)
    with a 768-wide shared expert, one decode token and a batch of four."""
    import torch
    H, E, K, F, S = 2048, 128, 8, 768, 768
    spec = make_layer(3, H, E, K, F, S, MIXED)
    from kadan_amd import ops
    dev = to_device(torch, device, spec)
    for rows in (1, 4):
        x = synth.normal(30 + rows, 1, rows * H).reshape(rows, H)
        want, idx, w = oracle.moe_gguf_forward(spec, x)
        y, sel, ws = ops.moe_gguf(dev, torch.from_numpy(x).to(device))
        assert np.array_equal(sel.cpu().numpy(), idx)
        assert_close(y.cpu().numpy(), want, what=f"qwen3 shape rows={rows}")


@pytest.mark.parametrize("encs", [MIXED, SPLIT], ids=["mixed", "split"])
def test_moe_gguf_prefill_chunk(device, oracle, encs):
    """A 512-token prefill chunk at Qwen3-30B-A3B's geometry (4096 slots over 128
    experts).  Each token's output depends only on its own row and routing, so the
    oracle runs on a sample of tokens (the first, the last, and a seeded spread)."""
    import torch
    H, E, K, F, S, rows = 2048, 128, 8, 768, 768, 512
    spec = make_layer(9, H, E, K, F, S, encs)
    from kadan_amd import ops
    x = synth.normal(91, 1, rows * H).reshape(rows, H)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, ws = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device),
                              status=status)
    y, sel, ws = y.cpu().numpy(), sel.cpu().numpy(), ws.cpu().numpy()
    assert int(status.item()) == 0 and np.isfinite(y).all()
    pick = np.union1d(np.random.default_rng(92).choice(rows, 22, replace=False), [0, rows - 1])
    want, idx, w = oracle.moe_gguf_forward(spec, x[pick])
    assert np.array_equal(sel[pick], idx)
    assert np.abs(ws[pick] - w).max() < 1e-6
    assert_close(y[pick], want, what=f"moe_gguf prefill chunk {len(pick)} sampled tokens")
    # deterministic: the same call again gives the same bits
    y2, _, _ = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device))
    assert np.array_equal(y, y2.cpu().numpy())


def test_moe_gguf_grouped_fp16_range_fallback(device, oracle):
    """An expert gate scale whose dequantised weights could pass the fp16 range (d = 1000)
    makes the grouped GEMM flag the call, which then redoes its expert products on the
    8-row GEMV items (exact decode): y is still the exact product and status stays 0."""
    import torch
    H, E, K, F, S, rows = 512, 16, 4, 256, 512, 32
    spec = make_layer(12, H, E, K, F, S, MIXED)
    enc, arr = spec["gate_exps"]
    arr = arr.copy()
    big = np.array([1000.0], np.float16).view(np.uint16)[0]
    arr[:, :, 0], arr[:, :, 1] = big & 255, big >> 8  # d of every expert's first block
    spec["gate_exps"] = (enc, arr)
    x = synth.normal(13, 1, rows * H).reshape(rows, H)
    want, idx, w = oracle.moe_gguf_forward(spec, x)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, _ = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device),
                             status=status)
    assert np.array_equal(sel.cpu().numpy(), idx)
    assert int(status.item()) == 0
    assert_close(y.cpu().numpy(), want, what="moe_gguf grouped fp16-range fallback")


def test_moe_gguf_nonfinite_weight_status(device):
    import torch
    H, E, K, F, S = 256, 8, 2, 256, 256
    spec = make_layer(5, H, E, K, F, S, MIXED)
    enc, arr = spec["down_shexp"]
    arr = arr.copy()
    arr[3, 0], arr[3, 1] = 0x00, 0x7C  # +inf d in the shared down projection (Q4_K)
    spec["down_shexp"] = (enc, arr)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.moe_gguf(to_device(torch, device, spec), torch.ones(1, H, device=device), status=status)
    assert int(status.item()) == 1


@pytest.mark.parametrize("copies", [1, 32])
def test_moe_gguf_known_answer(device, copies):
    """The closed-form layer with a shared expert (tests/util.py known_answer_moe_gguf):
    2 tokens (the per-slot decode path) and the same 2 tokens 32 times over (64 rows: the
    grouped prefill GEMM for the Q8_0 experts)."""
    import torch
    from kadan_amd import ops
    from tests.util import known_answer_moe_gguf
    spec, x, want, idx = known_answer_moe_gguf()
    x = np.tile(x, (copies, 1))
    want = np.tile(want, (copies, 1))
    y, sel, _ = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device))
    assert np.array_equal(sel.cpu().numpy(), np.tile(idx, (copies, 1)))
    assert_close(y.cpu().numpy(), want, what=f"moe_gguf known answer rows={2 * copies}")


@pytest.mark.parametrize("rows", [1, 64])
def test_moe_gguf_nonfinite_shared_gate_status(device, rows):
    """ffn_gate_inp_shexp is a weight like any other: a NaN in it sets status bit 1 (the
    combine kernel takes its dot product; decode and grouped paths alike)."""
    import torch
    from kadan_amd import ops
    H, E, K, F, S = 256, 8, 2, 256, 256
    spec = make_layer(6, H, E, K, F, S, MIXED)
    spec["shared_gate"] = spec["shared_gate"].copy()
    spec["shared_gate"][200] = np.nan
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.moe_gguf(to_device(torch, device, spec), torch.ones(rows, H, device=device),
                 status=status)
    assert int(status.item()) == 1
    spec["shared_gate"][200] = 0.5  # finite again: nothing flagged
    status.zero_()
    ops.moe_gguf(to_device(torch, device, spec), torch.ones(rows, H, device=device),
                 status=status)
    assert int(status.item()) == 0


def test_moe_gguf_rejections(device):
    import torch
    from kadan_amd import KdqError, ops
    H, E, K, F, S = 256, 8, 2, 256, 256
    dev = to_device(torch, device, make_layer(6, H, E, K, F, S, MIXED))
    with pytest.raises(KdqError, match="kdq_projection_shape"):
        ops.moe_gguf(dict(dev, top_k=9), torch.ones(1, H, device=device))
    with pytest.raises(KdqError, match="kdq_projection_shape"):  # rows > 4096
        ops.moe_gguf(dev, torch.ones(4097, H, device=device))
    with pytest.raises(KdqError, match="kdq_projection_shape"):  # rows * top_k > 8192
        ops.moe_gguf(dict(dev, top_k=8), torch.ones(1025, H, device=device))


@pytest.mark.parametrize("rows", [4, 16, 256])
def test_moe_gguf_packed_stacks_bit_identical(device, oracle, rows):
    """kdq_moe_gguf_packed over resident tile-packed copies (expert stacks and shared
    matrices packed once, as a weight bank keeps them) gives the same bits as
    kdq_moe_gguf, which packs them in the call: 4 rows (the per-slot decode path: the
    expert GEMVs over the packed stacks, bit-identical to the row-major form), 16 (the
    experts on the grouped GEMM, the shared expert on 8-row items) and 256 (the shared
    expert on the dense GEMM too); checked against the oracle too."""
    import torch
    H, E, K, F, S = 512, 16, 8, 256, 512
    spec = make_layer(60 + rows, H, E, K, F, S, MIXED)
    from kadan_amd import ops
    dev = to_device(torch, device, spec)
    packed = ops.moe_gguf_pack(dev)
    assert sorted(k for k in packed if k != "checked") == sorted(NAMES[1:])
    assert packed["checked"]
    x = synth.normal(61 + rows, 1, rows * H).reshape(rows, H)
    xd = torch.from_numpy(x).to(device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, ws = ops.moe_gguf(dev, xd, status=status, packed=packed)
    y0, sel0, ws0 = ops.moe_gguf(dev, xd)
    assert np.array_equal(y.cpu().numpy(), y0.cpu().numpy())
    assert np.array_equal(sel.cpu().numpy(), sel0.cpu().numpy())
    assert np.array_equal(ws.cpu().numpy(), ws0.cpu().numpy())
    assert int(status.item()) == 0
    want, idx, _ = oracle.moe_gguf_forward(spec, x)
    assert np.array_equal(sel.cpu().numpy(), idx)
    assert_close(y.cpu().numpy(), want, what=f"moe_gguf_packed rows={rows}")


def test_moe_gguf_shared_gemm_fp16_range_fallback(device, oracle):
    """A shared gate scale whose dequantised weights could pass the fp16 range (Q8_0
    d = 1000) at 256 rows, where the shared expert runs on the dense GEMM: the call redoes
    the shared expert (and the experts) on the exact-decode rows, so y is still the exact
    product and status stays 0."""
    import torch
    H, E, K, F, S, rows = 512, 16, 4, 256, 512, 256
    spec = make_layer(14, H, E, K, F, S, MIXED)
    enc, arr = spec["gate_shexp"]
    arr = arr.copy()
    big = np.array([1000.0], np.float16).view(np.uint16)[0]
    arr[:, 0], arr[:, 1] = big & 255, big >> 8  # d of every row's first Q8_0 block
    spec["gate_shexp"] = (enc, arr)
    x = synth.normal(15, 1, rows * H).reshape(rows, H)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, _ = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device),
                             status=status)
    assert int(status.item()) == 0
    pick = np.arange(0, rows, 7)
    want, idx, _ = oracle.moe_gguf_forward(spec, x[pick])
    assert np.array_equal(sel.cpu().numpy()[pick], idx)
    assert_close(y.cpu().numpy()[pick], want, what="moe_gguf shared GEMM fp16-range fallback")


def test_moe_gguf_packed_unchecked_still_falls_back(device, oracle):
    """Resident packed copies of a layer whose expert gate has a scale past the fp16 range
    (Q4_K d = 1000): kdq_gguf_gemm_check flags it, so the copies are not marked checked and
    the 200-row call still waits for the GEMM's flag and redoes its products exactly."""
    import torch
    H, E, K, F, S, rows = 512, 16, 8, 256, 512, 200
    spec = make_layer(17, H, E, K, F, S, MIXED)
    enc, arr = spec["gate_exps"]
    arr = arr.copy()
    big = np.array([1000.0], np.float16).view(np.uint16)[0]
    arr[:, :, 0], arr[:, :, 1] = big & 255, big >> 8
    spec["gate_exps"] = (enc, arr)
    from kadan_amd import ops
    dev = to_device(torch, device, spec)
    packed = ops.moe_gguf_pack(dev)
    assert not packed["checked"]
    x = synth.normal(18, 1, rows * H).reshape(rows, H)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    y, sel, _ = ops.moe_gguf(dev, torch.from_numpy(x).to(device), status=status, packed=packed)
    assert int(status.item()) == 0
    pick = np.arange(0, rows, 9)
    want, idx, _ = oracle.moe_gguf_forward(spec, x[pick])
    assert np.array_equal(sel.cpu().numpy()[pick], idx)
    assert_close(y.cpu().numpy()[pick], want, what="moe_gguf_packed unchecked fallback")


def test_moe_gguf_shared_gemm_nonfinite_status(device):
    """A non-finite scale in the shared down (Q4_K) at 256 rows (the shared expert on the
    dense GEMM) reaches the caller's status as bit 1."""
    import torch
    H, E, K, F, S, rows = 256, 8, 2, 256, 256, 256
    spec = make_layer(16, H, E, K, F, S, MIXED)
    enc, arr = spec["down_shexp"]
    arr = arr.copy()
    arr[3, 0], arr[3, 1] = 0x00, 0x7C  # +inf d
    spec["down_shexp"] = (enc, arr)
    from kadan_amd import ops
    status = torch.zeros(1, dtype=torch.int32, device=device)
    ops.moe_gguf(to_device(torch, device, spec), torch.ones(rows, H, device=device),
                 status=status)
    assert int(status.item()) & 1


def test_moe_gguf_paired_gemm_bit_identical(device):
    """Gate and up stored alike run as one paired GEMM whose epilogue applies the SwiGLU
    (the experts' grouped GEMM and, from 256 rows, the shared expert's dense one); the
    same weights with the up rows stored 16 bytes apart (another layout) run as two GEMMs
    and the SwiGLU pass.  Both give the same bits (256 rows, MIXED)."""
    import torch
    H, E, K, F, S, rows = 512, 16, 8, 256, 512, 256
    spec = make_layer(19, H, E, K, F, S, MIXED)
    other = dict(spec)
    for name in ("up_exps", "up_shexp"):
        enc, arr = spec[name]
        padded = np.zeros(arr.shape[:-1] + (arr.shape[-1] + 16,), np.uint8)
        padded[..., :arr.shape[-1]] = arr
        other[name] = (enc, padded)
    from kadan_amd import ops
    x = torch.from_numpy(synth.normal(20, 1, rows * H).reshape(rows, H)).to(device)
    y, sel, _ = ops.moe_gguf(to_device(torch, device, spec), x)
    y2, sel2, _ = ops.moe_gguf(to_device(torch, device, other), x)
    assert np.array_equal(sel.cpu().numpy(), sel2.cpu().numpy())
    assert np.array_equal(y.cpu().numpy(), y2.cpu().numpy())


FUSED_DECODE = [  # (gate/up experts, down experts, shared gate/up, shared down)
    (Q4_K, Q6_K, Q8_0, Q4_K), (Q4_K, Q4_K, Q4_K, Q6_K), (Q4_K, Q6_K, Q4_K, Q4_K),
    (Q4_K, Q4_K, Q8_0, Q6_K)]


@pytest.mark.parametrize("tokens", [1, 3, 8])
@pytest.mark.parametrize("resident", [False, True], ids=["rows", "packed"])
@pytest.mark.parametrize("encs", FUSED_DECODE, ids=lambda e: "-".join(map(str, e)))
@pytest.mark.parametrize("H", [2048, 4096])
def test_moe_gguf_fused_decode(device, oracle, encs, resident, H, tokens):
    """Up to 8 tokens on the fused decode (one launch that computes the router, routes in
    its last router workgroup -- one token by the whole workgroup, several by a wavefront
    each -- and runs every slot's expert gate / up and the shared expert's, then one that
    runs every down and lets the last workgroup of each token's row block combine it):
    each instantiated encoding mix, over row-major and resident packed stacks, hidden 2048
    and 4096 (8 and 16 wavefronts), 1, 3 and 8 tokens (8 tokens of hidden 4096, past the
    64 KB of staged router rows, take the staged path).  Three calls in a row with
    different tokens (the row-block counters reset between calls), each against the
    oracle, routing exact."""
    import torch
    E, K, F, S = 32, 8, 768, 512
    gu, dn, sgu, sdn = encs
    layer_encs = {"gate_exps": gu, "up_exps": gu, "down_exps": dn, "gate_shexp": sgu,
                  "up_shexp": sgu, "down_shexp": sdn}
    spec = make_layer(70 + H // 1024 + dn, H, E, K, F, S, layer_encs)
    from kadan_amd import ops
    dev = to_device(torch, device, spec)
    packed = ops.moe_gguf_pack(dev) if resident else None
    status = torch.zeros(1, dtype=torch.int32, device=device)
    for call in range(3):
        x = synth.normal(71 + call + H + 10 * tokens, 1, tokens * H).reshape(tokens, H)
        want, idx, w = oracle.moe_gguf_forward(spec, x)
        y, sel, ws = ops.moe_gguf(dev, torch.from_numpy(x).to(device), status=status,
                                  packed=packed)
        assert np.array_equal(sel.cpu().numpy(), idx)
        # the device's logits are fp32 sums of H products, the oracle's double: at hidden
        # 4096 the renormalised weights differ by up to ~1e-6 (1.01e-6 seen at 8 tokens)
        assert np.abs(ws.cpu().numpy() - w).max() < (1e-6 if H <= 2048 else 2e-6)
        assert_close(y.cpu().numpy(), want, what=f"fused decode {encs} call {call}")
    assert int(status.item()) == 0


def test_moe_gguf_fused_decode_graph_replays(device):
    """The fused decode captured in a HIP graph and replayed: the call's epoch lives on the
    device (the down launch advances it), so every replay routes its own token rather than
    reading the words an earlier replay published.  Six replays with a new token copied in
    between, eager calls in between too, each replay equal bit for bit to the eager result
    for its token."""
    import torch
    from kadan_amd import ops
    H, E, K, F, S = 2048, 32, 8, 768, 512
    encs = {"gate_exps": Q4_K, "up_exps": Q4_K, "down_exps": Q6_K, "gate_shexp": Q8_0,
            "up_shexp": Q8_0, "down_shexp": Q4_K}
    spec = make_layer(90, H, E, K, F, S, encs)
    dev = to_device(torch, device, spec)
    xs = [torch.from_numpy(synth.normal(91 + i, 1, H).reshape(1, H)).to(device)
          for i in range(5)]
    eager = []
    for x in xs:
        y, sel, w = ops.moe_gguf(dev, x)
        eager.append((y.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()))
    static_x = xs[0].clone()
    ops.moe_gguf(dev, static_x)  # workspace and kernel attributes set up before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y, sel, w = ops.moe_gguf(dev, static_x)
    for n, i in enumerate([1, 3, 0, 4, 2, 2]):
        static_x.copy_(xs[i])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(sel.cpu().numpy(), eager[i][1]), f"replay {n}"
        assert np.array_equal(w.cpu().numpy(), eager[i][2]), f"replay {n}"
        assert np.array_equal(y.cpu().numpy(), eager[i][0]), f"replay {n}"
        j = (i + 1) % 5  # the program's own eager work between replays
        ye, se, _ = ops.moe_gguf(dev, xs[j])
        assert np.array_equal(se.cpu().numpy(), eager[j][1])
        assert np.array_equal(ye.cpu().numpy(), eager[j][0])


@pytest.mark.parametrize("rows,seed", [(256, 2), (512, 3)])
def test_moe_gguf_grouped_matches_fp16_model(device, oracle, rows, seed):
    """The grouped-GEMM layer (experts and the shared expert on the prefill GEMMs) equals
    its numeric design, tests/util.py moe_gguf_fp16_model: x and h rounded to fp16 once
    after a per-row power-of-two scale, each weight as the GEMM's dequantisation forms it
    in fp16, everything else float64.  The device differs from that model only in fp32
    accumulation order (rel-L2 <= 1e-4), while the model itself differs from the exact
    product by the fp16 roundings: at this seed max-abs 2.4e-2 of the RMS at outputs 30x
    the RMS (weights 1.9e-2, x 7.8e-3, h 5.0e-3 of it), i.e. ~8e-4 of those outputs."""
    import torch
    from tests.util import moe_gguf_fp16_model, rel_l2, normalized_max_abs
    H, E, K, F, S = 512, 16, 4, 256, 512
    spec = make_layer(100 + seed * 7 + rows, H, E, K, F, S, MIXED)
    x = synth.normal(200 + seed + rows, 1, rows * H).reshape(rows, H)
    want, idx, w = oracle.moe_gguf_forward(spec, x)
    from kadan_amd import ops
    y, sel, _ = ops.moe_gguf(to_device(torch, device, spec), torch.from_numpy(x).to(device))
    assert np.array_equal(sel.cpu().numpy(), idx)
    model = moe_gguf_fp16_model(oracle, spec, x, idx, w.astype(np.float64))
    y = y.cpu().numpy().astype(np.float64)
    assert rel_l2(y, model) <= 1e-4, rel_l2(y, model)
    assert normalized_max_abs(y, model) <= 1e-2, normalized_max_abs(y, model)
    assert rel_l2(y, want) <= 1e-3

"""GPU parity of the tile-packed resident GGUF layout (kdq_gguf_pack, kdq_gemv_packed,
kdq_gemv_packed_batch).

The layout is checked byte for byte against a numpy restatement of its definition
(include/kadan_amd.h), so a wrong lane, piece or side-data offset fails here before any
product does.  The packed product must equal kdq_gemv on the row-major bytes bit for
bit (the same per-row reduction order), and the oracle's double product of exactly
decoded weights within rel-L2 <= 1e-3 and max-abs <= 2e-2 of the output RMS.
"""
import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close, bits_equal

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
ENCODINGS = [Q8_0, Q4_0, Q4_K, Q6_K]
BLOCK = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}
UNIT = {Q4_K: 2304, Q4_0: 2304, Q8_0: 4352, Q6_K: 3360}
PIECES = {Q4_K: 2, Q4_0: 2, Q8_0: 4, Q6_K: 3}
SCALE_AT = {Q4_K: 0, Q4_0: 0, Q8_0: 0, Q6_K: 208}  # first fp16 block scale


def numpy_pack(encoding, w, n_in):
    """Restates the packed layout: tiles of 16 rows, per (tile, 256-value group) one unit;
    lane l = 16 G + s (chunk G, row slot s) owns the 16-byte code pieces at p*1024 + 16 l,
    then the side data (Q4_K: row slot s's 16-byte header at 2048 + 16 s; Q4_0 / Q8_0: the
    two block scales of chunk G as one dword at pieces*1024 + 4 l).  Q6_K: chunk G = 2h + p
    takes ql bytes 32G..32G+31 (pieces 0, 1); piece 2 holds its qh bit pairs, byte 4m + i
    = pairs(8m + i) << 4 | pairs(8m + 4 + i) with pairs(t) = qh[32h+t] bits 2p..2p+1 |
    bits 4+2p..5+2p << 2; side: scales 8h+2p, 8h+2p+1, 8h+4+2p, 8h+5+2p as one dword at
    3072 + 4 l, and row slot s's d at 3328 + 2 s."""
    n_out = w.shape[0]
    groups, tiles = n_in // 256, (n_out + 15) // 16
    rows = np.zeros((tiles * 16, w.shape[1]), np.uint8)
    rows[:n_out] = w
    units = np.zeros((tiles, groups, UNIT[encoding]), np.uint8)
    side = PIECES[encoding] * 1024
    for t in range(tiles):
        for g in range(groups):
            u = units[t, g]
            for lane in range(64):
                G, s = lane // 16, lane % 16
                row = rows[16 * t + s]
                if encoding == Q6_K:
                    block = row[210 * g:210 * (g + 1)].astype(np.uint32)
                    h, p = G // 2, G % 2
                    u[16 * lane:16 * lane + 16] = block[32 * G:32 * G + 16]
                    u[1024 + 16 * lane:1024 + 16 * lane + 16] = block[32 * G + 16:32 * G + 32]
                    qh = block[128 + 32 * h:160 + 32 * h]
                    pairs = ((qh >> (2 * p)) & 3) | (((qh >> (4 + 2 * p)) & 3) << 2)
                    for m in range(4):
                        for i in range(4):
                            u[2048 + 16 * lane + 4 * m + i] = \
                                (pairs[8 * m + i] << 4) | pairs[8 * m + 4 + i]
                    sc = 192 + 8 * h + 2 * p
                    u[3072 + 4 * lane:3076 + 4 * lane] = block[[sc, sc + 1, sc + 4, sc + 5]]
                    u[3328 + 2 * s:3330 + 2 * s] = block[208:210]
                elif encoding == Q4_K:
                    block = row[144 * g:144 * (g + 1)]
                    for p in range(2):
                        u[p * 1024 + 16 * lane:p * 1024 + 16 * lane + 16] = \
                            block[16 + 32 * G + 16 * p:32 + 32 * G + 16 * p]
                    u[side + 16 * s:side + 16 * s + 16] = block[:16]
                else:
                    bb = BLOCK[encoding]
                    b0 = (8 * g + 2 * G) * bb
                    for p in range(PIECES[encoding]):
                        if encoding == Q4_0:
                            src = b0 + p * bb + 2
                        else:
                            src = b0 + (p // 2) * bb + 2 + 16 * (p % 2)
                        u[p * 1024 + 16 * lane:p * 1024 + 16 * lane + 16] = row[src:src + 16]
                    u[side + 4 * lane:side + 4 * lane + 2] = row[b0:b0 + 2]
                    u[side + 4 * lane + 2:side + 4 * lane + 4] = row[b0 + bb:b0 + bb + 2]
    return units.reshape(-1)


@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("n_in,n_out", [(256, 1), (512, 37), (1024, 48), (768, 16)])
def test_pack_layout_bytes(device, encoding, n_in, n_out):
    import torch
    from kadan_amd import ops
    w = synth.gguf_weights(encoding, 0x9A + n_out, n_out, n_in)
    packed = ops.gguf_pack(encoding, torch.from_numpy(w).to(device), n_in)
    torch.cuda.synchronize()
    assert packed.numel() == (n_out + 15) // 16 * (n_in // 256) * UNIT[encoding]
    assert np.array_equal(packed.cpu().numpy(), numpy_pack(encoding, w, n_in))


def test_pack_strided_rows(device):
    """Rows further apart than their packed size (row_bytes > minimum) pack the same."""
    import torch
    from kadan_amd import ops
    import kadan_amd
    n_in, n_out = 512, 20
    w = synth.gguf_weights(Q4_K, 5, n_out, n_in)
    wide = np.zeros((n_out, w.shape[1] + 10), np.uint8)
    wide[:, :w.shape[1]] = w
    dw = torch.from_numpy(wide).to(device)
    out = torch.empty(ops.gguf_packed_bytes(Q4_K, n_in, n_out), dtype=torch.uint8, device=device)
    kadan_amd.call("kdq_gguf_pack", Q4_K, dw.data_ptr(), wide.shape[1], n_in, n_out,
                   out.data_ptr(), ops._stream())
    assert np.array_equal(out.cpu().numpy(), numpy_pack(Q4_K, w, n_in))


PRODUCT_SHAPES = [  # (rows, n_in, n_out)
    (1, 256, 1), (1, 256, 7), (1, 512, 64), (2, 1024, 33), (3, 2048, 100), (1, 4096, 257),
    (8, 4096, 64), (5, 14336, 40), (1, 14336, 130), (4, 8192, 96), (9, 1024, 24),
    (1, 4096, 14336), (1, 14336, 4096),
]


@pytest.mark.parametrize("encoding", ENCODINGS)
@pytest.mark.parametrize("rows,n_in,n_out", PRODUCT_SHAPES)
def test_gemv_packed_matches(device, oracle, encoding, rows, n_in, n_out):
    import torch
    from kadan_amd import ops
    w = synth.gguf_weights(encoding, 0x51 + n_in + n_out, n_out, n_in)
    x = synth.normal(0x52 + rows, 3, rows * n_in).reshape(rows, n_in)
    dw = torch.from_numpy(w).to(device)
    dx = torch.from_numpy(x).to(device)
    packed = ops.gguf_pack(encoding, dw, n_in)
    st = torch.zeros(1, dtype=torch.int32, device=device)
    got = ops.gemv_packed(encoding, packed, dx, n_out, status=st).cpu().numpy()
    row_major = ops.gemv(encoding, dw, dx, n_out).cpu().numpy()
    assert bits_equal(got, row_major), "packed product differs from the row-major one"
    assert int(st.item()) == 0
    if n_in * n_out <= 4096 * 4096:  # the oracle's double product on the smaller shapes
        assert_close(got, oracle.gemv(encoding, w, x, n_in, n_out),
                     what=f"enc={encoding} {rows}x{n_in}->{n_out}")


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_gemv_packed_nonfinite_scale(device, encoding):
    """A non-finite block scale in a live row sets the status flag; zero rows that pad
    the last tile never do."""
    import torch
    from kadan_amd import ops
    n_in, n_out = 512, 21
    w = synth.gguf_weights(encoding, 77, n_out, n_in)
    x = torch.from_numpy(synth.normal(78, 1, n_in).reshape(1, n_in)).to(device)
    st = torch.zeros(1, dtype=torch.int32, device=device)
    ops.gemv_packed(encoding, ops.gguf_pack(encoding, torch.from_numpy(w).to(device), n_in),
                    x, n_out, status=st)
    assert int(st.item()) == 0
    bad = w.copy()
    at = SCALE_AT[encoding]
    bad[20, at], bad[20, at + 1] = 0x00, 0x7C  # +inf scale in the last row's first block
    st.zero_()
    y = ops.gemv_packed(encoding, ops.gguf_pack(encoding, torch.from_numpy(bad).to(device), n_in),
                        x, n_out, status=st)
    assert int(st.item()) == 1
    assert not np.isfinite(y[0, 20].item())


@pytest.mark.parametrize("encoding", ENCODINGS)
def test_gemv_packed_batch_matches_single(device, encoding):
    """A submission over packed weights (fused same-shape jobs, a shared input, jobs of
    other shapes) equals one kdq_gemv_packed per job bit for bit."""
    import torch
    from kadan_amd import ops
    specs = [(1, 4096, 1000), (1, 4096, 777), (2, 1024, 64), (1, 4096, 16), (3, 512, 40)]
    jobs, singles = [], []
    shared = torch.from_numpy(synth.normal(90, 1, 4096).reshape(1, 4096)).to(device)
    for i, (rows, n_in, n_out) in enumerate(specs):
        w = torch.from_numpy(synth.gguf_weights(encoding, 91 + i, n_out, n_in)).to(device)
        packed = ops.gguf_pack(encoding, w, n_in)
        x = shared if (rows, n_in) == (1, 4096) else torch.from_numpy(
            synth.normal(95 + i, 1, rows * n_in).reshape(rows, n_in)).to(device)
        y = torch.full((rows, n_out), float("nan"), device=device)
        jobs.append({"encoding": encoding, "weights": packed, "columns": n_out, "input": x,
                     "output": y})
        singles.append(ops.gemv_packed(encoding, packed, x, n_out))
    ops.gemv_packed_batch(jobs)
    for j, s in zip(jobs, singles):
        assert bits_equal(j["output"].cpu().numpy(), s.cpu().numpy())


def test_packed_rejections(device):
    import torch
    import kadan_amd
    from kadan_amd import ops
    w = torch.zeros(16, 144, dtype=torch.uint8, device=device)
    # in % 256 != 0 has no packed form
    assert ops.gguf_packed_bytes(Q4_0, 96, 16) == 0
    with pytest.raises(kadan_amd.KdqError):
        kadan_amd.call("kdq_gguf_pack", Q4_0, w.data_ptr(), 54, 96, 16, w.data_ptr() + 4096,
                       ops._stream())
    # in beyond what the MFMA kernel's LDS holds is unsupported, before any launch
    big = 64 * 1024
    packed = torch.zeros(ops.gguf_packed_bytes(Q4_K, big, 16), dtype=torch.uint8, device=device)
    x = torch.zeros(1, big, device=device)
    with pytest.raises(kadan_amd.KdqUnsupported):
        ops.gemv_packed(Q4_K, packed, x, 16)
    # misaligned packed pointer
    y = torch.empty(1, 16, device=device)
    x = torch.zeros(1, 256, device=device)
    buf = torch.zeros(2304 + 64, dtype=torch.uint8, device=device)
    with pytest.raises(kadan_amd.KdqError):
        kadan_amd.call("kdq_gemv_packed", Q4_K, buf.data_ptr() + 4, x.data_ptr(), 1, 256, 16,
                       y.data_ptr(), 16, None, ops._stream())

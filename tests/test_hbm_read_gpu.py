"""GPU check of the read-ceiling probe kdq_hbm_read: every 16-byte unit of the buffer is
read exactly once, so each workgroup's word is the xor of the 32-bit words of its share
(contiguous shares of ceil(units / workgroups) units rounded up to a multiple of 64;
trailing workgroups may be empty); the read-only form stores a workgroup's fold only
where it equals `match`."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _folds(data, nbytes, workgroups):
    units = nbytes // 16
    per = (-(-units // workgroups) + 63) // 64 * 64
    words = data.reshape(units, 4)
    out = np.zeros(workgroups, np.uint32)
    for b in range(workgroups):
        share = words[b * per:min(units, (b + 1) * per)]
        out[b] = np.bitwise_xor.reduce(share.ravel()) if share.size else np.uint32(0)
    return out


@pytest.mark.parametrize("threads", [256, 1024])
@pytest.mark.parametrize("nbytes,workgroups", [(16, 1), (4096, 3), (1 << 20, 256),
                                               (33103872, 256), (33030144, 1024),
                                               (16 * 1001, 4096)])
def test_hbm_read_folds_every_word(device, nbytes, workgroups, threads):
    import torch
    from kadan_amd import ops
    data = np.random.default_rng(nbytes).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(data.view(np.int32)).to(device)
    want = _folds(data, nbytes, workgroups)
    sink = torch.full((workgroups,), -1, dtype=torch.int32, device=device)
    ops.hbm_read(buf, sink, workgroups, threads)
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)
    # read-only form: only the workgroups whose fold equals `match` store
    sink.fill_(-1)
    ops.hbm_read(buf, sink, workgroups, threads, store_all=False, match=int(want[0]))
    got = sink.cpu().numpy().view(np.uint32)
    hit = want == want[0]
    assert np.array_equal(got[hit], want[hit])
    assert (got[~hit] == np.uint32(0xFFFFFFFF)).all()

"""kdq_moe_mxfp4_packed_noalloc (the allocation-free entry point, its scratch in a static
device array) against kdq_moe_mxfp4_packed, through the C ABI: two calls in a row, the
second with fewer tokens (the array keeps the first call's contents), each bit-identical
to the allocating entry point in output and routing; a layer whose scratch exceeds the
array is refused before any launch."""
import ctypes

import numpy as np
import pytest

import kadan_amd
from kadan_amd import ops, synth

pytestmark = pytest.mark.gpu


def _call_noalloc(torch, x, logits, top_k, inter, packed):
    t, h = x.shape
    e = logits.shape[1]
    dev = x.device
    y = torch.full((t, h), float("nan"), dtype=torch.float32, device=dev)
    idx = torch.full((t, top_k), -1, dtype=torch.int32, device=dev)
    w = torch.full((t, top_k), float("nan"), dtype=torch.float32, device=dev)
    offsets = torch.full((e + 1,), -1, dtype=torch.int32, device=dev)
    perm = torch.full((t * top_k,), -1, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    kadan_amd.call("kdq_moe_mxfp4_packed_noalloc", x.data_ptr(), logits.data_ptr(), t, h, inter,
                   e, top_k, packed[0].data_ptr(), packed[1].data_ptr(), packed[2].data_ptr(),
                   y.data_ptr(), idx.data_ptr(), w.data_ptr(), offsets.data_ptr(),
                   perm.data_ptr(), stream)
    return y, idx, w, offsets, perm


@pytest.mark.parametrize("hidden,inter,experts,tokens", [(2880, 2880, 32, (64, 1)),
                                                         (256, 192, 8, (37, 5))])
def test_noalloc_matches_allocating_entry(device, hidden, inter, experts, tokens):
    import torch
    top_k = 4
    weights = synth.moe_weights_torch(0x7A, experts, hidden, inter, device)
    packed = [ops.moe_mxfp4_pack(*weights[0], experts, inter, hidden),
              ops.moe_mxfp4_pack(*weights[1], experts, inter, hidden),
              ops.moe_mxfp4_pack(*weights[2], experts, hidden, inter)]
    for n in tokens:  # the second call is smaller: the array holds the first's contents
        x, logits = synth.moe_inputs(0x7B + n, n, hidden, experts)
        xb = torch.from_numpy(x).to(device).view(torch.bfloat16)
        lg = torch.from_numpy(logits).to(device)
        got = _call_noalloc(torch, xb, lg, top_k, inter, packed)
        want = ops.moe_mxfp4_packed(xb, lg, top_k, inter, *packed, routing=True)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert np.array_equal(a.cpu().numpy().view(np.uint8), b.cpu().numpy().view(np.uint8))


def test_noalloc_refuses_what_does_not_fit(device):
    """C4 geometry at 512 tokens needs about 103 MiB of scratch: refused with the scratch
    status before any launch (the output keeps its contents)."""
    import torch
    hidden = inter = 2880
    experts, top_k, tokens = 32, 4, 512
    packed = [torch.zeros(kadan_amd.lib().kdq_moe_mxfp4_packed_bytes(experts, r, c),
                          dtype=torch.uint8, device=device)
              for r, c in ((inter, hidden), (inter, hidden), (hidden, inter))]
    x = torch.zeros(tokens, hidden, dtype=torch.bfloat16, device=device)
    logits = torch.zeros(tokens, experts, dtype=torch.float32, device=device)
    with pytest.raises(kadan_amd.KdqError, match="kdq_projection_scratch"):
        _call_noalloc(torch, x, logits, top_k, inter, packed)

"""CPU checks of the C ABI: the library loads, exports every entry point that
include/kadan_amd.h declares, and rejects invalid arguments before any launch."""
import ctypes as C
import os
import re

import numpy as np

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kadan_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kdq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for expected in ["kdq_dequantize", "kdq_gemv", "kdq_gemv_batch", "kdq_gemm_q4_0",
                     "kdq_gemm_q4_0_packed",
                     "kdq_moe_route", "kdq_moe_mxfp4", "kdq_mxfp4_dequantize",
                     "kdq_moe_mxfp4_pack", "kdq_moe_mxfp4_packed", "kdq_moe_mxfp4_packed_bytes"]:
        assert expected in names


def test_library_exports_every_declared_symbol():
    import kadan_amd
    lib = kadan_amd.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python wrapper binds exactly the declared set
    assert sorted(kadan_amd.exported_symbols()) == declared_functions()


def test_block_geometry():
    import kadan_amd
    lib = kadan_amd.lib()
    assert (lib.kdq_block_values(2), lib.kdq_block_bytes(2)) == (32, 18)
    assert (lib.kdq_block_values(8), lib.kdq_block_bytes(8)) == (32, 34)
    assert (lib.kdq_block_values(12), lib.kdq_block_bytes(12)) == (256, 144)
    assert lib.kdq_block_values(3) == 0
    assert lib.kdq_row_bytes(12, 4096) == 2304
    assert lib.kdq_row_bytes(8, 4096) == 4352
    assert lib.kdq_row_bytes(2, 4096) == 2304
    assert lib.kdq_row_bytes(12, 100) == 0


def test_status_strings():
    import kadan_amd
    lib = kadan_amd.lib()
    assert lib.kdq_status_string(0) == b"ok"
    assert lib.kdq_status_string(2) == b"kdq_projection_shape"
    assert lib.kdq_status_string(4) == b"kdq_alias"


# Argument validation happens on the host before any HIP call, so these run without
# a GPU: the pointers are never dereferenced.
FAKE_W, FAKE_X, FAKE_Y = 0x10000000, 0x20000000, 0x30000000


def test_gemv_argument_errors():
    import kadan_amd
    lib = kadan_amd.lib()
    # unknown encoding
    assert lib.kdq_gemv(3, FAKE_W, 144, FAKE_X, 1, 256, 4, FAKE_Y, 4, None, None) == 3
    # null pointers / zero sizes
    assert lib.kdq_gemv(12, None, 144, FAKE_X, 1, 256, 4, FAKE_Y, 4, None, None) == 1
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 0, 256, 4, FAKE_Y, 4, None, None) == 1
    # ragged row, short row bytes, stride < out, too many rows
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 1, 200, 4, FAKE_Y, 4, None, None) == 2
    assert lib.kdq_gemv(12, FAKE_W, 100, FAKE_X, 1, 256, 4, FAKE_Y, 4, None, None) == 2
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 1, 256, 4, FAKE_Y, 3, None, None) == 2
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 4097, 256, 4, FAKE_Y, 4, None, None) == 2
    # output overlapping the weights or the input
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 1, 256, 4, FAKE_W + 16, 4, None, None) == 4
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X, 1, 256, 4, FAKE_X, 4, None, None) == 4
    # misaligned activations
    assert lib.kdq_gemv(12, FAKE_W, 144, FAKE_X + 4, 1, 256, 4, FAKE_Y, 4, None, None) == 7


def test_batch_validates_every_job_first():
    import kadan_amd
    lib = kadan_amd.lib()
    jobs = (kadan_amd.MatvecJob * 2)()
    jobs[0] = kadan_amd.MatvecJob(FAKE_W, FAKE_X, FAKE_Y, 0, 144, 4, 256, 4, 1, 12)
    jobs[1] = kadan_amd.MatvecJob(FAKE_W, FAKE_X, FAKE_Y + 4096, 0, 144, 4, 200, 4, 1, 12)
    # the second job is ragged: nothing may be launched for the first one either
    assert lib.kdq_gemv_batch(C.addressof(jobs), 2, None) == 2
    assert lib.kdq_gemv_batch(None, 0, None) == 0


def test_dequantize_argument_errors():
    import kadan_amd
    lib = kadan_amd.lib()
    assert lib.kdq_dequantize(12, FAKE_W, 144, 1, 200, FAKE_Y, None, None) == 2
    assert lib.kdq_dequantize(12, FAKE_W, 144, 1, 256, FAKE_Y + 4, None, None) == 7
    assert lib.kdq_dequantize(12, FAKE_W, 144, 1, 256, FAKE_W, None, None) == 4


def test_moe_packed_geometry_and_argument_errors():
    import kadan_amd
    lib = kadan_amd.lib()
    # 32 experts x 2880 x 2880: codes E*R*C/2, scales E * R/32 * ceil(45/4) * 256
    assert lib.kdq_moe_mxfp4_packed_bytes(32, 2880, 2880) == 32 * 2880 * 1440 + 32 * 90 * 12 * 256
    assert lib.kdq_moe_mxfp4_packed_bytes(1, 32, 64) == 1024 + 256
    assert lib.kdq_moe_mxfp4_packed_bytes(1, 48, 64) == 0
    assert lib.kdq_moe_mxfp4_packed_bytes(1, 32, 96) == 0
    pack = lib.kdq_moe_mxfp4_pack
    assert pack(FAKE_W, FAKE_W + 65536, 1, 48, 64, FAKE_Y, None) == 2
    assert pack(FAKE_W, FAKE_W + 65536, 1, 32, 64, FAKE_Y + 16, None) == 7
    assert pack(FAKE_W + 4, FAKE_W + 65536, 1, 32, 64, FAKE_Y, None) == 7
    assert pack(FAKE_W, FAKE_W + 65536, 1, 32, 64, FAKE_W + 256, None) == 4
    assert pack(None, FAKE_W, 1, 32, 64, FAKE_Y, None) == 1


def test_product_path_has_no_cpu_fallback(monkeypatch, tmp_path):
    """Without the built library the package raises instead of computing on the CPU."""
    import kadan_amd
    monkeypatch.setattr(kadan_amd, "LIBRARY", str(tmp_path / "missing.so"))
    monkeypatch.setattr(kadan_amd, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kadan_amd.lib()


def test_gguf_packed_geometry_and_argument_errors():
    import kadan_amd
    lib = kadan_amd.lib()
    # tiles of 16 rows x groups of 256 values, one unit of 16 x group bytes each
    assert lib.kdq_gguf_packed_bytes(12, 4096, 14336) == 14336 * 2304
    assert lib.kdq_gguf_packed_bytes(12, 256, 17) == 2 * 2304
    assert lib.kdq_gguf_packed_bytes(8, 512, 16) == 2 * 4352
    assert lib.kdq_gguf_packed_bytes(2, 512, 1) == 2 * 2304
    assert lib.kdq_gguf_packed_bytes(14, 4096, 14336) == 14336 * 16 * 210  # Q6_K
    assert lib.kdq_gguf_packed_bytes(14, 768, 17) == 2 * 3 * 3360
    assert lib.kdq_gguf_packed_bytes(2, 96, 16) == 0
    assert lib.kdq_gguf_packed_bytes(3, 256, 16) == 0
    pack = lib.kdq_gguf_pack
    assert pack(3, FAKE_W, 144, 256, 16, FAKE_Y, None) == 3
    assert pack(12, None, 144, 256, 16, FAKE_Y, None) == 1
    assert pack(12, FAKE_W, 100, 256, 16, FAKE_Y, None) == 2
    assert pack(2, FAKE_W, 54, 96, 16, FAKE_Y, None) == 2
    assert pack(12, FAKE_W, 144, 256, 16, FAKE_Y + 4, None) == 7
    assert pack(12, FAKE_W, 144, 256, 16, FAKE_W + 256, None) == 4
    gp = lib.kdq_gemv_packed
    assert gp(12, FAKE_W, FAKE_X, 1, 200, 4, FAKE_Y, 4, None, None) == 2
    assert gp(12, FAKE_W, FAKE_X, 1, 256, 4, FAKE_Y, 3, None, None) == 2
    assert gp(12, FAKE_W, FAKE_X, 4097, 256, 4, FAKE_Y, 4, None, None) == 2
    assert gp(12, FAKE_W, FAKE_X, 1, 256, 4, FAKE_W + 16, 4, None, None) == 4
    assert gp(12, FAKE_W + 4, FAKE_X, 1, 256, 4, FAKE_Y, 4, None, None) == 7
    assert gp(12, FAKE_W, FAKE_X + 4, 1, 256, 4, FAKE_Y, 4, None, None) == 7
    jobs = (kadan_amd.MatvecJob * 2)()
    jobs[0] = kadan_amd.MatvecJob(FAKE_W, FAKE_X, FAKE_Y, 0, 0, 4, 256, 4, 1, 12)
    jobs[1] = kadan_amd.MatvecJob(FAKE_W, FAKE_X, FAKE_Y + 4096, 0, 0, 4, 200, 4, 1, 12)
    assert lib.kdq_gemv_packed_batch(C.addressof(jobs), 2, None) == 2
    assert lib.kdq_gemv_packed_batch(None, 0, None) == 0


def test_gemm_packed_argument_errors():
    import kadan_amd
    lib = kadan_amd.lib()
    g = lib.kdq_gemm_q4_0_packed
    assert g(None, 16, 256, FAKE_X, 1, FAKE_Y, None) == 1
    assert g(FAKE_W, 16, 256, FAKE_X, 0, FAKE_Y, None) == 1
    assert g(FAKE_W, 16, 200, FAKE_X, 1, FAKE_Y, None) == 2        # k % 256
    assert g(FAKE_W, 1 << 24, 256, FAKE_X, 1, FAKE_Y, None) == 2   # n too large
    assert g(FAKE_W + 4, 16, 256, FAKE_X, 1, FAKE_Y, None) == 7    # packed not 16-aligned
    assert g(FAKE_W, 16, 256, FAKE_X + 8, 1, FAKE_Y, None) == 7    # activations not 16-aligned
    assert g(FAKE_W, 16, 256, FAKE_X, 1, FAKE_Y + 1, None) == 7    # output not 2-aligned
    assert g(FAKE_W, 16, 256, FAKE_X, 1, FAKE_W + 32, None) == 4   # output inside packed
    assert g(FAKE_W, 16, 256, FAKE_X, 1, FAKE_X + 64, None) == 4   # output inside x


def test_synth_torch_streams_match_numpy():
    """The torch SplitMix64 streams (used to build C4/C5 weights on the device) give the
    numpy generator's bytes bit for bit."""
    import torch
    from kadan_amd import synth
    a = synth.moe_weights(7, 3, 128, 192)
    b = synth.moe_weights_torch(7, 3, 128, 192, "cpu")
    for (blocks, scales), (tb, ts) in zip(a, b):
        assert np.array_equal(blocks, tb.numpy()) and np.array_equal(scales, ts.numpy())
    assert np.array_equal(synth.splitmix64(5, 9, 1000).view(np.int64),
                          synth.splitmix64_torch(5, 9, 1000, "cpu").numpy())
    assert torch.equal(synth._umod_small(torch.tensor([-1], dtype=torch.int64), 9),
                       torch.tensor([(2 ** 64 - 1) % 9]))


def test_gemm_check_and_moe_gguf_packed_argument_errors():
    """kdq_gguf_gemm_check and kdq_moe_gguf_packed refuse bad arguments before any launch:
    null pointers, encodings the prefill GEMM does not read, a K off the 256-value grid,
    and misaligned device pointers (a resident packed copy included)."""
    import kadan_amd
    lib = kadan_amd.lib()
    chk = lib.kdq_gguf_gemm_check
    assert chk(12, None, 16, 256, FAKE_Y, None) == 1
    assert chk(12, FAKE_W, 16, 256, None, None) == 1
    assert chk(2, FAKE_W, 16, 256, FAKE_Y, None) == 3      # Q4_0: not read by the GEMM
    assert chk(12, FAKE_W, 16, 200, FAKE_Y, None) == 2     # k % 256
    assert chk(12, FAKE_W + 4, 16, 256, FAKE_Y, None) == 7  # packed not 16-aligned
    assert chk(12, FAKE_W, 16, 256, FAKE_Y + 2, None) == 7  # flags not 4-aligned
    H, E, K, F, S = 256, 8, 2, 256, 256
    layer = kadan_amd.MoeGgufLayer(H, E, K, F, S)
    q4k = lambda rows: kadan_amd.GgufTensor(FAKE_W, 144, rows * 144, 12)
    layer.router = kadan_amd.GgufTensor(FAKE_W, H * 4, 0, 0)
    layer.gate_exps, layer.up_exps, layer.down_exps = q4k(F), q4k(F), q4k(H)
    layer.gate_shexp = layer.up_shexp = layer.down_shexp = kadan_amd.GgufTensor(FAKE_W, 144, 0, 12)
    layer.shared_gate = FAKE_W
    stacks = kadan_amd.MoeGgufPackedStacks(FAKE_W + 8, None, None, None, None, None, 1)
    f = lib.kdq_moe_gguf_packed
    assert f(None, C.addressof(stacks), FAKE_X, 1, FAKE_Y, None, None, None, None) == 1
    assert f(C.addressof(layer), C.addressof(stacks), FAKE_X, 1, FAKE_Y, None, None, None,
             None) == 7

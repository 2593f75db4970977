"""Checkpoint bytes through the device path: GGUF rows decoded on the device
(GgufFiles::decode_rows, the literal blocks of IW/tests/gguf_checkpoint.cpp:399-460),
GGUF expert tensors as the weight source of HipDenseCompute::dense_gguf_source (decode-
time product and prefill GEMM) against the oracle, and a GPT-OSS MXFP4 expert set loaded
from a safetensors shard into the MoE layer against the oracle."""
import numpy as np
import pytest

from kadan_amd import synth
from tests import formats
from tests.formats import Gguf, Safetensors
from tests.test_checkpoint import literal_blocks, metadata
from tests.test_dense_compute_gpu import FINITE, Probe
from tests.util import assert_close

pytestmark = pytest.mark.gpu

Q8_0, Q3_K, Q4_K, Q6_K = 8, 11, 12, 14


@pytest.fixture()
def probe(device):
    p = Probe()
    yield p
    p.close()


def test_read_rows_decodes_literal_blocks(tmp_path, probe):
    q3, q4, q8 = literal_blocks()
    formats.write_gguf(tmp_path / "m.gguf", metadata(),
                       [("q3", Q3_K, [256, 2, 2], q3), ("q4", Q4_K, [256, 2, 2], q4),
                        ("q8", Q8_0, [256, 2, 2], q8)])
    g = Gguf(str(tmp_path))
    assert (g.read_rows(probe, "q3", 1, 1, 256) == 512).all()  # 128 * d, d = 4
    v = g.read_rows(probe, "q4", 1, 0, 256)  # d = 3: 3 at low nibbles, 6 at high
    assert np.array_equal(v, np.where(np.arange(256) % 64 < 32, 3.0, 6.0).astype(np.float32))
    v = g.read_rows(probe, "q8", 0, 1, 256)  # d = 2
    assert np.array_equal(v, (2.0 * (np.arange(256) % 32 - 16)).astype(np.float32))
    both = g.read_rows(probe, "q8", 1, 0, 512)  # two rows: d = 3, 4
    assert np.array_equal(both[256:], (4.0 * (np.arange(256) % 32 - 16)).astype(np.float32))
    g.close()


@pytest.mark.parametrize("enc", [Q4_K, Q6_K, Q8_0])
@pytest.mark.parametrize("rows", [3, 40])
def test_gguf_expert_through_dense_gguf_source(tmp_path, probe, oracle, enc, rows):
    """A 2-expert tensor [512 in, 384 out, 2] in a GGUF file: expert 1 through the
    checkpoint's own identity and packed-row source (3 rows: decode-time product; 40 rows:
    the prefill GEMM)."""
    n_in, n_out = 512, 384
    w = synth.gguf_weights(enc, 0xF1, 2 * n_out, n_in)
    formats.write_gguf(tmp_path / "m.gguf", metadata(),
                       [("blk.0.ffn_up_exps.weight", enc, [n_in, n_out, 2], w.tobytes())])
    g = Gguf(str(tmp_path))
    x = synth.normal(0xF2, rows, rows * n_in).reshape(rows, n_in)
    res, y = g.dense_source(probe, "blk.0.ffn_up_exps.weight", 1, x, n_out)
    assert res == FINITE
    assert_close(y, oracle.gemv(enc, w[n_out:], x, n_in, n_out),
                 what=f"gguf file -> dense_gguf_source enc={enc} rows={rows}")
    assert probe.retained == w.size // 2  # the bank holds the one expert slice
    g.close()


def test_safetensors_mxfp4_experts_into_the_moe_layer(tmp_path, probe, oracle):
    """GPT-OSS expert tensors (<prefix>_blocks U8 [E, rows, groups, 16], <prefix>_scales U8
    [E, rows, groups]) loaded by SafetensorsFile::mxfp4_experts into
    HipDenseCompute::moe_mxfp4."""
    experts, hidden, inter, tokens, top_k = 4, 128, 192, 5, 2
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(0xF3, experts, hidden, inter)
    tensors = {}
    for name, b, s, rows, cols in (("gate", gb, gs, inter, hidden), ("up", ub, us, inter, hidden),
                                   ("down", db, ds, hidden, inter)):
        tensors[f"model.layers.0.mlp.experts.{name}_blocks"] = (
            "U8", [experts, rows, cols // 32, 16], b.tobytes())
        tensors[f"model.layers.0.mlp.experts.{name}_scales"] = (
            "U8", [experts, rows, cols // 32], s.tobytes())
    path = str(tmp_path / "model-00001-of-00001.safetensors")
    formats.write_safetensors(path, tensors, {"format": "pt"})
    x, logits = synth.moe_inputs(0xF4, tokens, hidden, experts)
    want, idx, w, _, _ = oracle.moe_forward(x, logits, top_k, gb, gs, ub, us, db, ds)
    s = Safetensors(path)
    p = "model.layers.0.mlp.experts."
    res, y, sel, rw = s.moe(probe, p + "gate", p + "up", p + "down", x, logits, top_k, hidden)
    assert res == FINITE
    assert np.array_equal(sel, idx)
    assert_close(y, want, what="safetensors experts -> moe_mxfp4")
    s.close()

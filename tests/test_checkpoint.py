"""The on-disk readers (include/kadan_amd_checkpoint.hpp) on the CPU, against the cases of
the reference's own reader tests: IW/tests/gguf_checkpoint.cpp:399-540 (reader_rows: a
split set with literal Q3_K / Q4_K / Q8_0 blocks, identities, packed rows, metadata,
range / cancel / changed-file refusals) and IW/tests/checkpoint.cpp:229-380 (the GPT-OSS
MXFP4 expert fixture: rows of one expert, budget, shape and scale refusals).  Decoded
values are checked in test_checkpoint_gpu.py (the decode runs on the device)."""
import os

import numpy as np
import pytest

from tests import formats
from tests.formats import (ARRAY, BOOL, F32, I32, STRING, U32, U64, Gguf, ReaderError,
                           Safetensors)

Q8_0, Q3_K, Q4_K = 8, 11, 12


def literal_blocks():
    """Per (expert, row) one block set with fp16 multiplier 1, 2, 3, 4 (IW/tests/
    gguf_checkpoint.cpp:399-425): Q3_K all weights 128 d; Q4_K scales 1 and codes 0x21
    (d at low nibbles, 2d at high); Q8_0 codes -16..15 times d."""
    q3, q4, q8 = bytearray(), bytearray(), bytearray()
    for d in (0x3C00, 0x4000, 0x4200, 0x4400):
        b3 = bytearray(110)
        b3[108], b3[109] = d & 255, d >> 8
        q3 += b3
        b4 = bytearray(144)
        b4[0], b4[1] = d & 255, d >> 8
        b4[4:16] = bytes([1] * 12)
        b4[16:] = bytes([0x21] * 128)
        q4 += b4
        for _ in range(8):
            q8 += bytes([d & 255, d >> 8]) + bytes((v & 255) for v in range(-16, 16))
    return bytes(q3), bytes(q4), bytes(q8)


def metadata(split=None, total=4):
    m = []
    if split is not None:
        m += [("split.no", U32, split), ("split.count", U32, 2), ("split.tensors.count", U32, total)]
    m += [("muse-spark.hash_offsets", ARRAY, (U64, [0, 300001275])),
          ("general.architecture", STRING, "muse-spark"),
          ("muse-spark.expert_weights_norm", BOOL, True),
          ("muse-spark.temperature", F32, 0.5),
          ("muse-spark.attention_swa", ARRAY, (BOOL, [True, False, True])),
          ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "b"])),
          ("tokenizer.ggml.token_type", ARRAY, (I32, [1, 3])),
          ("general.alignment", U32, 32)]
    return m


@pytest.fixture()
def split_set(tmp_path):
    q3, q4, q8 = literal_blocks()
    vec = np.array([1, -2, 3, -4], np.float32).tobytes()
    formats.write_gguf(tmp_path / "muse-00001-of-00002.gguf", metadata(0), [])
    formats.write_gguf(tmp_path / "muse-00002-of-00002.gguf", metadata(1),
                       [("vector", 0, [4], vec), ("q3", Q3_K, [256, 2, 2], q3),
                        ("q4", Q4_K, [256, 2, 2], q4), ("q8", Q8_0, [256, 2, 2], q8)])
    return str(tmp_path), {"q3": q3, "q4": q4, "q8": q8}


def test_gguf_split_set_tensors_and_identity(split_set):
    root, data = split_set
    g = Gguf(root)
    assert g.tensor_count() == 4
    shape, rank, kind, nbytes = g.tensor("q3")
    assert shape == (256, 2, 2) and rank == 3 and kind == Q3_K and nbytes == 440
    id0, id1 = g.identity("q3", 0), g.identity("q3", 1)
    assert id0[8] == id1[7] and id0[8] - id0[7] == 220  # consecutive 220-byte slices
    st = os.stat(os.path.join(root, "muse-00002-of-00002.gguf"))
    assert id0[:3] == [st.st_dev, st.st_ino, st.st_size]
    with pytest.raises(ReaderError, match="gguf_expert_range"):
        g.identity("q3", 2)
    with pytest.raises(ReaderError, match="gguf_missing_tensor"):
        g.tensor("absent")
    g.close()


def test_gguf_packed_rows(split_set):
    root, data = split_set
    g = Gguf(root)
    for name, raw in data.items():
        row = len(raw) // 4
        assert g.read_packed(name, 1, 0, 2 * row).tobytes() == raw[2 * row:4 * row]
        assert g.read_packed(name, 0, 1, row).tobytes() == raw[row:2 * row]
        assert g.read_packed(name, 0, 2, 0).size == 0
        for expert, first, n in ((2, 0, row), (0, 2, row), (0, 2**64 - 1, 0), (0, 0, row - 1)):
            with pytest.raises(ReaderError, match="gguf_row_range"):
                g.read_packed(name, expert, first, n)
    assert g.read_vector("vector", 4).tolist() == [1, -2, 3, -4]
    with pytest.raises(ReaderError, match="gguf_row_range"):
        g.read_packed("vector", 0, 0, 0)  # rank 1: no rows
    with pytest.raises(ReaderError, match="gguf_cancelled"):
        g.read_packed("q3", 0, 0, 110, cancelled=True)
    g.close()


def test_gguf_metadata(split_set):
    root, _ = split_set
    g = Gguf(root)
    assert g.meta("general.architecture", 0) == "muse-spark"
    assert g.meta("split.count", 1) == 2
    assert g.meta("muse-spark.temperature", 2) == 0.5
    assert g.meta("muse-spark.expert_weights_norm", 3) is True
    assert g.meta("tokenizer.ggml.tokens", 4) == ["a", "b"]
    assert g.meta("tokenizer.ggml.token_type", 5) == [1, 3]
    assert g.meta("muse-spark.hash_offsets", 5) == [0, 300001275]
    assert g.meta("muse-spark.attention_swa", 7) == [True, False, True]
    assert g.meta("general.architecture", 8) and not g.meta("absent", 8)
    with pytest.raises(ReaderError, match="gguf_metadata_integer"):
        g.meta("general.architecture", 1)
    with pytest.raises(ReaderError, match="gguf_missing_metadata"):
        g.meta("missing", 0)
    g.close()


def test_gguf_changed_file_and_cancel(split_set):
    root, _ = split_set
    with pytest.raises(ReaderError, match="gguf_cancelled"):
        Gguf(root, cancelled=True)
    g = Gguf(root)
    g.check_unchanged()
    with open(os.path.join(root, "muse-00002-of-00002.gguf"), "ab") as f:
        f.write(b"\0")
    with pytest.raises(ReaderError, match="gguf_checkpoint_changed"):
        g.check_unchanged()
    with pytest.raises(ReaderError, match="gguf_checkpoint_changed"):
        g.read_packed("q3", 0, 0, 110)
    g.close()


def test_gguf_single_file_and_refusals(tmp_path):
    q3, q4, q8 = literal_blocks()
    one = tmp_path / "one"
    one.mkdir()
    formats.write_gguf(one / "model.gguf", metadata(), [("q8", Q8_0, [256, 4], q8)])
    g = Gguf(str(one))
    assert g.tensor_count() == 1 and g.tensor("q8")[0] == (256, 4, 1)
    assert g.read_packed("q8", 0, 3, 272).tobytes() == q8[3 * 272:]
    g.close()
    cases = {
        "gguf_version": lambda d: (d / "m.gguf").write_bytes(b"GGUF" + b"\2\0\0\0" + bytes(40)),
        "gguf_tensor_type": lambda d: formats.write_gguf(d / "m.gguf", [],
                                                         [("t", 3, [32, 1], bytes(20))]),
        "gguf_tensor_block_alignment": lambda d: formats.write_gguf(
            d / "m.gguf", [], [("t", Q8_0, [48, 1], bytes(51))]),
        "gguf_split_name": lambda d: [formats.write_gguf(d / n, metadata(i), [])
                                      for i, n in enumerate(("a-00001-of-00002.gguf",
                                                             "a-00003-of-00002.gguf"))],
        "gguf_split_metadata": lambda d: [formats.write_gguf(d / n, metadata(i ^ 1), [])
                                          for i, n in enumerate(("a-00001-of-00002.gguf",
                                                                 "a-00002-of-00002.gguf"))],
    }
    for code, make in cases.items():
        d = tmp_path / code
        d.mkdir()
        make(d)
        with pytest.raises(ReaderError, match=code):
            Gguf(str(d))
    # overlapping payloads: a hand-built header whose two tensors share offset 0
    d = tmp_path / "overlap"
    d.mkdir()
    raw = bytearray(formats.gguf_bytes([], [("a", Q8_0, [32, 1], bytes(34)),
                                            ("b", Q8_0, [32, 1], bytes(34))]))
    at = raw.find(b"\x01\0\0\0\0\0\0\0b", 24) + 9 + 4 + 16 + 4  # name "b", rank, 2 dims, type
    raw[at:at + 8] = bytes(8)
    (d / "m.gguf").write_bytes(bytes(raw))
    with pytest.raises(ReaderError, match="gguf_tensor_overlap"):
        Gguf(str(d))


# ------------------------------------------------------------- safetensors / MXFP4

def mxfp4_fixture(path, invalid_scale=False):
    """IW/tests/checkpoint.cpp:229-239: blocks U8 [2, 3, 2, 16] of 0xA2 (+1, -1) with
    byte 128 = 0x71 (+0.5, +6), scales 124 .. 135 (byte 8 = 255 when invalid)."""
    blocks = bytearray([0xA2] * 192)
    blocks[128] = 0x71
    scales = bytes(255 if invalid_scale and i == 8 else 124 + i for i in range(12))
    formats.write_safetensors(path, {"p_blocks": ("U8", [2, 3, 2, 16], bytes(blocks)),
                                     "p_scales": ("U8", [2, 3, 2], scales)},
                              {"format": "pt"})


def test_mxfp4_expert_rows(tmp_path, oracle):
    path = str(tmp_path / "model.safetensors")
    mxfp4_fixture(path)
    s = Safetensors(path)
    cols, blocks, scales = s.load_rows("p", 1, 1, 2, groups=2, budget=68)
    assert cols == 64
    rc, values = oracle.mxfp4_decode_rows(blocks, scales, 2, 64)
    assert rc == 0
    want = np.array([(-1 if i % 2 else 1) * (32, 64, 128, 256)[i // 32] for i in range(128)],
                    np.float32)
    want[0], want[1] = 16, 192
    assert np.array_equal(values.ravel(), want)
    _, b, sc = s.load_rows("p", 1, 2, 1, groups=2, budget=34)
    assert oracle.mxfp4_decode_rows(b, sc, 1, 64)[1][0, 0] == 128
    _, b, sc = s.load_rows("p", 0, 0, 1, groups=2, budget=34)
    assert oracle.mxfp4_decode_rows(b, sc, 1, 64)[1][0, 0] == 0.125
    ident = s.identity("p_blocks")
    assert ident[8] - ident[7] == 192
    s.close()


def test_mxfp4_load_refusals(tmp_path):
    path = str(tmp_path / "model.safetensors")
    mxfp4_fixture(path)
    s = Safetensors(path)
    with pytest.raises(ReaderError, match="payload_budget"):
        s.load_rows("p", 1, 1, 2, groups=2, budget=67)
    for expert, first, count in ((2, 0, 1), (2**64 - 1, 0, 1), (0, 2, 2), (0, 2**64 - 1, 2)):
        with pytest.raises(ReaderError, match="mxfp4_expert_shape"):
            s.load_rows("p", expert, first, count, groups=2, budget=68)
    for prefix, count in (("p", 0), ("", 1)):
        with pytest.raises(ReaderError, match="projection_range_or_name"):
            s.load_rows(prefix, 0, 0, count, groups=2, budget=68)
    with pytest.raises(ReaderError, match="missing_tensor"):
        s.load_rows("absent", 0, 0, 1, groups=2, budget=68)
    s.close()
    mxfp4_fixture(path, invalid_scale=True)
    s = Safetensors(path)
    with pytest.raises(ReaderError, match="invalid_block_scale"):
        s.load_rows("p", 1, 1, 2, groups=2, budget=68)
    assert s.load_rows("p", 0, 0, 1, groups=2, budget=34)[0] == 64  # other rows unread
    s.close()


@pytest.mark.parametrize("blocks,scales,code", [
    (("I8", [2, 3, 2, 16]), ("U8", [2, 3, 2]), "mxfp4_dtype"),
    (("U8", [2, 3, 2, 16]), ("I8", [2, 3, 2]), "mxfp4_dtype"),
    (("U8", [2, 3, 32]), ("U8", [2, 3, 2]), "mxfp4_expert_shape"),
    (("U8", [2, 3, 4, 8]), ("U8", [2, 3, 2]), "mxfp4_expert_shape"),
    (("U8", [2, 3, 2, 16]), ("U8", [2, 6]), "mxfp4_expert_shape"),
])
def test_mxfp4_layout_refusals(tmp_path, blocks, scales, code):
    path = str(tmp_path / "model.safetensors")
    formats.write_safetensors(path, {"p_blocks": (blocks[0], blocks[1], bytes(192)),
                                     "p_scales": (scales[0], scales[1], bytes(12))})
    s = Safetensors(path)
    with pytest.raises(ReaderError, match=code):
        s.load_rows("p", 0, 0, 1, groups=2, budget=204)
    s.close()


def test_safetensors_header_refusals(tmp_path):
    path = tmp_path / "bad.safetensors"
    path.write_bytes((10**9).to_bytes(8, "little") + b"{}")
    with pytest.raises(ReaderError, match="safetensors_header_size"):
        Safetensors(str(path))
    formats.write_safetensors(str(path), {"a": ("U8", [4], bytes(4)), "b": ("U8", [4], bytes(4))})
    raw = bytearray(path.read_bytes())
    raw = raw.replace(b"[4, 8]", b"[2, 6]")  # b now overlaps a
    path.write_bytes(bytes(raw))
    with pytest.raises(ReaderError, match="safetensors_tensor_overlap"):
        Safetensors(str(path))


# ------------------------------------------------------------- header refusals

def raw_safetensors(path, header_text: str, payload: bytes):
    """A file with this exact JSON header text (padded with spaces to 8 bytes)."""
    text = header_text.encode("latin-1")
    text += b" " * ((8 - len(text) % 8) % 8)
    path.write_bytes(len(text).to_bytes(8, "little") + text + payload)


@pytest.mark.parametrize("header,payload,code", [
    # a gap between two tensors, and payload bytes no tensor covers
    ('{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]},'
     '"b":{"dtype":"U8","shape":[4],"data_offsets":[6,10]}}', bytes(10), "safetensors_tensor_gap"),
    ('{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(6),
     "safetensors_payload_coverage"),
    ('{"a":{"dtype":"U8","shape":[4],"data_offsets":[2,6]}}', bytes(6), "safetensors_tensor_gap"),
    # a field twice, a tensor twice, __metadata__ twice, an unknown field, a missing one
    ('{"a":{"dtype":"U8","dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_duplicate"),
    ('{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]},'
     '"a":{"dtype":"U8","shape":[4],"data_offsets":[4,8]}}', bytes(8), "safetensors_duplicate"),
    ('{"__metadata__":{"k":"v"},"__metadata__":{"k":"w"},'
     '"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4), "safetensors_duplicate"),
    ('{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4],"extra":1}}', bytes(4),
     "safetensors_tensor"),
    ('{"a":{"dtype":"U8","shape":[4]}}', bytes(0), "safetensors_tensor"),
    # non-ASCII text, raw or escaped; \\u with fewer than four hex digits
    ('{"é":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_ascii"),
    ('{"\\u00e9":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_ascii"),
    ('{"\\u12zz":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_json"),
    ('{"\\u004":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_json"),
    # numbers that are not plain unsigned integers; sizes that disagree; unknown dtype
    ('{"a":{"dtype":"U8","shape":[-4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_integer"),
    ('{"a":{"dtype":"U8","shape":[4.0],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_integer"),
    ('{"a":{"dtype":"U8","shape":[18446744073709551616],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_header_integer"),
    ('{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,4]}}', bytes(4),
     "safetensors_tensor_shape"),
    ('{"a":{"dtype":"Q4","shape":[4],"data_offsets":[0,4]}}', bytes(4), "safetensors_dtype"),
    # not JSON, or trailing text after the object
    ('{"a":', bytes(0), "safetensors_header_json"),
    ('{} x', bytes(0), "safetensors_header_json"),
    ('[]', bytes(0), "safetensors_header"),
])
def test_safetensors_refusals(tmp_path, header, payload, code):
    path = tmp_path / "m.safetensors"
    raw_safetensors(path, header, payload)
    with pytest.raises(ReaderError, match=code):
        Safetensors(str(path))


def test_safetensors_accepts_escapes_metadata_and_empty_tensors(tmp_path):
    path = tmp_path / "m.safetensors"
    raw_safetensors(path, '{"__metadata__":{"format":"pt","note":"a\\u0041\\n"},'
                          '"x\\/y":{"dtype":"U8","shape":[4],"data_offsets":[0,4]},'
                          '"e":{"dtype":"F32","shape":[0,3],"data_offsets":[4,4]}}',
                    bytes([1, 2, 3, 4]))
    s = Safetensors(str(path))
    ident = s.identity("x/y")
    assert ident[8] - ident[7] == 4
    assert s.metadata("note") == "aA\n"
    with pytest.raises(ReaderError, match="safetensors_missing_metadata"):
        s.metadata("absent")
    s.close()


def test_readers_refuse_a_fifo_without_blocking(tmp_path):
    fifo = tmp_path / "m.safetensors"
    os.mkfifo(fifo)
    with pytest.raises(ReaderError, match="checkpoint_not_regular_file"):
        Safetensors(str(fifo))
    d = tmp_path / "g"
    d.mkdir()
    os.mkfifo(d / "m.gguf")
    with pytest.raises(ReaderError, match="gguf_not_regular_file"):
        Gguf(str(d))


def _gguf_dir(tmp_path, name, raw: bytes):
    d = tmp_path / name
    d.mkdir()
    (d / "m.gguf").write_bytes(raw)
    return str(d)


def test_gguf_header_refusals(tmp_path):
    import struct
    good = formats.gguf_bytes(metadata(), [("q8", Q8_0, [32, 1], bytes(34))])
    assert Gguf(_gguf_dir(tmp_path, "good", good)).tensor_count() == 1
    cases = {
        "gguf_magic": b"GGUG" + good[4:],
        # more pairs / tensors than the header could hold
        "gguf_header_count": good[:8] + struct.pack("<QQ", 1, 1 << 40) + good[24:],
        # an array whose element count the file cannot hold
        "gguf_array_limit": formats.gguf_bytes([("k", ARRAY, (U64, [1]))], [])
        .replace(struct.pack("<IQ", U64, 1), struct.pack("<IQ", U64, 1 << 50)),
        "gguf_duplicate_key": formats.gguf_bytes([("k", U32, 1), ("k", U32, 2)], []),
        "gguf_string_nul": formats.gguf_bytes([("k\0x", U32, 1)], []),
        "gguf_metadata_key": formats.gguf_bytes([("", U32, 1)], []),
        "gguf_metadata_type": formats.gguf_bytes([("k", U32, 1)], []).replace(
            struct.pack("<I", U32) + struct.pack("<I", 1), struct.pack("<I", 13) + struct.pack("<I", 1)),
        "gguf_invalid_metadata": formats.gguf_bytes([("k", BOOL, True)], [])[:-1] + b"\x02",
        "gguf_alignment": formats.gguf_bytes([("general.alignment", U32, 24)], []),
        "gguf_duplicate_tensor": formats.gguf_bytes([], [("t", Q8_0, [32, 1], bytes(34)),
                                                         ("t", Q8_0, [32, 1], bytes(34))]),
        "gguf_tensor_rank": formats.gguf_bytes([], [("t", Q8_0, [32, 1, 1, 1], bytes(34))]),
        "gguf_tensor_shape": formats.gguf_bytes([], [("t", Q8_0, [32, 0], b"")]),
        "gguf_tensor_bounds": formats.gguf_bytes([], [("t", Q8_0, [32, 2], bytes(34))]),
        "gguf_read_bounds": good[:200],  # ends inside the metadata
    }
    for code, raw in cases.items():
        with pytest.raises(ReaderError, match=code):
            Gguf(_gguf_dir(tmp_path, code, raw))


def test_gguf_split_set_part_missing(tmp_path):
    formats.write_gguf(tmp_path / "a-00001-of-00003.gguf", metadata(0), [])
    formats.write_gguf(tmp_path / "a-00002-of-00003.gguf", metadata(1), [])
    with pytest.raises(ReaderError, match="gguf_split_count"):
        Gguf(str(tmp_path))
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(ReaderError, match="gguf_missing_files"):
        Gguf(str(empty))


def test_gguf_metadata_kinds(tmp_path):
    formats.write_gguf(tmp_path / "m.gguf",
                       [("neg", I32, -3), ("reals", ARRAY, (F32, [0.5, -2.0])),
                        ("big", ARRAY, (U64, [2**63])), ("s", STRING, "x")], [])
    g = Gguf(str(tmp_path))
    with pytest.raises(ReaderError, match="gguf_metadata_integer"):
        g.meta("neg", 1)  # a count is never negative
    assert g.meta("reals", 6) == [0.5, -2.0]
    with pytest.raises(ReaderError, match="gguf_metadata_integers"):
        g.meta("big", 5)  # beyond int64
    with pytest.raises(ReaderError, match="gguf_metadata_numbers"):
        g.meta("big", 6)
    with pytest.raises(ReaderError, match="gguf_metadata_strings"):
        g.meta("s", 4)  # a scalar is not an array
    with pytest.raises(ReaderError, match="gguf_metadata_boolean"):
        g.meta("s", 3)
    g.close()

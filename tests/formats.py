"""Writers of the on-disk weight formats for test fixtures (GGUF v3 and safetensors), from
the formats' public specifications, plus ctypes access to the C++ readers through the
test shim (tests/cpp/dense_compute_probe.cpp)."""
from __future__ import annotations

import ctypes
import json
import os
import struct

import numpy as np

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _text(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, value) -> bytes:
    if kind == STRING:
        return _text(value)
    if kind == ARRAY:
        element, items = value
        out = struct.pack("<IQ", element, len(items))
        if element == STRING:
            return out + b"".join(_text(s) for s in items)
        return out + b"".join(struct.pack(_SCALAR[element], v) for v in items)
    return struct.pack(_SCALAR[kind], value)


def gguf_bytes(metadata, tensors, alignment: int = 32) -> bytes:
    """metadata: [(key, type, value)] (ARRAY values: (element type, items));
    tensors: [(name, ggml type, shape in GGML order, payload bytes)]."""
    out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(metadata)))
    for key, kind, value in metadata:
        out += _text(key) + struct.pack("<I", kind) + _value(kind, value)
    offset = 0
    offsets = []
    for name, kind, shape, data in tensors:
        out += _text(name) + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", kind, offset)
        offsets.append(offset)
        offset = (offset + len(data) + alignment - 1) // alignment * alignment
    if tensors:
        while len(out) % alignment:
            out.append(0)
    begin = len(out)
    for (_, _, _, data), off in zip(tensors, offsets):
        while len(out) - begin < off:
            out.append(0)
        out += data
    return bytes(out)


def write_gguf(path, metadata, tensors, alignment: int = 32):
    with open(path, "wb") as f:
        f.write(gguf_bytes(metadata, tensors, alignment))


def write_safetensors(path, tensors, metadata=None):
    """tensors: {name: (dtype string, shape, bytes)}; data in insertion order."""
    header = {}
    offset = 0
    for name, (dtype, shape, data) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape),
                        "data_offsets": [offset, offset + len(data)]}
        offset += len(data)
    if metadata:
        header["__metadata__"] = metadata
    text = json.dumps(header).encode()
    text += b" " * ((8 - len(text) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text)
        for _, _, data in tensors.values():
            f.write(data)


# ---------------------------------------------------------------- the C++ readers

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp",
                     "libdense_compute_probe.so")
_c_p, _sz, _ull = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_ulonglong


class ReaderError(RuntimeError):
    pass


def _lib():
    lib = ctypes.CDLL(PROBE)
    lib.kcp_gguf_open.restype = _c_p
    lib.kcp_gguf_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, _sz]
    lib.kcp_gguf_close.argtypes = [_c_p]
    lib.kcp_gguf_tensor_count.restype = _sz
    lib.kcp_gguf_tensor_count.argtypes = [_c_p]
    lib.kcp_gguf_tensor.argtypes = [_c_p, ctypes.c_char_p, _c_p, _c_p, _c_p, _c_p,
                                    ctypes.c_char_p, _sz]
    lib.kcp_gguf_identity.argtypes = [_c_p, ctypes.c_char_p, _sz, _c_p, ctypes.c_char_p, _sz]
    lib.kcp_gguf_check_unchanged.argtypes = [_c_p, ctypes.c_char_p, _sz]
    lib.kcp_gguf_read_packed.argtypes = [_c_p, ctypes.c_char_p, _sz, _sz, _c_p, _sz,
                                         ctypes.c_int, ctypes.c_char_p, _sz]
    lib.kcp_gguf_read_vector.argtypes = [_c_p, ctypes.c_char_p, _c_p, _sz, ctypes.c_char_p, _sz]
    lib.kcp_gguf_meta.argtypes = [_c_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p, _sz,
                                  _c_p, _c_p, _c_p, ctypes.c_char_p, _sz]
    lib.kcp_gguf_read_rows.argtypes = [_c_p, _c_p, ctypes.c_char_p, _sz, _sz, _c_p, _sz,
                                       ctypes.c_char_p, _sz]
    lib.kcp_gguf_dense_source.argtypes = [_c_p, _c_p, ctypes.c_char_p, _sz, _c_p, _sz, _c_p,
                                          _c_p, ctypes.c_char_p, _sz]
    lib.kcp_st_open.restype = _c_p
    lib.kcp_st_open.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _sz]
    lib.kcp_st_close.argtypes = [_c_p]
    lib.kcp_st_identity.argtypes = [_c_p, ctypes.c_char_p, _c_p, ctypes.c_char_p, _sz]
    lib.kcp_st_metadata.argtypes = [_c_p, ctypes.c_char_p, ctypes.c_char_p, _sz, ctypes.c_char_p,
                                    _sz]
    lib.kcp_st_load_rows.argtypes = [_c_p, ctypes.c_char_p, _sz, _sz, _sz, _sz, _c_p, _sz,
                                     _c_p, _sz, _c_p, ctypes.c_char_p, _sz]
    lib.kcp_st_moe.argtypes = [_c_p, _c_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                               _c_p, _c_p, _sz, _sz, _c_p, _c_p, _c_p, _c_p, ctypes.c_char_p,
                               _sz]
    return lib


def _p(a):
    return a.ctypes.data_as(_c_p)


class Gguf:
    """GgufFiles (include/kadan_amd_checkpoint.hpp) over a directory."""

    def __init__(self, root: str, cancelled: bool = False):
        self.lib = _lib()
        self.err = ctypes.create_string_buffer(512)
        self.h = self.lib.kcp_gguf_open(root.encode(), int(cancelled), self.err, 512)
        if not self.h:
            raise ReaderError(self.err.value.decode())

    def close(self):
        if self.h:
            self.lib.kcp_gguf_close(self.h)
            self.h = None

    def _ok(self, rc):
        if rc:
            raise ReaderError(self.err.value.decode())

    def tensor_count(self):
        return self.lib.kcp_gguf_tensor_count(self.h)

    def tensor(self, name):
        shape = np.zeros(3, np.uint64)
        rank, kind, nbytes = ctypes.c_size_t(), ctypes.c_uint(), ctypes.c_ulonglong()
        self._ok(self.lib.kcp_gguf_tensor(self.h, name.encode(), _p(shape), ctypes.byref(rank),
                                          ctypes.byref(kind), ctypes.byref(nbytes), self.err, 512))
        return tuple(int(d) for d in shape), rank.value, kind.value, nbytes.value

    def identity(self, name, expert=0):
        out = np.zeros(9, np.uint64)
        self._ok(self.lib.kcp_gguf_identity(self.h, name.encode(), expert, _p(out), self.err, 512))
        return [int(v) for v in out]

    def check_unchanged(self):
        self._ok(self.lib.kcp_gguf_check_unchanged(self.h, self.err, 512))

    def read_packed(self, name, expert, first, nbytes, cancelled=False):
        out = np.zeros(max(nbytes, 1), np.uint8)
        self._ok(self.lib.kcp_gguf_read_packed(self.h, name.encode(), expert, first, _p(out),
                                               nbytes, int(cancelled), self.err, 512))
        return out[:nbytes]

    def read_vector(self, name, n):
        out = np.zeros(n, np.float32)
        self._ok(self.lib.kcp_gguf_read_vector(self.h, name.encode(), _p(out), n, self.err, 512))
        return out

    def meta(self, key, kind):
        text = ctypes.create_string_buffer(4096)
        ints = np.zeros(64, np.int64)
        nums = np.zeros(64, np.float64)
        count = ctypes.c_size_t(64)
        self._ok(self.lib.kcp_gguf_meta(self.h, key.encode(), kind, text, 4096, _p(ints),
                                        _p(nums), ctypes.byref(count), self.err, 512))
        n = count.value
        return {0: lambda: text.value.decode(), 1: lambda: int(ints[0]),
                2: lambda: float(nums[0]), 3: lambda: bool(ints[0]),
                4: lambda: text.value.decode().split("\x1f")[:-1],
                5: lambda: [int(v) for v in ints[:n]], 6: lambda: [float(v) for v in nums[:n]],
                7: lambda: [bool(v) for v in ints[:n]], 8: lambda: bool(ints[0])}[kind]()

    def read_rows(self, probe, name, expert, first, n):
        out = np.zeros(n, np.float32)
        self._ok(self.lib.kcp_gguf_read_rows(self.h, probe.h, name.encode(), expert, first,
                                             _p(out), n, self.err, 512))
        return out

    def dense_source(self, probe, name, expert, x, n_out):
        x = np.ascontiguousarray(x, np.float32)
        y = np.full((x.shape[0], n_out), np.nan, np.float32)
        res = ctypes.c_int(-1)
        self._ok(self.lib.kcp_gguf_dense_source(self.h, probe.h, name.encode(), expert, _p(x),
                                                x.shape[0], _p(y), ctypes.byref(res), self.err,
                                                512))
        return res.value, y


class Safetensors:
    """SafetensorsFile (include/kadan_amd_checkpoint.hpp) over one file."""

    def __init__(self, path: str):
        self.lib = _lib()
        self.err = ctypes.create_string_buffer(512)
        self.h = self.lib.kcp_st_open(path.encode(), self.err, 512)
        if not self.h:
            raise ReaderError(self.err.value.decode())

    def close(self):
        if self.h:
            self.lib.kcp_st_close(self.h)
            self.h = None

    def _ok(self, rc):
        if rc:
            raise ReaderError(self.err.value.decode())

    def identity(self, name):
        out = np.zeros(9, np.uint64)
        self._ok(self.lib.kcp_st_identity(self.h, name.encode(), _p(out), self.err, 512))
        return [int(v) for v in out]

    def metadata(self, key):
        text = ctypes.create_string_buffer(4096)
        self._ok(self.lib.kcp_st_metadata(self.h, key.encode(), text, 4096, self.err, 512))
        return text.value.decode()

    def load_rows(self, prefix, expert, first, count, groups, budget=1 << 30):
        blocks = np.zeros(count * groups * 16, np.uint8)
        scales = np.zeros(count * groups, np.uint8)
        cols = ctypes.c_size_t()
        self._ok(self.lib.kcp_st_load_rows(self.h, prefix.encode(), expert, first, count, budget,
                                           _p(blocks), blocks.size, _p(scales), scales.size,
                                           ctypes.byref(cols), self.err, 512))
        return cols.value, blocks.reshape(count, groups * 16), scales.reshape(count, groups)

    def moe(self, probe, gate, up, down, x_bf16, logits, top_k, hidden):
        x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
        logits = np.ascontiguousarray(logits, np.float32)
        tokens = x_bf16.shape[0]
        y = np.full((tokens, hidden), np.nan, np.float32)
        sel = np.full((tokens, top_k), -1, np.int32)
        w = np.zeros((tokens, top_k), np.float32)
        res = ctypes.c_int(-1)
        self._ok(self.lib.kcp_st_moe(self.h, probe.h, gate.encode(), up.encode(), down.encode(),
                                     _p(x_bf16), _p(logits), tokens, top_k, _p(y), _p(sel),
                                     _p(w), ctypes.byref(res), self.err, 512))
        return res.value, y, sel, w

"""ctypes bindings for the CPU checkers.  TEST INFRASTRUCTURE ONLY.

Only tests/, tests/golden/, ``__graft_entry__.smoke()`` and bench.py's
cpu_baseline leg may import this package.  The product library
(kadan_amd/libkadan_amd.so) never loads it.

* ``Oracle``  -- liboracle.so, the plain-C restatement of the reference path
  (oracle.c; every function cites the reference file:line it follows).
* ``Reference`` -- _ref/libkadan_ref.so, the reference's own sources compiled
  from /root/reference by oracle/Makefile (absent where the reference is absent).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkadan_ref.so")
REFERENCE_ROOT = "/root/reference/services/hikari/inference_worker"

Q4_0, Q8_0, Q4_K = 2, 8, 12
Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16 = 11, 14, 20, 23, 30
IQ3_XXS, IQ3_S, IQ2_S = 18, 21, 22
BLOCK_VALUES = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q3_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256,
                BF16: 1, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q3_K: 110, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136,
               BF16: 2, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82}


def build(reference: bool | None = None) -> None:
    """Compile liboracle.so, and _ref/ when the reference sources are present."""
    subprocess.check_call(["make", "-s", "-C", HERE, "-B", "oracle"])
    if reference is None:
        reference = os.path.isdir(REFERENCE_ROOT)
    if reference:
        subprocess.check_call(["make", "-s", "-C", HERE, "-B", "ref"])


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build(reference=False)
        lib = C.CDLL(path)
        self.lib = lib
        sz, vp, i = C.c_size_t, C.c_void_p, C.c_int
        lib.kdo_half_to_float.restype = C.c_float
        lib.kdo_half_to_float.argtypes = [C.c_uint16]
        lib.kdo_float_to_half.restype = C.c_uint16
        lib.kdo_float_to_half.argtypes = [C.c_float]
        lib.kdo_dequantize_row.argtypes = [i, vp, sz, vp]
        lib.kdo_gemv.argtypes = [i, vp, sz, vp, sz, sz, sz, vp, sz]
        lib.kdo_moe_gguf_forward.argtypes = [vp, vp, sz, vp, vp, vp]
        lib.kdo_quantize_row_q8_0.argtypes = [vp, sz, vp, vp]
        lib.kdo_quantize_row_q8_K.argtypes = [vp, sz, vp, vp, vp]
        lib.kdo_quantize_q8_f16.argtypes = [vp, sz, sz, vp, vp]
        lib.kdo_cpu_matvec.argtypes = [i, vp, sz, vp, sz, sz, sz, vp, i]
        lib.kdo_gemm_q4_0_q8.argtypes = [vp, sz, sz, vp, vp, sz, vp]
        for name in ("kdo_vec_dot_q8_0_q8_0", "kdo_vec_dot_q4_0_q8_0"):
            getattr(lib, name).restype = C.c_float
            getattr(lib, name).argtypes = [sz, vp, vp, vp]
        lib.kdo_vec_dot_q4_K_q8_K.restype = C.c_float
        lib.kdo_vec_dot_q4_K_q8_K.argtypes = [sz, vp, vp, vp, vp]
        lib.kdo_e2m1.restype = C.c_float
        lib.kdo_e2m1.argtypes = [C.c_uint8]
        lib.kdo_mxfp4_decode_rows.argtypes = [vp, vp, sz, sz, vp]
        lib.kdo_mxfp4_matvec.argtypes = [vp, vp, sz, sz, vp, vp]
        lib.kdo_moe_route.argtypes = [vp, sz, sz, sz, vp, vp]
        lib.kdo_moe_permute.argtypes = [vp, sz, sz, sz, vp, vp]
        lib.kdo_moe_forward.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp,
                                        vp, vp, vp, vp, vp, i]
        lib.kdo_moe_forward_f32.argtypes = [vp, vp, sz, sz, sz, sz, sz, vp, vp, vp, vp, vp,
                                            vp, vp, i]

    # -- scalars
    def half_to_float(self, bits: int) -> float:
        return self.lib.kdo_half_to_float(bits)

    def halves_to_float(self, bits: np.ndarray) -> np.ndarray:
        """Vectorised through the Q8_0 decode of code 1 (d * 1 is exact)."""
        bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
        blocks = np.zeros((bits.size, 34), np.uint8)
        blocks[:, 0] = bits & 0xFF
        blocks[:, 1] = bits >> 8
        blocks[:, 2] = 1
        out = self.dequantize(Q8_0, blocks.reshape(1, -1), bits.size * 32)
        return out.reshape(bits.size, 32)[:, 0].copy()

    def float_to_half(self, value: float) -> int:
        return self.lib.kdo_float_to_half(value)

    # -- GGUF blocks
    def dequantize(self, encoding: int, rows: np.ndarray, n_in: int) -> np.ndarray:
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        rows2 = rows.reshape(-1, rows.shape[-1])
        out = np.empty((rows2.shape[0], n_in), np.float32)
        for r in range(rows2.shape[0]):
            rc = self.lib.kdo_dequantize_row(encoding, _p(rows2[r]), n_in, _p(out[r]))
            if rc:
                raise ValueError(f"kdo_dequantize_row rc={rc}")
        return out

    def gemv(self, encoding, weights, x, n_in, n_out):
        weights = np.ascontiguousarray(weights, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
        y = np.empty((x.shape[0], n_out), np.float32)
        row_bytes = weights.size // n_out
        rc = self.lib.kdo_gemv(encoding, _p(weights), row_bytes, _p(x), x.shape[0], n_in, n_out,
                               _p(y), n_out)
        if rc:
            raise ValueError(f"kdo_gemv rc={rc}")
        return y

    def cpu_matvec(self, encoding, weights, x, n_in, n_out, threads=1):
        weights = np.ascontiguousarray(weights, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
        y = np.empty((x.shape[0], n_out), np.float32)
        rc = self.lib.kdo_cpu_matvec(encoding, _p(weights), weights.size // n_out, _p(x),
                                     x.shape[0], n_in, n_out, _p(y), threads)
        if rc:
            raise ValueError(f"kdo_cpu_matvec rc={rc}")
        return y

    def vec_dot(self, encoding, w, qs, d, bsums=None) -> float:
        """One weight row against quantized activations (Q8_0 codes + fp16 scales for
        Q8_0/Q4_0 weights; Q8_K codes + fp32 scales + bsums for Q4_K)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        if encoding == Q4_K:
            return self.lib.kdo_vec_dot_q4_K_q8_K(qs.size, _p(w), _p(qs),
                                                  _p(np.ascontiguousarray(d, np.float32)),
                                                  _p(np.ascontiguousarray(bsums, np.int16)))
        fn = self.lib.kdo_vec_dot_q8_0_q8_0 if encoding == Q8_0 else self.lib.kdo_vec_dot_q4_0_q8_0
        return fn(qs.size, _p(w), _p(qs), _p(np.ascontiguousarray(d, np.uint16)))

    # -- activation quantizers
    def quantize_row_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        qs = np.empty(x.size, np.int8)
        d = np.empty(x.size // 32, np.uint16)
        self.lib.kdo_quantize_row_q8_0(_p(x), x.size, _p(qs), _p(d))
        return qs, d

    def quantize_row_q8_K(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        qs = np.empty(x.size, np.int8)
        d = np.empty(x.size // 256, np.float32)
        bsums = np.empty(x.size // 16, np.int16)
        self.lib.kdo_quantize_row_q8_K(_p(x), x.size, _p(qs), _p(d), _p(bsums))
        return qs, d, bsums

    def quantize_q8_f16(self, x_half: np.ndarray):
        x_half = np.ascontiguousarray(x_half, dtype=np.uint16)
        m, k = x_half.shape
        qs = np.empty((m, k), np.int8)
        d = np.empty((m, k // 32), np.float32)
        self.lib.kdo_quantize_q8_f16(_p(x_half), m, k, _p(qs), _p(d))
        return qs, d

    def gemm_q4_0_q8(self, weights, n_out, k, xq, xd):
        weights = np.ascontiguousarray(weights, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        xd = np.ascontiguousarray(xd, dtype=np.float32)
        m = xq.shape[0]
        y = np.empty((m, n_out), np.float32)
        rc = self.lib.kdo_gemm_q4_0_q8(_p(weights), n_out, k, _p(xq), _p(xd), m, _p(y))
        if rc:
            raise ValueError(f"kdo_gemm_q4_0_q8 rc={rc}")
        return y

    # -- MXFP4 / MoE
    def e2m1(self, code: int) -> float:
        return self.lib.kdo_e2m1(code)

    def mxfp4_decode_rows(self, blocks, scales, rows, cols):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.empty((rows, cols), np.float32)
        rc = self.lib.kdo_mxfp4_decode_rows(_p(blocks), _p(scales), rows, cols, _p(out))
        return rc, out

    def mxfp4_matvec(self, blocks, scales, rows, cols, x):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, np.float32)
        rc = self.lib.kdo_mxfp4_matvec(_p(blocks), _p(scales), rows, cols, _p(x), _p(y))
        return rc, y

    def moe_route(self, logits, top_k):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        t, e = logits.shape
        idx = np.empty((t, top_k), np.int32)
        w = np.empty((t, top_k), np.float32)
        self.lib.kdo_moe_route(_p(logits), t, e, top_k, _p(idx), _p(w))
        return idx, w

    def moe_permute(self, idx, experts):
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        t, k = idx.shape
        offsets = np.empty(experts + 1, np.int32)
        perm = np.empty(t * k, np.int32)
        self.lib.kdo_moe_permute(_p(idx), t, k, experts, _p(offsets), _p(perm))
        return offsets, perm

    def moe_gguf_forward(self, spec: dict, x):
        """kdo_moe_gguf_forward: (y [rows, hidden], idx, w [rows, top_k])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows = x.shape[0]
        host = dict(spec)
        for name in MOE_TENSORS:
            enc, arr = spec[name]
            host[name] = (int(enc), np.ascontiguousarray(arr, dtype=np.uint8))
        host["shared_gate"] = np.ascontiguousarray(spec["shared_gate"], dtype=np.float32)
        keep = []
        layer = moe_gguf_layer(host, lambda a: a.ctypes.data, keep)
        y = np.empty((rows, spec["hidden"]), np.float32)
        idx = np.empty((rows, spec["top_k"]), np.int32)
        w = np.empty((rows, spec["top_k"]), np.float32)
        rc = self.lib.kdo_moe_gguf_forward(C.addressof(layer), _p(x), rows, _p(y), _p(idx),
                                           _p(w))
        if rc:
            raise ValueError(f"kdo_moe_gguf_forward rc={rc}")
        return y, idx, w

    def moe_forward(self, x_bf16, logits, top_k, gate_b, gate_s, up_b, up_s, down_b, down_s,
                    threads=1):
        x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        t, h = x_bf16.shape
        e = logits.shape[1]
        inter = gate_s.shape[1]
        arrays = [np.ascontiguousarray(a, dtype=np.uint8)
                  for a in (gate_b, gate_s, up_b, up_s, down_b, down_s)]
        y = np.empty((t, h), np.float32)
        idx = np.empty((t, top_k), np.int32)
        w = np.empty((t, top_k), np.float32)
        offsets = np.empty(e + 1, np.int32)
        perm = np.empty(t * top_k, np.int32)
        rc = self.lib.kdo_moe_forward(_p(x_bf16), _p(logits), t, h, inter, e, top_k,
                                      *[_p(a) for a in arrays], _p(y), _p(idx), _p(w),
                                      _p(offsets), _p(perm), threads)
        if rc:
            raise ValueError(f"kdo_moe_forward rc={rc}")
        return y, idx, w, offsets, perm


    def moe_forward_f32(self, x_bf16, logits, top_k, gate_b, gate_s, up_b, up_s, down_b,
                        down_s, threads=1):
        """kdo_moe_forward_f32: the layer with AVX2 fp32 products (a timed CPU baseline,
        not a checker): y [tokens, hidden]."""
        x_bf16 = np.ascontiguousarray(x_bf16, dtype=np.uint16)
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        t, h = x_bf16.shape
        arrays = [np.ascontiguousarray(a, dtype=np.uint8)
                  for a in (gate_b, gate_s, up_b, up_s, down_b, down_s)]
        y = np.empty((t, h), np.float32)
        rc = self.lib.kdo_moe_forward_f32(_p(x_bf16), _p(logits), t, h, gate_s.shape[1],
                                          logits.shape[1], top_k, *[_p(a) for a in arrays],
                                          _p(y), threads)
        if rc:
            raise ValueError(f"kdo_moe_forward_f32 rc={rc}")
        return y


class GgufTensor(C.Structure):
    _fields_ = [("weights", C.c_void_p), ("row_bytes", C.c_size_t),
                ("expert_bytes", C.c_size_t), ("encoding", C.c_int)]


class MoeGgufLayer(C.Structure):
    _fields_ = [("hidden", C.c_size_t), ("experts", C.c_size_t), ("top_k", C.c_size_t),
                ("ff", C.c_size_t), ("shared_ff", C.c_size_t)] + [
        (name, GgufTensor) for name in ("router", "gate_exps", "up_exps", "down_exps",
                                        "gate_shexp", "up_shexp", "down_shexp")] + [
        ("shared_gate", C.c_void_p)]


MOE_TENSORS = ("router", "gate_exps", "up_exps", "down_exps", "gate_shexp", "up_shexp",
               "down_shexp")


def moe_gguf_layer(spec: dict, pointer, keep: list) -> MoeGgufLayer:
    """spec: hidden, experts, top_k, ff, shared_ff, shared_gate (float32 [hidden]) and per
    tensor name (encoding, uint8 array [rows, row_bytes] or [experts, rows, row_bytes]).
    `pointer(array)` gives the address to store (host or device); `keep` holds what must
    stay alive."""
    layer = MoeGgufLayer(spec["hidden"], spec["experts"], spec["top_k"], spec["ff"],
                         spec["shared_ff"])
    for name in MOE_TENSORS:
        enc, arr = spec[name]
        keep.append(arr)
        expert_bytes = arr.shape[1] * arr.shape[2] if arr.ndim == 3 else 0
        setattr(layer, name, GgufTensor(pointer(arr), arr.shape[-1], expert_bytes, enc))
    keep.append(spec["shared_gate"])
    layer.shared_gate = pointer(spec["shared_gate"])
    return layer


class Reference:
    """The reference's own compiled code (oracle/_ref).  ``available()`` first."""

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_SO)

    def __init__(self, path: str = REF_SO):
        lib = C.CDLL(path)
        self.lib = lib
        sz, vp, i = C.c_size_t, C.c_void_p, C.c_int
        lib.kdr_half_to_float.restype = C.c_float
        lib.kdr_half_to_float.argtypes = [C.c_uint16]
        lib.kdr_ggml_to_float.argtypes = [i, vp, C.c_int64, vp]
        lib.kdr_kadan_decode_block.argtypes = [i, vp, vp]
        lib.kdr_quantize_row.argtypes = [i, vp, vp, C.c_int64]
        lib.kdr_vec_dot.argtypes = [i, i, vp, vp, vp]
        lib.kdr_cpu_matvec.argtypes = [i, vp, sz, vp, sz, sz, sz, vp, i]
        lib.kdr_e2m1.restype = C.c_float
        lib.kdr_e2m1.argtypes = [C.c_uint8]
        lib.kdr_mxfp4_decode_rows.argtypes = [vp, vp, sz, sz, vp]
        lib.kdr_mxfp4_matvec.argtypes = [vp, vp, sz, sz, vp, vp]
        lib.kdr_moe_route.argtypes = [vp, sz, sz, sz, vp, vp]

    def moe_route(self, logits, top_k):
        """Routing with the C++ library's std::partial_sort (kdr_moe_route)."""
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        t, e = logits.shape
        idx = np.empty((t, top_k), np.int32)
        w = np.empty((t, top_k), np.float32)
        self.lib.kdr_moe_route(_p(logits), t, e, top_k, _p(idx), _p(w))
        return idx, w

    def half_to_float(self, bits: int) -> float:
        return self.lib.kdr_half_to_float(bits)

    def to_float(self, ggml_type: int, rows: np.ndarray, n: int) -> np.ndarray:
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        rows2 = rows.reshape(-1, rows.shape[-1])
        out = np.empty((rows2.shape[0], n), np.float32)
        for r in range(rows2.shape[0]):
            if self.lib.kdr_ggml_to_float(ggml_type, _p(rows2[r]), n, _p(out[r])):
                raise ValueError("kdr_ggml_to_float")
        return out

    def kadan_decode_block(self, ggml_type: int, block: np.ndarray) -> np.ndarray | None:
        block = np.ascontiguousarray(block, dtype=np.uint8)
        out = np.empty(BLOCK_VALUES[ggml_type], np.float32)
        if self.lib.kdr_kadan_decode_block(ggml_type, _p(block), _p(out)):
            return None
        return out

    def quantize_row(self, dot_type: int, x: np.ndarray, nbytes: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.zeros(nbytes, np.uint8)
        if self.lib.kdr_quantize_row(dot_type, _p(x), _p(y), x.size):
            raise ValueError("kdr_quantize_row")
        return y

    def vec_dot(self, ggml_type: int, n: int, w: np.ndarray, xq: np.ndarray) -> float:
        out = np.zeros(1, np.float32)
        if self.lib.kdr_vec_dot(ggml_type, n, _p(np.ascontiguousarray(w)),
                                _p(np.ascontiguousarray(xq)), _p(out)):
            raise ValueError("kdr_vec_dot")
        return float(out[0])

    def cpu_matvec(self, ggml_type, weights, x, n_in, n_out, threads=1):
        weights = np.ascontiguousarray(weights, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, n_in)
        y = np.empty((x.shape[0], n_out), np.float32)
        rc = self.lib.kdr_cpu_matvec(ggml_type, _p(weights), weights.size // n_out, _p(x),
                                     x.shape[0], n_in, n_out, _p(y), threads)
        if rc:
            raise ValueError(f"kdr_cpu_matvec rc={rc}")
        return y

    def e2m1(self, code: int) -> float:
        return self.lib.kdr_e2m1(code)

    def mxfp4_decode_rows(self, blocks, scales, rows, cols):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.empty((rows, cols), np.float32)
        rc = self.lib.kdr_mxfp4_decode_rows(_p(blocks), _p(scales), rows, cols, _p(out))
        return rc, out

    def mxfp4_matvec(self, blocks, scales, rows, cols, x):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, np.float32)
        rc = self.lib.kdr_mxfp4_matvec(_p(blocks), _p(scales), rows, cols, _p(x), _p(y))
        return rc, y

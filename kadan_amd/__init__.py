"""kadan_amd: MI355X (gfx950) quantized-weight matmul path.

Python access to the C ABI of include/kadan_amd.h (libkadan_amd.so, built in-tree by
``kadan_amd.build``).  torch provides device memory and streams only; every
computation runs in the HIP kernels of kadan_amd/csrc.  There is no CPU fallback:
if the library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os

PACKAGE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(PACKAGE, "libkadan_amd.so")
HOST_LIBRARY = os.path.join(PACKAGE, "libkadan_amd_host.so")

Q4_0, Q8_0, Q4_K = 2, 8, 12
Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16 = 11, 14, 20, 23, 30
IQ3_XXS, IQ3_S, IQ2_S = 18, 21, 22
BLOCK_VALUES = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q3_K: 256, Q6_K: 256, IQ4_NL: 32, IQ4_XS: 256,
                BF16: 1, IQ3_XXS: 256, IQ3_S: 256, IQ2_S: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q3_K: 110, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136,
               BF16: 2, IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82}

STATUS = {0: "ok", 1: "kdq_argument", 2: "kdq_projection_shape", 3: "kdq_unsupported",
          4: "kdq_alias", 5: "kdq_hip", 6: "kdq_projection_scratch", 7: "kdq_alignment"}


class KdqError(RuntimeError):
    def __init__(self, function: str, status: int, hip: str = ""):
        self.status = status
        text = STATUS.get(status, f"status {status}")
        super().__init__(f"{function}: {text}" + (f" ({hip})" if hip else ""))


class KdqUnsupported(KdqError):
    pass


class GgufTensor(C.Structure):
    """kdq_gguf_tensor (include/kadan_amd.h)."""
    _fields_ = [("weights", C.c_void_p), ("row_bytes", C.c_size_t),
                ("expert_bytes", C.c_size_t), ("encoding", C.c_int32)]


MOE_GGUF_TENSORS = ("router", "gate_exps", "up_exps", "down_exps", "gate_shexp", "up_shexp",
                    "down_shexp")


class MoeGgufPackedStacks(C.Structure):
    """kdq_moe_gguf_packed_stacks (include/kadan_amd.h)."""
    _fields_ = [(name, C.c_void_p) for name in MOE_GGUF_TENSORS[1:]] + [
        ("checked", C.c_uint)]


class MoeGgufLayer(C.Structure):
    """kdq_moe_gguf_layer (include/kadan_amd.h)."""
    _fields_ = [("hidden", C.c_size_t), ("experts", C.c_size_t), ("top_k", C.c_size_t),
                ("ff", C.c_size_t), ("shared_ff", C.c_size_t)] + [
        (name, GgufTensor) for name in MOE_GGUF_TENSORS] + [("shared_gate", C.c_void_p)]


# (name, argtypes); every entry point returns int
_SZ, _VP, _I = C.c_size_t, C.c_void_p, C.c_int
_SIGNATURES = {
    "kdq_dequantize": [_I, _VP, _SZ, _SZ, _SZ, _VP, _VP, _VP],
    "kdq_gemv": [_I, _VP, _SZ, _VP, _SZ, _SZ, _SZ, _VP, _SZ, _VP, _VP],
    "kdq_gemv_exact": [_I, _VP, _SZ, _VP, _SZ, _SZ, _SZ, _VP, _SZ, _VP, _VP],
    "kdq_gemv_batch": [_VP, _SZ, _VP],
    "kdq_gguf_pack": [_I, _VP, _SZ, _SZ, _SZ, _VP, _VP],
    "kdq_gemv_packed": [_I, _VP, _VP, _SZ, _SZ, _SZ, _VP, _SZ, _VP, _VP],
    "kdq_gemv_packed_batch": [_VP, _SZ, _VP],
    "kdq_gemm_q4_0": [_VP, _SZ, _SZ, _VP, _SZ, _VP, _VP],
    "kdq_gemm_q4_0_packed": [_VP, _SZ, _SZ, _VP, _SZ, _VP, _VP],
    "kdq_gemm_packed": [_I, _VP, _SZ, _SZ, _VP, _SZ, _VP, _VP, _VP],
    "kdq_gemm_rows": [_I, _VP, _SZ, _SZ, _SZ, _VP, _SZ, _VP, _VP, _VP],
    "kdq_moe_gguf": [_VP, _VP, _SZ, _VP, _VP, _VP, _VP, _VP],
    "kdq_moe_gguf_packed": [_VP, _VP, _VP, _SZ, _VP, _VP, _VP, _VP, _VP],
    "kdq_gguf_gemm_check": [_I, _VP, _SZ, _SZ, _VP, _VP],
    "kdq_quantize_q8": [_VP, _SZ, _SZ, _VP, _VP, _VP],
    "kdq_moe_route": [_VP, _SZ, _SZ, _SZ, _VP, _VP, _VP, _VP, _VP],
    "kdq_mxfp4_dequantize": [_VP, _VP, _SZ, _SZ, _VP, _VP, _VP],
    "kdq_moe_mxfp4": [_VP, _VP, _SZ, _SZ, _SZ, _SZ, _SZ, _VP, _VP, _VP, _VP, _VP, _VP,
                      _VP, _VP, _VP, _VP, _VP, _VP],
    "kdq_moe_mxfp4_pack": [_VP, _VP, _SZ, _SZ, _SZ, _VP, _VP],
    "kdq_moe_mxfp4_packed": [_VP, _VP, _SZ, _SZ, _SZ, _SZ, _SZ, _VP, _VP, _VP, _VP, _VP, _VP,
                             _VP, _VP, _VP],
    "kdq_moe_mxfp4_packed_noalloc": [_VP, _VP, _SZ, _SZ, _SZ, _SZ, _SZ, _VP, _VP, _VP, _VP,
                                     _VP, _VP, _VP, _VP, _VP],
    "kdq_hbm_read": [_VP, _SZ, _VP, _SZ, _I, _I, C.c_uint, _VP],
    "kdq_release_scratch": [],
}
_OTHER = {
    "kdq_status_string": (C.c_char_p, [_I]),
    "kdq_last_hip_error": (C.c_char_p, []),
    "kdq_block_values": (_SZ, [_I]),
    "kdq_block_bytes": (_SZ, [_I]),
    "kdq_row_bytes": (_SZ, [_I, _SZ]),
    "kdq_gguf_packed_bytes": (_SZ, [_I, _SZ, _SZ]),
    "kdq_gemm_rows_values": (_SZ, [_I]),
    "kdq_gemv_packed_supported": (_I, [_I, _SZ]),
    "kdq_moe_mxfp4_packed_bytes": (_SZ, [_SZ, _SZ, _SZ]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded product library.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is missing: build it with `python -m kadan_amd.build` "
                "(there is no CPU fallback)")
        handle = C.CDLL(LIBRARY)
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = C.c_int
            fn.argtypes = args
        for name, (res, args) in _OTHER.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES) + list(_OTHER)


class MatvecJob(C.Structure):
    """kdq_matvec_job of include/kadan_amd.h."""
    _fields_ = [("weights", C.c_void_p), ("input", C.c_void_p), ("output", C.c_void_p),
                ("status", C.c_void_p), ("row_bytes", C.c_size_t), ("stride", C.c_size_t),
                ("in_", C.c_uint32), ("columns", C.c_uint32), ("rows", C.c_uint32),
                ("encoding", C.c_int32)]


def check(function: str, status: int) -> None:
    if status == 0:
        return
    hip = lib().kdq_last_hip_error().decode() if status == 5 else ""
    if status == 3:
        raise KdqUnsupported(function, status, hip)
    raise KdqError(function, status, hip)


def call(function: str, *args) -> None:
    check(function, getattr(lib(), function)(*args))


def row_bytes(encoding: int, n_in: int) -> int:
    return int(lib().kdq_row_bytes(encoding, n_in))


from . import ops  # noqa: E402,F401  (torch-facing wrappers)

"""torch-facing wrappers over the C ABI (device tensors in, device tensors out).

Each function validates shapes on the host, passes raw device pointers and the
current HIP stream to the corresponding ``kdq_*`` entry point, and raises
``KdqError`` on a non-zero status.  Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes

import torch

from . import BLOCK_BYTES, BLOCK_VALUES, MatvecJob, call, lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, dtype, name: str) -> None:
    if not t.is_cuda or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous {dtype} device tensor")


def dequantize(encoding: int, packed: torch.Tensor, n_in: int,
               status: torch.Tensor | None = None) -> torch.Tensor:
    """packed: uint8 [rows, row_bytes] -> fp32 [rows, n_in] (kdq_dequantize)."""
    _need(packed, torch.uint8, "packed")
    rows = packed.shape[0]
    out = torch.empty(rows, n_in, dtype=torch.float32, device=packed.device)
    call("kdq_dequantize", encoding, packed.data_ptr(), packed.shape[1], rows, n_in,
         out.data_ptr(), _ptr(status), _stream())
    return out


def gemv(encoding: int, weights: torch.Tensor, x: torch.Tensor, n_out: int,
         out: torch.Tensor | None = None, status: torch.Tensor | None = None,
         exact: bool = False) -> torch.Tensor:
    """y[r, c] = sum_k decode(W[c, k]) x[r, k].  weights uint8 [n_out, row_bytes],
    x fp32 [rows, n_in] -> y fp32 [rows, n_out] (kdq_gemv / kdq_gemv_exact)."""
    _need(weights, torch.uint8, "weights")
    _need(x, torch.float32, "x")
    x2 = x.reshape(-1, x.shape[-1])
    rows, n_in = x2.shape
    if weights.shape[0] != n_out:
        raise ValueError("weights rows != n_out")
    if out is None:
        out = torch.empty(rows, n_out, dtype=torch.float32, device=x.device)
    fn = "kdq_gemv_exact" if exact else "kdq_gemv"
    call(fn, encoding, weights.data_ptr(), weights.shape[1], x2.data_ptr(), rows, n_in, n_out,
         out.data_ptr(), out.stride(0) if out.dim() == 2 else n_out, _ptr(status), _stream())
    return out


def gemv_batch(jobs: list[dict]) -> None:
    """One submission of several products (kdq_gemv_batch).  Each job: dict with
    encoding, weights (uint8 [columns, row_bytes]), input (fp32 [rows, in]),
    output (fp32 [rows, stride]), optional status."""
    import ctypes as C
    table = (MatvecJob * len(jobs))()
    for i, j in enumerate(jobs):
        w, x, y = j["weights"], j["input"], j["output"]
        x2 = x.reshape(-1, x.shape[-1])
        table[i] = MatvecJob(w.data_ptr(), x2.data_ptr(), y.data_ptr(),
                             _ptr(j.get("status")) or 0, w.shape[1],
                             y.stride(0) if y.dim() == 2 else w.shape[0],
                             x2.shape[1], w.shape[0], x2.shape[0], j["encoding"])
    call("kdq_gemv_batch", C.addressof(table) if jobs else None, len(jobs), _stream())


def gguf_packed_bytes(encoding: int, n_in: int, n_out: int) -> int:
    return int(lib().kdq_gguf_packed_bytes(encoding, n_in, n_out))


def gguf_pack(encoding: int, weights: torch.Tensor, n_in: int) -> torch.Tensor:
    """Row-major packed rows uint8 [n_out, row_bytes] -> the tile-packed resident form,
    uint8 [kdq_gguf_packed_bytes] (kdq_gguf_pack)."""
    _need(weights, torch.uint8, "weights")
    n_out = weights.shape[0]
    nbytes = gguf_packed_bytes(encoding, n_in, n_out)
    if not nbytes:
        raise ValueError("shape has no packed form (in % 256 != 0)")
    out = torch.empty(nbytes, dtype=torch.uint8, device=weights.device)
    call("kdq_gguf_pack", encoding, weights.data_ptr(), weights.shape[1], n_in, n_out,
         out.data_ptr(), _stream())
    return out


def gemv_packed(encoding: int, packed: torch.Tensor, x: torch.Tensor, n_out: int,
                out: torch.Tensor | None = None,
                status: torch.Tensor | None = None) -> torch.Tensor:
    """gemv over tile-packed weights (kdq_gemv_packed)."""
    _need(packed, torch.uint8, "packed")
    _need(x, torch.float32, "x")
    x2 = x.reshape(-1, x.shape[-1])
    rows, n_in = x2.shape
    if packed.numel() != gguf_packed_bytes(encoding, n_in, n_out):
        raise ValueError("packed size does not match (encoding, n_in, n_out)")
    if out is None:
        out = torch.empty(rows, n_out, dtype=torch.float32, device=x.device)
    call("kdq_gemv_packed", encoding, packed.data_ptr(), x2.data_ptr(), rows, n_in, n_out,
         out.data_ptr(), out.stride(0) if out.dim() == 2 else n_out, _ptr(status), _stream())
    return out


def gemv_packed_batch(jobs: list[dict]) -> None:
    """One submission over packed weights (kdq_gemv_packed_batch).  Each job: dict with
    encoding, weights (packed uint8), columns, input (fp32 [rows, in]), output
    (fp32 [rows, stride]), optional status."""
    import ctypes as C
    table = (MatvecJob * len(jobs))()
    for i, j in enumerate(jobs):
        w, x, y = j["weights"], j["input"], j["output"]
        x2 = x.reshape(-1, x.shape[-1])
        table[i] = MatvecJob(w.data_ptr(), x2.data_ptr(), y.data_ptr(),
                             _ptr(j.get("status")) or 0, 0,
                             y.stride(0) if y.dim() == 2 else j["columns"],
                             x2.shape[1], j["columns"], x2.shape[0], j["encoding"])
    call("kdq_gemv_packed_batch", C.addressof(table) if jobs else None, len(jobs), _stream())


def quantize_q8(x_f16: torch.Tensor):
    """fp16 [m, k] -> (int8 [m, k], fp32 [m, k/32]) (kdq_quantize_q8)."""
    _need(x_f16, torch.float16, "x")
    m, k = x_f16.shape
    q = torch.empty(m, k, dtype=torch.int8, device=x_f16.device)
    d = torch.empty(m, k // 32, dtype=torch.float32, device=x_f16.device)
    call("kdq_quantize_q8", x_f16.data_ptr(), m, k, q.data_ptr(), d.data_ptr(), _stream())
    return q, d


def gemm_q4_0(weights: torch.Tensor, x_f16: torch.Tensor, n_out: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """Q4_0 weights uint8 [n_out, k/32*18] x fp16 [m, k] -> fp16 [m, n_out] (kdq_gemm_q4_0)."""
    _need(weights, torch.uint8, "weights")
    _need(x_f16, torch.float16, "x")
    m, k = x_f16.shape
    if out is None:
        out = torch.empty(m, n_out, dtype=torch.float16, device=x_f16.device)
    call("kdq_gemm_q4_0", weights.data_ptr(), n_out, k, x_f16.data_ptr(), m, out.data_ptr(),
         _stream())
    return out


def gemm_q4_0_packed(packed: torch.Tensor, x_f16: torch.Tensor, n_out: int,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Tile-packed Q4_0 weights (gguf_pack) x fp16 [m, k] -> fp16 [m, n_out]
    (kdq_gemm_q4_0_packed)."""
    _need(packed, torch.uint8, "packed")
    _need(x_f16, torch.float16, "x")
    m, k = x_f16.shape
    if packed.numel() != gguf_packed_bytes(2, k, n_out):  # KDQ_Q4_0
        raise ValueError("packed size does not match (k, n_out)")
    if out is None:
        out = torch.empty(m, n_out, dtype=torch.float16, device=x_f16.device)
    call("kdq_gemm_q4_0_packed", packed.data_ptr(), n_out, k, x_f16.data_ptr(), m,
         out.data_ptr(), _stream())
    return out


def gemm_packed(encoding: int, packed: torch.Tensor, x: torch.Tensor, n_out: int,
                out: torch.Tensor | None = None,
                status: torch.Tensor | None = None) -> torch.Tensor:
    """Tile-packed Q4_K / Q8_0 / Q6_K weights (gguf_pack) x fp32 [m, k] -> fp32 [m, n_out]
    (kdq_gemm_packed, the prefill product)."""
    _need(packed, torch.uint8, "packed")
    _need(x, torch.float32, "x")
    m, k = x.shape
    if packed.numel() != gguf_packed_bytes(encoding, k, n_out):
        raise ValueError("packed size does not match (k, n_out)")
    if out is None:
        out = torch.empty(m, n_out, dtype=torch.float32, device=x.device)
    call("kdq_gemm_packed", encoding, packed.data_ptr(), n_out, k, x.data_ptr(), m,
         out.data_ptr(), _ptr(status), _stream())
    return out


def gemm_rows(encoding: int, w: torch.Tensor, x: torch.Tensor, n_out: int,
              out: torch.Tensor | None = None,
              status: torch.Tensor | None = None) -> torch.Tensor:
    """Row-major GGUF rows [n_out, row_bytes] (uint8, as the file holds them) x fp32
    [m, k] -> fp32 [m, n_out] (kdq_gemm_rows, the prefill product of every encoding)."""
    _need(w, torch.uint8, "w")
    _need(x, torch.float32, "x")
    m, k = x.shape
    if w.dim() != 2 or w.shape[0] != n_out:
        raise ValueError("w must be [n_out, row_bytes]")
    if out is None:
        out = torch.empty(m, n_out, dtype=torch.float32, device=x.device)
    call("kdq_gemm_rows", encoding, w.data_ptr(), w.shape[1], n_out, k, x.data_ptr(), m,
         out.data_ptr(), _ptr(status), _stream())
    return out


def gguf_gemm_check(encoding: int, packed: torch.Tensor, n_out: int, n_in: int) -> int:
    """The prefill GEMM's scale checks over a tile-packed matrix (kdq_gguf_gemm_check):
    bit 1 a non-finite scale, bit 2 a dequantised weight that could pass the fp16 range
    (waits for the device)."""
    flags = torch.zeros(1, dtype=torch.int32, device=packed.device)
    call("kdq_gguf_gemm_check", encoding, packed.data_ptr(), n_out, n_in, flags.data_ptr(),
         _stream())
    return int(flags.item())


def moe_gguf_pack(spec: dict) -> dict:
    """Tile-packed copies (kdq_gguf_pack) of a GGUF MoE spec's expert stacks and shared
    matrices, for moe_gguf(..., packed=...): name -> uint8 device tensor, for the
    encodings the prefill GEMM reads packed (Q4_K, Q8_0, Q6_K), and "checked": every copy
    passed kdq_gguf_gemm_check with no flag."""
    from . import MOE_GGUF_TENSORS
    H, F, S = spec["hidden"], spec["ff"], spec["shared_ff"]
    shape = {"gate_exps": (H, F), "up_exps": (H, F), "down_exps": (F, H),
             "gate_shexp": (H, S), "up_shexp": (H, S), "down_shexp": (S, H)}
    out = {}
    for name in MOE_GGUF_TENSORS[1:]:
        enc, t = spec[name]
        if enc not in (12, 8, 14):  # Q4_K, Q8_0, Q6_K
            continue
        n_in, rows = shape[name]
        count = rows * (t.shape[0] if t.dim() == 3 else 1)
        out[name] = gguf_pack(enc, t.reshape(count, t.shape[-1]), n_in)
    out["checked"] = all(gguf_gemm_check(spec[n][0], out[n], shape[n][1] * (
        spec[n][1].shape[0] if spec[n][1].dim() == 3 else 1), shape[n][0]) == 0
        for n in list(out))
    return out


def moe_gguf(spec: dict, x: torch.Tensor, status: torch.Tensor | None = None,
             packed: dict | None = None):
    """GGUF MoE layer (kdq_moe_gguf; kdq_moe_gguf_packed when `packed` holds resident
    tile-packed copies from moe_gguf_pack).  spec: hidden, experts, top_k, ff, shared_ff,
    shared_gate (fp32 device tensor [hidden]) and per tensor name (encoding, uint8 device
    tensor [rows, row_bytes] or [experts, rows, row_bytes]).  x fp32 [rows, hidden] ->
    (y fp32 [rows, hidden], selected int32 [rows, top_k], weights fp32 [rows, top_k])."""
    from . import MOE_GGUF_TENSORS, GgufTensor, MoeGgufLayer, MoeGgufPackedStacks
    _need(x, torch.float32, "x")
    layer = MoeGgufLayer(spec["hidden"], spec["experts"], spec["top_k"], spec["ff"],
                         spec["shared_ff"])
    for name in MOE_GGUF_TENSORS:
        enc, t = spec[name]
        _need(t, torch.uint8, name)
        expert_bytes = t.shape[1] * t.shape[2] if t.dim() == 3 else 0
        setattr(layer, name, GgufTensor(t.data_ptr(), t.shape[-1], expert_bytes, enc))
    _need(spec["shared_gate"], torch.float32, "shared_gate")
    layer.shared_gate = spec["shared_gate"].data_ptr()
    rows = x.shape[0]
    y = torch.empty(rows, spec["hidden"], dtype=torch.float32, device=x.device)
    sel = torch.empty(rows, spec["top_k"], dtype=torch.int32, device=x.device)
    w = torch.empty(rows, spec["top_k"], dtype=torch.float32, device=x.device)
    if packed is None:
        call("kdq_moe_gguf", ctypes.addressof(layer), x.data_ptr(), rows, y.data_ptr(),
             sel.data_ptr(), w.data_ptr(), _ptr(status), _stream())
    else:
        stacks = MoeGgufPackedStacks(*[packed[n].data_ptr() if n in packed else None
                                       for n in MOE_GGUF_TENSORS[1:]],
                                     int(bool(packed.get("checked", False))))
        call("kdq_moe_gguf_packed", ctypes.addressof(layer), ctypes.addressof(stacks),
             x.data_ptr(), rows, y.data_ptr(), sel.data_ptr(), w.data_ptr(), _ptr(status),
             _stream())
    return y, sel, w


def moe_route(logits: torch.Tensor, top_k: int):
    """fp32 [tokens, experts] -> idx, w, offsets, perm (kdq_moe_route)."""
    _need(logits, torch.float32, "logits")
    t, e = logits.shape
    dev = logits.device
    idx = torch.empty(t, top_k, dtype=torch.int32, device=dev)
    w = torch.empty(t, top_k, dtype=torch.float32, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(t * top_k, dtype=torch.int32, device=dev)
    call("kdq_moe_route", logits.data_ptr(), t, e, top_k, idx.data_ptr(), w.data_ptr(),
         offsets.data_ptr(), perm.data_ptr(), _stream())
    return idx, w, offsets, perm


def mxfp4_dequantize(blocks: torch.Tensor, scales: torch.Tensor, rows: int, cols: int,
                     status: torch.Tensor | None = None) -> torch.Tensor:
    _need(blocks, torch.uint8, "blocks")
    _need(scales, torch.uint8, "scales")
    out = torch.empty(rows, cols, dtype=torch.float32, device=blocks.device)
    call("kdq_mxfp4_dequantize", blocks.data_ptr(), scales.data_ptr(), rows, cols,
         out.data_ptr(), _ptr(status), _stream())
    return out


def moe_mxfp4(x_bf16: torch.Tensor, logits: torch.Tensor, top_k: int, gate_blocks, gate_scales,
              up_blocks, up_scales, down_blocks, down_scales, routing: bool = False,
              out: torch.Tensor | None = None):
    """The MXFP4 MoE layer (kdq_moe_mxfp4).  Returns y fp32 [tokens, hidden], plus
    (idx, w, offsets, perm) when ``routing``."""
    _need(x_bf16, torch.bfloat16, "x")
    _need(logits, torch.float32, "logits")
    t, h = x_bf16.shape
    e = logits.shape[1]
    inter = gate_scales.shape[1]
    dev = x_bf16.device
    for name, a in (("gate_blocks", gate_blocks), ("gate_scales", gate_scales),
                    ("up_blocks", up_blocks), ("up_scales", up_scales),
                    ("down_blocks", down_blocks), ("down_scales", down_scales)):
        _need(a, torch.uint8, name)
    if out is None:
        out = torch.empty(t, h, dtype=torch.float32, device=dev)
    extra = [None] * 4
    if routing:
        extra = [torch.empty(t, top_k, dtype=torch.int32, device=dev),
                 torch.empty(t, top_k, dtype=torch.float32, device=dev),
                 torch.empty(e + 1, dtype=torch.int32, device=dev),
                 torch.empty(t * top_k, dtype=torch.int32, device=dev)]
    call("kdq_moe_mxfp4", x_bf16.data_ptr(), logits.data_ptr(), t, h, inter, e, top_k,
         gate_blocks.data_ptr(), gate_scales.data_ptr(), up_blocks.data_ptr(),
         up_scales.data_ptr(), down_blocks.data_ptr(), down_scales.data_ptr(), out.data_ptr(),
         *[_ptr(a) for a in extra], _stream())
    return (out, *extra) if routing else out


def moe_mxfp4_pack(blocks: torch.Tensor, scales: torch.Tensor, experts: int, rows: int,
                   cols: int) -> torch.Tensor:
    """One projection tensor in the packed resident layout (kdq_moe_mxfp4_pack)."""
    _need(blocks, torch.uint8, "blocks")
    _need(scales, torch.uint8, "scales")
    n = lib().kdq_moe_mxfp4_packed_bytes(experts, rows, cols)
    if not n:
        raise ValueError("rows % 32 and cols % 64 must be 0")
    packed = torch.empty(n, dtype=torch.uint8, device=blocks.device)
    call("kdq_moe_mxfp4_pack", blocks.data_ptr(), scales.data_ptr(), experts, rows, cols,
         packed.data_ptr(), _stream())
    return packed


def moe_mxfp4_packed(x_bf16: torch.Tensor, logits: torch.Tensor, top_k: int, inter: int,
                     gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor,
                     routing: bool = False, out: torch.Tensor | None = None):
    """kdq_moe_mxfp4_packed: the layer over packed weights (moe_mxfp4_pack)."""
    _need(x_bf16, torch.bfloat16, "x")
    _need(logits, torch.float32, "logits")
    t, h = x_bf16.shape
    e = logits.shape[1]
    dev = x_bf16.device
    for name, a in (("gate", gate), ("up", up), ("down", down)):
        _need(a, torch.uint8, name)
    if out is None:
        out = torch.empty(t, h, dtype=torch.float32, device=dev)
    extra = [None] * 4
    if routing:
        extra = [torch.empty(t, top_k, dtype=torch.int32, device=dev),
                 torch.empty(t, top_k, dtype=torch.float32, device=dev),
                 torch.empty(e + 1, dtype=torch.int32, device=dev),
                 torch.empty(t * top_k, dtype=torch.int32, device=dev)]
    call("kdq_moe_mxfp4_packed", x_bf16.data_ptr(), logits.data_ptr(), t, h, inter, e, top_k,
         gate.data_ptr(), up.data_ptr(), down.data_ptr(), out.data_ptr(),
         *[_ptr(a) for a in extra], _stream())
    return (out, *extra) if routing else out


def hbm_read(buffer: torch.Tensor, sink: torch.Tensor, workgroups: int,
             threads: int = 256, store_all: bool = True, match: int = 0) -> None:
    """kdq_hbm_read: one streaming read of `buffer` (the HBM read ceiling's probe) over
    `workgroups` workgroups of `threads` lanes; `sink` holds one int32 per workgroup,
    written always (store_all) or where the workgroup's fold equals `match`."""
    _need(sink, torch.int32, "sink")
    if not buffer.is_cuda or not buffer.is_contiguous() or sink.numel() < workgroups:
        raise ValueError("hbm_read: a contiguous device buffer and a sink per workgroup")
    call("kdq_hbm_read", buffer.data_ptr(), buffer.numel() * buffer.element_size(),
         sink.data_ptr(), workgroups, threads, int(store_all), match & 0xFFFFFFFF, _stream())


__all__ = ["dequantize", "gemv", "gemv_batch", "quantize_q8", "gemm_q4_0", "gemm_q4_0_packed",
           "gemm_packed", "hbm_read",
           "moe_gguf", "moe_route",
           "mxfp4_dequantize", "moe_mxfp4", "moe_mxfp4_pack", "moe_mxfp4_packed", "lib",
           "BLOCK_BYTES", "BLOCK_VALUES"]

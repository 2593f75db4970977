"""Seeded synthetic inputs of the benchmark configurations (stored bits are the ground
truth: every consumer -- HIP path, oracle, bench -- reads the same arrays).

Generator: SplitMix64 over a per-tensor stream (seed, tensor id); uniform values from
the top 53 bits; N(0,1) by Box-Muller; fp16/bf16 by round-to-nearest-even from fp32.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, tensor: int, n: int) -> np.ndarray:
    """n 64-bit outputs of SplitMix64 started at hash(seed, tensor)."""
    base = np.uint64((seed * 0x100000001B3 + tensor * 0x9E3779B1) & 0xFFFFFFFFFFFFFFFF)
    out = np.empty(n, np.uint64)
    chunk = 1 << 18  # cache-sized pieces, updated in place
    t = np.empty(chunk, np.uint64)
    with np.errstate(over="ignore"):
        for start in range(0, n, chunk):
            z = out[start:start + chunk]
            w = t[:z.size]
            z[:] = np.arange(start + 1, start + z.size + 1, dtype=np.uint64)
            np.multiply(z, _GOLDEN, out=z)
            np.add(z, base, out=z)
            for shift, mul in ((30, _M1), (27, _M2)):
                np.right_shift(z, np.uint64(shift), out=w)
                np.bitwise_xor(z, w, out=z)
                np.multiply(z, mul, out=z)
            np.right_shift(z, np.uint64(31), out=w)
            np.bitwise_xor(z, w, out=z)
    return out


def uniform(seed: int, tensor: int, n: int) -> np.ndarray:
    """float64 in [0, 1)."""
    return (splitmix64(seed, tensor, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, tensor: int, n: int) -> np.ndarray:
    """float32 N(0,1) by Box-Muller."""
    m = (n + 1) // 2
    u = uniform(seed, tensor, 2 * m)
    u1 = 1.0 - u[:m]  # (0, 1]
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u[m:]
    z = np.concatenate([r * np.cos(t), r * np.sin(t)])[:n]
    return z.astype(np.float32)


def random_bytes(seed: int, tensor: int, n: int) -> np.ndarray:
    return splitmix64(seed, tensor, (n + 7) // 8).view(np.uint8)[:n].copy()


def to_half_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))
    return (b >> np.uint64(16)).astype(np.uint16)


def bf16_bits_to_float(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- GGUF weights

def q8_0_weights(seed: int, n_out: int, n_in: int, scale: float = 0.01) -> np.ndarray:
    """[n_out, n_in/32*34]: int8 codes uniform in [-127, 127], d = fp16(|N|*scale)."""
    nb = n_in // 32
    blocks = np.empty((n_out, nb, 34), np.uint8)
    codes = (splitmix64(seed, 1, n_out * nb * 32) % np.uint64(255)).astype(np.int16) - 127
    blocks[:, :, 2:] = codes.astype(np.int8).view(np.uint8).reshape(n_out, nb, 32)
    d = to_half_bits(np.abs(normal(seed, 2, n_out * nb)) * scale).reshape(n_out, nb)
    blocks[:, :, 0] = d & 0xFF
    blocks[:, :, 1] = d >> 8
    return blocks.reshape(n_out, nb * 34)


def q4_0_weights(seed: int, n_out: int, n_in: int, scale: float = 0.02) -> np.ndarray:
    """[n_out, n_in/32*18]: uniform nibbles, d = fp16(|N|*scale)."""
    nb = n_in // 32
    blocks = np.empty((n_out, nb, 18), np.uint8)
    blocks[:, :, 2:] = random_bytes(seed, 1, n_out * nb * 16).reshape(n_out, nb, 16)
    d = to_half_bits(np.abs(normal(seed, 2, n_out * nb)) * scale).reshape(n_out, nb)
    blocks[:, :, 0] = d & 0xFF
    blocks[:, :, 1] = d >> 8
    return blocks.reshape(n_out, nb * 18)


def q4_k_weights(seed: int, n_out: int, n_in: int, scale: float = 0.005) -> np.ndarray:
    """[n_out, n_in/256*144]: uniform scale bytes (every 6-bit sc/m uniform) and nibbles,
    d, dmin = fp16(|N|*scale)."""
    nb = n_in // 256
    blocks = random_bytes(seed, 1, n_out * nb * 144).reshape(n_out, nb, 144)
    d = to_half_bits(np.abs(normal(seed, 2, n_out * nb)) * scale).reshape(n_out, nb)
    dmin = to_half_bits(np.abs(normal(seed, 3, n_out * nb)) * scale).reshape(n_out, nb)
    blocks[:, :, 0] = d & 0xFF
    blocks[:, :, 1] = d >> 8
    blocks[:, :, 2] = dmin & 0xFF
    blocks[:, :, 3] = dmin >> 8
    return blocks.reshape(n_out, nb * 144)


# (block values, block bytes, byte offset of the fp16 block scale, scale magnitude) of
# the formats whose code bytes may be uniform random: every code, sub-block scale and
# high-bit byte is then a valid encoding
_RANDOM_CODE_FORMATS = {11: (256, 110, 108, 0.005),   # Q3_K
                        14: (256, 210, 208, 0.0005),  # Q6_K
                        20: (32, 18, 0, 0.0005),      # IQ4_NL
                        23: (256, 136, 0, 0.0002),    # IQ4_XS
                        18: (256, 98, 0, 0.0001),     # IQ3_XXS
                        22: (256, 82, 0, 0.0002),     # IQ2_S
                        21: (256, 110, 0, 0.0001)}    # IQ3_S


def random_code_weights(encoding: int, seed: int, n_out: int, n_in: int) -> np.ndarray:
    """[n_out, n_in/values*bytes]: uniform code and scale bytes, the fp16 block scale
    d = fp16(|N|*scale) (Q3_K, Q6_K, IQ4_NL, IQ4_XS, IQ3_XXS, IQ2_S, IQ3_S)."""
    values, nbytes, at, scale = _RANDOM_CODE_FORMATS[encoding]
    nb = n_in // values
    blocks = random_bytes(seed, 1, n_out * nb * nbytes).reshape(n_out, nb, nbytes)
    d = to_half_bits(np.abs(normal(seed, 2, n_out * nb)) * scale).reshape(n_out, nb)
    blocks[:, :, at] = d & 0xFF
    blocks[:, :, at + 1] = d >> 8
    return blocks.reshape(n_out, nb * nbytes)


def bf16_weights(seed: int, n_out: int, n_in: int, scale: float = 0.02) -> np.ndarray:
    """[n_out, 2*n_in]: bf16 bits of N(0,1)*scale."""
    b = to_bf16_bits(normal(seed, 1, n_out * n_in) * scale)
    return b.view(np.uint8).reshape(n_out, 2 * n_in)


def gguf_weights(encoding: int, seed: int, n_out: int, n_in: int) -> np.ndarray:
    if encoding == 8:
        return q8_0_weights(seed, n_out, n_in)
    if encoding == 2:
        return q4_0_weights(seed, n_out, n_in)
    if encoding == 12:
        return q4_k_weights(seed, n_out, n_in)
    if encoding == 30:
        return bf16_weights(seed, n_out, n_in)
    if encoding in _RANDOM_CODE_FORMATS:
        return random_code_weights(encoding, seed, n_out, n_in)
    raise ValueError(encoding)


# ---------------------------------------------------------------- MXFP4 MoE

def mxfp4_weights(seed: int, tensor: int, experts: int, rows: int, cols: int,
                  exp_lo: int = -8, exp_hi: int = 0):
    """GPT-OSS layout: blocks u8 [experts, rows, cols/2] (uniform nibbles), scales u8
    [experts, rows, cols/32] = 127 + U{exp_lo..exp_hi}."""
    blocks = random_bytes(seed, 2 * tensor, experts * rows * cols // 2)
    span = exp_hi - exp_lo + 1
    e = (splitmix64(seed, 2 * tensor + 1, experts * rows * cols // 32) % np.uint64(span))
    scales = (e.astype(np.int32) + 127 + exp_lo).astype(np.uint8)
    return blocks.reshape(experts, rows, cols // 2), scales.reshape(experts, rows, cols // 32)


def moe_inputs(seed: int, tokens: int, hidden: int, experts: int, hot: int = 0,
               hot_boost: float = 3.0):
    """x bf16 bits [tokens, hidden] ~ N(0,1); logits fp32 [tokens, experts] ~ N(0,1).
    With hot > 0, tokens t % 4 == 0 get +hot_boost on `hot` seeded experts."""
    x = to_bf16_bits(normal(seed, 100, tokens * hidden)).reshape(tokens, hidden)
    logits = normal(seed, 101, tokens * experts).reshape(tokens, experts)
    if hot:
        order = np.argsort(splitmix64(seed, 102, experts), kind="stable")
        hot_experts = np.sort(order[:hot])
        logits[0::4, hot_experts] += np.float32(hot_boost)
    return x, logits


def moe_weights(seed: int, experts: int, hidden: int, inter: int):
    gate = mxfp4_weights(seed, 10, experts, inter, hidden)
    up = mxfp4_weights(seed, 11, experts, inter, hidden)
    down = mxfp4_weights(seed, 12, experts, hidden, inter)
    return gate, up, down


# ------------------------------------------- the same streams generated by torch

def _mask(bits: int) -> int:
    """(1 << bits) - 1 as a signed 64-bit value."""
    return (1 << bits) - 1 if bits < 64 else -1


def _signed(v: int) -> int:
    v &= 0xFFFFFFFFFFFFFFFF
    return v - (1 << 64) if v >> 63 else v


def splitmix64_torch(seed: int, tensor: int, n: int, device):
    """splitmix64(seed, tensor, n) as a torch int64 tensor on `device`, bit for bit:
    two's-complement int64 addition, multiplication and xor wrap exactly as uint64 does,
    and logical right shifts are arithmetic shifts masked to the kept bits."""
    import torch
    base = (seed * 0x100000001B3 + tensor * 0x9E3779B1) & 0xFFFFFFFFFFFFFFFF
    out = torch.empty(n, dtype=torch.int64, device=device)
    chunk = 1 << 26
    golden, m1, m2 = (_signed(int(v)) for v in (_GOLDEN, _M1, _M2))
    for start in range(0, n, chunk):
        i = torch.arange(start + 1, min(n, start + chunk) + 1, dtype=torch.int64, device=device)
        z = i * golden + _signed(base)
        z = (z ^ ((z >> 30) & _mask(34))) * m1
        z = (z ^ ((z >> 27) & _mask(37))) * m2
        out[start:start + i.numel()] = z ^ ((z >> 31) & _mask(33))
    return out


def _umod_small(v, m: int):
    """v mod m for int64 tensors holding uint64 bits, m < 2^31."""
    hi = (v >> 32) & _mask(32)
    lo = v & _mask(32)
    return ((hi % m) * ((1 << 32) % m) + lo % m) % m


def mxfp4_weights_torch(seed: int, tensor: int, experts: int, rows: int, cols: int, device,
                        exp_lo: int = -8, exp_hi: int = 0):
    """mxfp4_weights as uint8 torch tensors on `device` (the same bytes)."""
    import torch
    n = experts * rows * cols // 2
    blocks = splitmix64_torch(seed, 2 * tensor, (n + 7) // 8, device).view(torch.uint8)[:n]
    e = _umod_small(splitmix64_torch(seed, 2 * tensor + 1, experts * rows * cols // 32,
                                     device), exp_hi - exp_lo + 1)
    scales = (e + 127 + exp_lo).to(torch.uint8)
    return (blocks.reshape(experts, rows, cols // 2).clone(),
            scales.reshape(experts, rows, cols // 32))


def moe_weights_torch(seed: int, experts: int, hidden: int, inter: int, device):
    """moe_weights as device tensors, bit-identical, generated on the device."""
    gate = mxfp4_weights_torch(seed, 10, experts, inter, hidden, device)
    up = mxfp4_weights_torch(seed, 11, experts, inter, hidden, device)
    down = mxfp4_weights_torch(seed, 12, experts, hidden, inter, device)
    return gate, up, down

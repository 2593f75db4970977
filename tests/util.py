"""Comparison helpers and hand-derived cases shared by the parity tests."""
import json
import math
import os

import numpy as np

# Tolerances of the quantized matmul path for fp32-accumulated outputs (rel-L2, and
# max-abs after normalising by the reference output RMS).
REL_L2 = 1e-3
MAX_ABS = 2e-2


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    denom = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (denom if denom else 1.0))


def normalized_max_abs(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    return float(np.max(np.abs(a - e)) / (rms if rms else 1.0)) if e.size else 0.0


def assert_close(actual, expected, rel=REL_L2, mabs=MAX_ABS, what=""):
    r = rel_l2(actual, expected)
    m = normalized_max_abs(actual, expected)
    log = os.environ.get("KDQ_PARITY_LOG")
    if log and what:  # measured margins, one JSON line per comparison
        with open(log, "a") as f:
            f.write(json.dumps({"what": what, "rel_l2": r, "max_abs_over_rms": m}) + "\n")
    assert r <= rel and m <= mabs, f"{what}: rel_l2={r:.3e} (<= {rel}) max_abs/rms={m:.3e} (<= {mabs})"
    return r, m


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32).view(np.uint32)
    b = np.ascontiguousarray(b, np.float32).view(np.uint32)
    return a.shape == b.shape and bool(np.array_equal(a, b))


def known_answer_moe():
    """An MXFP4 MoE layer (2 tokens, 4 experts, top-2, hidden = inter = 64) whose output
    follows in closed form from MoeLayer::forward's definition (IW/src/models/text/
    qwen_layers.cpp:378-492), computed here in float64 without any of the oracle's code:

      gate_e = 2^-e * ones;  up_e[n, c] = 2^(e % 2) for c < 32, else 0;
      down_e[d, c] = 2^-(1 + e // 2) * q(d), q(d) = E2M1 value of code 1 + d % 7;
      x_t[c] = v_t for c < 32, 2 v_t after (v = 1/16, -1/32, exact in bf16);
      g = 96 v 2^-e,  u = 32 v 2^(e % 2),  h = silu(g) u,  down_d = 64 2^-(1+e//2) q(d) h,
      y_t[d] = sum_i w_i down_{e_i, d},  w = p / sum of the two chosen p.

    Logits [2, 1, 0, -inf] choose experts 0, 1; [-1, 3, 0.5, 2] choose 1, 3.  A dropped
    silu, swapped gate/up, a transposed down or a misplaced routing weight each change y.
    Returns (x bf16 bits, logits, (gate, up, down) as (blocks, scales), y, idx)."""
    H = I = 64
    E = 4
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    gate_b = np.full((E, I, H // 2), 0x22, np.uint8)
    gate_s = np.array([[[127 - e] * (H // 32)] * I for e in range(E)], np.uint8)
    up_b = np.zeros((E, I, H // 2), np.uint8)
    up_b[:, :, :16] = 0x22
    up_s = np.array([[[127 + e % 2, 127]] * I for e in range(E)], np.uint8)
    codes = np.array([1 + d % 7 for d in range(H)], np.uint8)
    down_b = np.broadcast_to((codes | (codes << 4))[None, :, None], (E, H, I // 2)).copy()
    down_s = np.array([[[126 - e // 2] * (I // 32)] * H for e in range(E)], np.uint8)
    v = [1.0 / 16, -1.0 / 32]
    x = np.zeros((2, H), np.float32)
    for t in range(2):
        x[t, :32], x[t, 32:] = v[t], 2 * v[t]
    x_bits = (x.view(np.uint32) >> 16).astype(np.uint16)  # exact: bf16 keeps these
    logits = np.array([[2, 1, 0, -np.inf], [-1, 3, 0.5, 2]], np.float32)
    idx = np.array([[0, 1], [1, 3]], np.int32)
    y = np.zeros((2, H), np.float64)
    for t in range(2):
        top = max(float(l) for l in logits[t])
        p = [math.exp(float(l) - top) for l in logits[t]]
        p = [q / sum(p) for q in p]
        chosen = [p[e] for e in idx[t]]
        for i, e in enumerate(idx[t]):
            g = 96 * v[t] * 2.0 ** -e
            u = 32 * v[t] * 2.0 ** (e % 2)
            h = g / (1 + math.exp(-g)) * u
            for d in range(H):
                down = 64 * 2.0 ** -(1 + e // 2) * e2m1[1 + d % 7] * h
                y[t, d] += chosen[i] / sum(chosen) * down
    return x_bits, logits, ((gate_b, gate_s), (up_b, up_s), (down_b, down_s)), y, idx


def _q8_0_rows(rows, cols, d_of_row, q_of):
    """Q8_0 rows [rows, cols]: per row fp16 d = d_of_row(r) (a power of two) and codes
    q_of(r, c) (int8), blocks of 32 as [d:fp16][qs:int8 x 32]."""
    out = np.zeros((rows, cols // 32 * 34), np.uint8)
    for r in range(rows):
        d = np.float16(d_of_row(r)).view(np.uint16)
        for b in range(cols // 32):
            out[r, 34 * b] = d & 255
            out[r, 34 * b + 1] = d >> 8
            out[r, 34 * b + 2:34 * b + 34] = [np.int8(q_of(r, 32 * b + i)).view(np.uint8)
                                              for i in range(32)]
    return out


def known_answer_moe_gguf():
    """A GGUF MoE layer with a shared expert (2 tokens, hidden 64, 4 experts, top-2,
    expert ff 32, shared ff 32; every matrix Q8_0, the router F32) whose output follows
    in closed form from MoeLayer::forward's definition (IW/src/models/text/
    qwen_layers.cpp:378-492), computed here in float64 without any of the oracle's code:

      x_t = v_t * ones, v = 1/16, -1/32;  router[e, :] = rho_e = 1/2, 1/4, 0, -1/4,
      so logits = 64 v rho: token 0 [2, 1, 0, -1] picks experts 0, 1; token 1
      [-1, -1/2, 0, 1/2] picks 3, 2;
      gate_e = 2^-e,  up_e = 2^(e % 2)  (every weight):  g = 64 v 2^-e,  u = 64 v 2^(e % 2);
      down_e[d, :] = 2^-(1 + e // 2) (1 + d % 7):  down_e(h)[d] = 32 2^-(1 + e // 2) (1 + d % 7) h;
      shared: gate 1/2, up 1,  down[d, :] = (1 + d % 5) / 4,  gate vector 1/8, so
      s_t = 8 v and the shared term is sigmoid(8 v) * 8 (1 + d % 5) silu(32 v) 64 v;
      y_t[d] = sum_i w_i down_{e_i}(h_i)[d] + that shared term, w = p_i / (p_0 + p_1).

    A dropped shared expert or gate, sigmoid swapped for silu, gate/up swapped, a
    transposed down or a misplaced routing weight each change y.  Returns (spec in the
    layout kdq_moe_gguf takes, x [2, 64] float32, y [2, 64] float64, idx [2, 2])."""
    H, E, K, F, S = 64, 4, 2, 32, 32
    Q8 = 8
    v = [1.0 / 16, -1.0 / 32]
    rho = [0.5, 0.25, 0.0, -0.25]
    x = np.array([[v[0]] * H, [v[1]] * H], np.float32)
    router = np.array([[r] * H for r in rho], np.float32)
    gate = np.stack([_q8_0_rows(F, H, lambda r, e=e: 2.0 ** -e, lambda r, c: 1)
                     for e in range(E)])
    up = np.stack([_q8_0_rows(F, H, lambda r, e=e: 2.0 ** (e % 2), lambda r, c: 1)
                   for e in range(E)])
    down = np.stack([_q8_0_rows(H, F, lambda r, e=e: 2.0 ** -(1 + e // 2),
                                lambda r, c: 1 + r % 7) for e in range(E)])
    spec = dict(hidden=H, experts=E, top_k=K, ff=F, shared_ff=S,
                shared_gate=np.full(H, 0.125, np.float32),
                router=(0, router.view(np.uint8).reshape(E, -1)),
                gate_exps=(Q8, gate), up_exps=(Q8, up), down_exps=(Q8, down),
                gate_shexp=(Q8, _q8_0_rows(S, H, lambda r: 0.5, lambda r, c: 1)),
                up_shexp=(Q8, _q8_0_rows(S, H, lambda r: 1.0, lambda r, c: 1)),
                down_shexp=(Q8, _q8_0_rows(H, S, lambda r: 0.25, lambda r, c: 1 + r % 5)))
    idx = np.array([[0, 1], [3, 2]], np.int32)
    silu = lambda a: a / (1 + math.exp(-a))
    y = np.zeros((2, H), np.float64)
    for t in range(2):
        logits = [64 * v[t] * r for r in rho]
        top = max(logits)
        p = [math.exp(l - top) for l in logits]
        p = [q / sum(p) for q in p]
        chosen = [p[e] for e in idx[t]]
        for i, e in enumerate(idx[t]):
            h = silu(64 * v[t] * 2.0 ** -e) * 64 * v[t] * 2.0 ** (e % 2)
            for d in range(H):
                y[t, d] += chosen[i] / sum(chosen) * 32 * 2.0 ** -(1 + e // 2) * (1 + d % 7) * h
        hs = silu(32 * v[t]) * 64 * v[t]
        gate_t = 1 / (1 + math.exp(-8 * v[t]))
        for d in range(H):
            y[t, d] += gate_t * 32 * 0.25 * (1 + d % 5) * hs
    return spec, x, y, idx


def near_tie_logits(seed, rows, experts, top_k):
    """Router logits whose top-k boundary sits among values a few ulps apart.

    Per row: logits ~ N(0, sigma) with sigma from {0.5, 2, 6} (the widest spreads give
    probabilities below 2^-22, where the double total's summation order matters); then
    top_k + 2 experts get one value v plus 0..4 ulps each, v either the row's maximum or
    up to 3 below it, so exp(l - max) of the group are near-equal or equal floats and
    their order is decided in the last bits of expf, of the total and of the division.
    A quarter of the rows put a second group of near-equal values just above the
    first."""
    g = np.random.default_rng(seed)
    sigma = g.choice(np.array([0.5, 2.0, 6.0], np.float32), size=rows)
    logits = (g.standard_normal((rows, experts)).astype(np.float32) * sigma[:, None])
    m = min(experts, top_k + 2)
    for r in range(rows):
        top = logits[r].max()
        v = np.float32(top - (0.0 if r % 3 == 0 else g.uniform(0.0, 3.0)))
        group = g.choice(experts, size=m, replace=False)
        steps = g.integers(0, 5, size=m).astype(np.int32)
        logits[r, group] = (np.full(m, v, np.float32).view(np.int32) + steps).view(np.float32)
        if r % 4 == 1:
            second = g.choice(experts, size=2, replace=False)
            w = np.float32(v + np.float32(1e-3))
            logits[r, second] = (np.full(2, w, np.float32).view(np.int32) +
                                 g.integers(0, 3, size=2).astype(np.int32)).view(np.float32)
    return logits


# ---------------------------------------------------------------- fp16 operand model

def _fp16(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def sigma_fp16(a):
    """a rounded as the prefill GEMMs stage it: per row a power of two sigma with
    max|a| / sigma in [2^14, 2^15), fp16(a / sigma) * sigma."""
    a = np.asarray(a, np.float64)
    m = np.abs(a).max(axis=-1, keepdims=True)
    e = np.floor(np.log2(np.maximum(m, 1e-300))) + 1
    s = 2.0 ** (e - 15)
    return _fp16(a / s) * s


def gemm_fp16_weights(oracle, encoding, rows, n_in):
    """Rows as the prefill GEMM's dequantisation gives them (float64 of fp16 values):
    Q4_K fma16(q, fp16(d sc), fp16(-dmin m)), Q6_K fp16((q - 32) * fp16(d sc)), Q8_0
    fp16(q d) (d is fp16 already: exact); the codes and scales are read back from the
    exactly decoded values and the block bytes."""
    rows = np.ascontiguousarray(rows)
    n = rows.shape[0]
    exact = oracle.dequantize(encoding, rows, n_in).astype(np.float64)
    if encoding == 8:  # Q8_0
        return _fp16(exact)
    nb = n_in // 256
    if encoding == 14:  # Q6_K
        blk = rows.reshape(n, nb, 210)
        d = blk[..., 208:210].copy().view(np.float16).astype(np.float64)[..., 0]
        sc = blk[..., 192:208].view(np.int8).astype(np.float64)
        s = np.repeat(d[..., None] * sc, 16, axis=-1).reshape(n, n_in)
        with np.errstate(invalid="ignore", divide="ignore"):
            q = np.where(s != 0, np.round(exact / s), 0)
        return _fp16(q * _fp16(s))
    if encoding == 12:  # Q4_K
        blk = rows.reshape(n, nb, 144)
        d = blk[..., 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
        dmin = blk[..., 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
        sb = blk[..., 4:16].astype(np.int64)
        sc = np.zeros((n, nb, 8))
        m = np.zeros((n, nb, 8))
        for k in range(8):
            if k < 4:
                sc[..., k], m[..., k] = sb[..., k] & 63, sb[..., k + 4] & 63
            else:
                sc[..., k] = (sb[..., k + 4] & 15) | ((sb[..., k - 4] >> 6) << 4)
                m[..., k] = (sb[..., k + 4] >> 4) | ((sb[..., k] >> 6) << 4)
        a = np.repeat(d[..., None] * sc, 32, axis=-1).reshape(n, n_in)
        c = np.repeat(dmin[..., None] * m, 32, axis=-1).reshape(n, n_in)
        with np.errstate(invalid="ignore", divide="ignore"):
            q = np.where(a != 0, np.round((exact + c) / a), 0)
        return _fp16(q * _fp16(a) + _fp16(-c))  # one rounding of the fp16 fma
    raise ValueError(encoding)


def moe_gguf_fp16_model(oracle, spec, x, idx, w):
    """The GGUF MoE layer with every product on the prefill GEMMs' numeric model: x and h
    staged by sigma_fp16, weights as gemm_fp16_weights, float64 accumulation and
    element-wise work (the routing taken as given)."""
    H, E, K, F, S = (spec[k] for k in ("hidden", "experts", "top_k", "ff", "shared_ff"))

    def wt(name, n_in):
        enc, arr = spec[name]
        flat = arr.reshape(-1, arr.shape[-1])
        return gemm_fp16_weights(oracle, enc, flat, n_in).reshape(*arr.shape[:-1], n_in)

    silu = lambda v: v / (1.0 + np.exp(-v))
    gate, up, down = wt("gate_exps", H), wt("up_exps", H), wt("down_exps", F)
    xs = sigma_fp16(x)
    y = np.zeros((x.shape[0], H))
    for e in range(E):
        t, i = np.nonzero(idx == e)
        if t.size == 0:
            continue
        h = sigma_fp16(silu(xs[t] @ gate[e].T) * (xs[t] @ up[e].T))
        y[t] += w[t, i][:, None] * (h @ down[e].T)
    hs = sigma_fp16(silu(xs @ wt("gate_shexp", H).T) * (xs @ wt("up_shexp", H).T))
    g = 1.0 / (1.0 + np.exp(-(x.astype(np.float64) @ spec["shared_gate"].astype(np.float64))))
    return y + (hs @ wt("down_shexp", S).T) * g[:, None]

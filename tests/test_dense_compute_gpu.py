"""GPU tests of the C++ host layer kadan_amd::HipDenseCompute (include/
kadan_amd_dense_compute.hpp), driven through the C shim tests/cpp/dense_compute_probe.cpp.

Follows the contract the reference's DenseCompute tests check (IW/tests/
projection_validation.cpp, IW/tests/gguf_batch_partition.cpp:18-100, IW/tests/
worker_compute.cpp:540-601; IW = services/hikari/inference_worker): `unsupported`
before any source read or output write, bank hits read no rows,
non-retained weights are not banked, rejected inputs throw, batch results are
`unvalidated`.  Products must match the oracle within rel-L2 <= 1e-3 and max-abs <=
2e-2 of the output RMS.
"""
import ctypes
import os

import numpy as np
import pytest

from kadan_amd import synth
from tests.util import assert_close

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp",
                     "libdense_compute_probe.so")
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
Q3_K, IQ4_NL, IQ4_XS, BF16, IQ3_XXS = 11, 20, 23, 30, 18
UNSUPPORTED, UNVALIDATED, FINITE = 0, 1, 2

c_p = ctypes.c_void_p
c_sz = ctypes.c_size_t


def _p(a):
    return None if a is None else a.ctypes.data_as(c_p)


class Probe:
    def __init__(self):
        if not os.path.exists(PROBE):
            raise RuntimeError("tests/cpp/libdense_compute_probe.so is not built (run build())")
        self.lib = ctypes.CDLL(PROBE)
        L = self.lib
        L.kdc_create.restype = c_p
        L.kdc_create.argtypes = [ctypes.c_int, ctypes.c_char_p, c_sz]
        L.kdc_destroy.argtypes = [c_p]
        L.kdc_source_reads.restype = c_sz
        L.kdc_source_reads.argtypes = [c_p]
        L.kdc_retained.restype = c_sz
        L.kdc_retained.argtypes = [c_p]
        L.kdc_set_weight_limit.argtypes = [c_p, c_sz]
        L.kdc_release.restype = c_sz
        L.kdc_release.argtypes = [c_p, ctypes.c_ulonglong]
        L.kdc_release_scratch.argtypes = [c_p, ctypes.c_char_p, c_sz]
        L.kdc_dense_gguf.argtypes = [c_p, ctypes.c_ulonglong, ctypes.c_uint, c_p, c_sz, c_p, c_p,
                                     c_sz, c_sz, c_sz, c_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, c_p, ctypes.c_char_p, c_sz]
        L.kdc_dense_source.argtypes = [c_p, ctypes.c_ulonglong, c_p, c_p, c_p, c_sz, c_sz, c_sz,
                                       c_p, c_p, ctypes.c_char_p, c_sz]
        L.kdc_dense_gguf_batch.argtypes = [c_p, c_sz, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p,
                                           c_p, ctypes.c_char_p, c_sz]
        L.kdc_dense_gguf_q8.argtypes = [c_p, ctypes.c_ulonglong, c_p, c_sz, c_p, c_sz, c_sz, c_sz,
                                        c_p, c_p, ctypes.c_char_p, c_sz]
        L.kdc_moe_mxfp4.argtypes = [c_p, ctypes.c_ulonglong, c_sz, c_sz, c_sz] + [c_p] * 8 + [
            c_sz, c_sz, c_p, c_p, c_p, c_p, ctypes.c_char_p, c_sz]
        self.err = ctypes.create_string_buffer(512)
        self.h = L.kdc_create(0, self.err, 512)
        if not self.h:
            raise RuntimeError(self.err.value.decode())

    def close(self):
        self.lib.kdc_destroy(self.h)

    def _done(self, rc, result):
        if rc:
            raise RuntimeError(self.err.value.decode())
        return int(result.value)

    @property
    def reads(self):
        return self.lib.kdc_source_reads(self.h)

    @property
    def retained(self):
        return self.lib.kdc_retained(self.h)

    def set_weight_limit(self, nbytes):
        self.lib.kdc_set_weight_limit(self.h, nbytes)

    def release(self, ident):
        return self.lib.kdc_release(self.h, ident)

    def release_scratch(self):
        if self.lib.kdc_release_scratch(self.h, self.err, 512):
            raise RuntimeError(self.err.value.decode())

    def gguf(self, ident, enc, w, x, n_out, bias=None, retain=True, cancel=False,
             precise=False):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        rows, n_in = x.shape
        y = np.full((rows, n_out), np.nan, np.float32)
        res = ctypes.c_int(-1)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        rc = self.lib.kdc_dense_gguf(self.h, ident, enc, _p(w), w.size // n_out, _p(bias), _p(x),
                                     rows, n_in, n_out, _p(y), int(retain), int(cancel),
                                     int(precise), ctypes.byref(res), self.err, 512)
        return self._done(rc, res), y

    def dense_source(self, ident, w, x, bias=None):
        """F32 weights [out x in] through dense_source (a FloatWeightSource over w)."""
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        rows, n_in = x.shape
        n_out = w.shape[0]
        y = np.full((rows, n_out), np.nan, np.float32)
        res = ctypes.c_int(-1)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        rc = self.lib.kdc_dense_source(self.h, ident, _p(w), _p(bias), _p(x), rows, n_in, n_out,
                                       _p(y), ctypes.byref(res), self.err, 512)
        return self._done(rc, res), y

    def batch(self, jobs):
        """jobs: (ident, enc, weights, x, n_out); x objects may repeat to share an input."""
        n = len(jobs)
        ws = [np.ascontiguousarray(j[2], np.uint8) for j in jobs]
        xs = [j[3] for j in jobs]
        ys = [np.full((x.shape[0], j[4]), np.nan, np.float32) for x, j in zip(xs, jobs)]
        arr = lambda t, v: (t * n)(*v)
        res = ctypes.c_int(-1)
        rc = self.lib.kdc_dense_gguf_batch(
            self.h, n, arr(ctypes.c_ulonglong, [j[0] for j in jobs]),
            arr(ctypes.c_uint, [j[1] for j in jobs]), arr(c_p, [w.ctypes.data for w in ws]),
            arr(c_sz, [w.size // j[4] for w, j in zip(ws, jobs)]),
            arr(c_p, [x.ctypes.data for x in xs]), arr(c_sz, [x.shape[0] for x in xs]),
            arr(c_sz, [x.shape[1] for x in xs]), arr(c_sz, [j[4] for j in jobs]),
            arr(c_p, [y.ctypes.data for y in ys]), ctypes.byref(res), self.err, 512)
        return self._done(rc, res), ys

    def q8(self, ident, w, x_half, n_out):
        w = np.ascontiguousarray(w, np.uint8)
        x_half = np.ascontiguousarray(x_half, np.uint16)
        rows, n_in = x_half.shape
        y = np.zeros((rows, n_out), np.uint16)
        res = ctypes.c_int(-1)
        rc = self.lib.kdc_dense_gguf_q8(self.h, ident, _p(w), w.size // n_out, _p(x_half), rows,
                                        n_in, n_out, _p(y), ctypes.byref(res), self.err, 512)
        return self._done(rc, res), y

    def moe(self, ident, experts, hidden, inter, weights, x_bf16, logits, top_k):
        tokens = x_bf16.shape[0]
        y = np.full((tokens, hidden), np.nan, np.float32)
        sel = np.full((tokens, top_k), -1, np.int32)
        rw = np.zeros((tokens, top_k), np.float32)
        weights = [np.ascontiguousarray(a, np.uint8) for a in weights]
        res = ctypes.c_int(-1)
        rc = self.lib.kdc_moe_mxfp4(self.h, ident, experts, hidden, inter,
                                    *[_p(a) for a in weights],
                                    _p(np.ascontiguousarray(x_bf16, np.uint16)),
                                    _p(np.ascontiguousarray(logits, np.float32)), tokens, top_k,
                                    _p(y), _p(sel), _p(rw), ctypes.byref(res), self.err, 512)
        return self._done(rc, res), y, sel, rw


@pytest.fixture()
def probe(device):
    p = Probe()
    yield p
    p.close()


@pytest.mark.parametrize("enc", [Q8_0, Q4_0, Q4_K, Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16, IQ3_XXS, 21, 22])
@pytest.mark.parametrize("rows", [1, 3, 8, 20, 200])
def test_dense_gguf_source_parity_and_bank(probe, oracle, enc, rows):
    n_in, n_out = 1024, 96
    w = synth.gguf_weights(enc, 0xD0 + enc, n_out, n_in)
    x = synth.normal(0xD1, rows, rows * n_in).reshape(rows, n_in)
    bias = synth.normal(0xD2, 1, n_out)
    want = oracle.gemv(enc, w, x, n_in, n_out) + bias[None, :]
    res, y = probe.gguf(7, enc, w, x, n_out, bias=bias)
    assert res == FINITE
    assert_close(y, want, what=f"dense_gguf_source enc={enc} rows={rows}")
    assert probe.reads == n_out
    assert probe.retained == w.size
    res, y2 = probe.gguf(7, enc, w, x, n_out, bias=bias)  # bank hit: no source read
    assert res == FINITE and probe.reads == n_out
    assert np.array_equal(y, y2)
    assert probe.release(7) == w.size and probe.retained == 0


def test_dense_gguf_source_not_retained(probe, oracle):
    w = synth.gguf_weights(Q4_K, 0xD3, 64, 512)
    x = synth.normal(0xD4, 1, 512).reshape(1, 512)
    for _ in range(2):
        res, y = probe.gguf(9, Q4_K, w, x, 64, retain=False)
        assert res == FINITE
        assert_close(y, oracle.gemv(Q4_K, w, x, 512, 64), what="retain_misses=false")
    assert probe.reads == 128 and probe.retained == 0


def test_dense_gguf_source_unsupported_reads_nothing(probe):
    x = np.ones((1, 512), np.float32)
    w = np.zeros(64 * 512, np.uint8)
    res, y = probe.gguf(1, 3, w, x, 64)  # GGML type 3 (Q4_1): no encoding here
    assert res == UNSUPPORTED
    res, _ = probe.gguf(1, Q4_0, w, np.ones((1, 48), np.float32), 64)  # 48 % 32 != 0
    assert res == UNSUPPORTED
    assert probe.reads == 0 and np.isnan(y).all()


def test_dense_gguf_source_rejections(probe):
    w = synth.gguf_weights(Q8_0, 0xD5, 32, 256)
    x = synth.normal(0xD6, 1, 256).reshape(1, 256)
    x[0, 3] = np.nan
    with pytest.raises(RuntimeError, match="kdq_nonfinite_input"):
        probe.gguf(2, Q8_0, w, x, 32)
    with pytest.raises(RuntimeError, match="kdq_cancelled"):
        probe.gguf(2, Q8_0, w, np.ones((1, 256), np.float32), 32, cancel=True)
    bad = w.reshape(32, -1).copy()
    bad[4, 0], bad[4, 1] = 0x00, 0x7C  # +inf block scale
    with pytest.raises(RuntimeError, match="kdq_nonfinite_weight"):
        probe.gguf(3, Q8_0, bad, np.ones((1, 256), np.float32), 32)
    assert probe.reads == 32  # only the inf-scale weights were read


def test_dense_gguf_batch_shared_input(probe, oracle):
    """gate + up share one input span, down reads another (the reference's FFN batch)."""
    h, f = 512, 1536
    x = synth.normal(0xD7, 1, 2 * h).reshape(2, h)
    xf = synth.normal(0xD8, 1, 2 * f).reshape(2, f)
    wg = synth.gguf_weights(Q4_K, 0xD9, f, h)
    wu = synth.gguf_weights(Q4_0, 0xDA, f, h)
    wd = synth.gguf_weights(Q8_0, 0xDB, h, f)
    res, ys = probe.batch([(11, Q4_K, wg, x, f), (12, Q4_0, wu, x, f), (13, Q8_0, wd, xf, h)])
    assert res == UNVALIDATED
    assert_close(ys[0], oracle.gemv(Q4_K, wg, x, h, f), what="batch gate")
    assert_close(ys[1], oracle.gemv(Q4_0, wu, x, h, f), what="batch up")
    assert_close(ys[2], oracle.gemv(Q8_0, wd, xf, f, h), what="batch down")
    assert probe.reads == 2 * f + h


def test_dense_gguf_batch_row_groups_take_the_gemm(probe, oracle):
    """Routed-expert jobs at prefill (more than gguf_batch_rows rows, up to
    gguf_batch_max_rows) over packed Q4_K / Q6_K / Q8_0 run the prefill GEMM; a decode job
    in the same submission stays on the decode-time product."""
    h, f = 512, 384
    x40 = synth.normal(0xE1, 1, 40 * h).reshape(40, h)
    x16 = synth.normal(0xE2, 1, 16 * h).reshape(16, h)
    x2 = synth.normal(0xE3, 1, 2 * h).reshape(2, h)
    x300 = synth.normal(0xE4, 1, 300 * h).reshape(300, h)
    w1 = synth.gguf_weights(Q4_K, 0xE5, f, h)
    w2 = synth.gguf_weights(Q6_K, 0xE6, f, h)
    w3 = synth.gguf_weights(Q8_0, 0xE7, f, h)
    res, ys = probe.batch([(21, Q4_K, w1, x40, f), (22, Q6_K, w2, x16, f),
                           (23, Q8_0, w3, x2, f), (24, Q8_0, w3, x300, f)])
    assert res == UNVALIDATED
    assert_close(ys[0], oracle.gemv(Q4_K, w1, x40, h, f), what="batch gemm q4_k 40 rows")
    assert_close(ys[1], oracle.gemv(Q6_K, w2, x16, h, f), what="batch gemm q6_k 16 rows")
    assert_close(ys[2], oracle.gemv(Q8_0, w3, x2, h, f), what="batch decode q8_0 2 rows")
    assert_close(ys[3], oracle.gemv(Q8_0, w3, x300, h, f), what="batch gemm q8_0 300 rows")


def test_dense_gguf_source_prefill_fp16_range_fallback(probe, oracle):
    """A block scale whose dequantised weights could pass the fp16 range (d = 1000, codes up
    to 127) makes the prefill GEMM flag the call, which then runs the decode-time product:
    the result is still the exact product."""
    rows, n_in, n_out = 24, 512, 64
    w = synth.gguf_weights(Q8_0, 0xE8, n_out, n_in).reshape(n_out, -1).copy()
    big = np.array([1000.0], np.float16).view(np.uint16)[0]
    w[3, 0], w[3, 1] = big & 255, big >> 8
    x = synth.normal(0xE9, 1, rows * n_in).reshape(rows, n_in)
    res, y = probe.gguf(31, Q8_0, w, x, n_out)
    assert res == FINITE
    assert_close(y, oracle.gemv(Q8_0, w, x, n_in, n_out), what="prefill fp16-range fallback")


def test_dense_gguf_batch_unsupported_job_reads_nothing(probe):
    x = np.ones((1, 256), np.float32)
    w = synth.gguf_weights(Q8_0, 0xDC, 32, 256)
    res, ys = probe.batch([(1, Q8_0, w, x, 32), (2, 3, np.zeros(32 * 20, np.uint8), x, 32)])
    assert res == UNSUPPORTED and probe.reads == 0 and np.isnan(ys[0]).all()


def test_dense_gguf_q8_source(probe, oracle):
    rows, n_in, n_out = 40, 512, 192
    w = synth.q4_0_weights(0xDD, n_out, n_in)
    xh = synth.normal(0xDE, 1, rows * n_in).reshape(rows, n_in).astype(np.float16)
    res, y = probe.q8(21, w, xh.view(np.uint16), n_out)
    assert res == UNVALIDATED
    xq, xd = oracle.quantize_q8_f16(xh.view(np.uint16))
    want = oracle.gemm_q4_0_q8(w, n_out, n_in, xq, xd)
    assert_close(y.view(np.float16).astype(np.float32), want, what="dense_gguf_q8_source")


def test_moe_mxfp4_host_layer(probe, oracle):
    tokens, hidden, inter, experts, top_k = 9, 128, 192, 8, 2
    x, logits = synth.moe_inputs(0xDF, tokens, hidden, experts)
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(0xDF, experts, hidden, inter)
    want, idx, w, _, _ = oracle.moe_forward(x, logits, top_k, gb, gs, ub, us, db, ds)
    res, y, sel, rw = probe.moe(31, experts, hidden, inter, (gb, gs, ub, us, db, ds), x, logits,
                                top_k)
    assert res == FINITE
    assert np.array_equal(sel, idx)
    assert_close(rw, w, rel=1e-6, mabs=1e-5, what="routing weights")
    assert_close(y, want, what="moe host layer")
    banked = probe.retained
    assert banked >= gb.size + gs.size + ub.size + us.size + db.size + ds.size
    res, y2, _, _ = probe.moe(31, experts, hidden, inter, (gb, gs, ub, us, db, ds), x, logits,
                              top_k)
    assert res == FINITE and np.array_equal(y, y2) and probe.retained == banked
    assert probe.release(31) == banked
    probe.release_scratch()


def test_bank_keeps_products_packed(probe, oracle):
    """The bank keeps weights for the decode-time product in the tile-packed form (16-row
    tiles: 40 rows occupy 48 rows' bytes) and returns the same results from it."""
    import kadan_amd
    n_in, n_out, rows = 512, 40, 3
    w = synth.gguf_weights(Q4_K, 0xDA, n_out, n_in)
    x = synth.normal(0xDB, rows, rows * n_in).reshape(rows, n_in)
    res, y = probe.gguf(41, Q4_K, w, x, n_out)
    assert res == FINITE
    assert_close(y, oracle.gemv(Q4_K, w, x, n_in, n_out), what="packed bank")
    packed = kadan_amd.lib().kdq_gguf_packed_bytes(Q4_K, n_in, n_out)
    assert packed == 3 * 2 * 2304 and probe.retained == packed
    assert probe.release(41) == packed and probe.retained == 0


def test_bank_shares_one_copy_between_decode_and_prefill(probe, oracle):
    """Q4_0 weights banked by the decode product (tile-packed) serve the prefill GEMM of
    the same identity without a second upload, and the GEMM reads the packed copy."""
    import kadan_amd
    n_in, n_out, rows = 768, 72, 2
    w = synth.q4_0_weights(0xE1, n_out, n_in)
    x = synth.normal(0xE2, rows, rows * n_in).reshape(rows, n_in)
    res, y = probe.gguf(43, Q4_0, w, x, n_out)
    assert res == FINITE
    assert_close(y, oracle.gemv(Q4_0, w, x, n_in, n_out), what="decode from the bank")
    packed = kadan_amd.lib().kdq_gguf_packed_bytes(Q4_0, n_in, n_out)
    assert probe.retained == packed
    xh = synth.normal(0xE3, 1, 130 * n_in).reshape(130, n_in).astype(np.float16)
    res, yq = probe.q8(43, w, xh.view(np.uint16), n_out)
    assert res == UNVALIDATED and probe.reads == n_out and probe.retained == packed
    xq, xd = oracle.quantize_q8_f16(xh.view(np.uint16))
    want = oracle.gemm_q4_0_q8(w, n_out, n_in, xq, xd)
    assert_close(yq.view(np.float16).astype(np.float32), want, what="prefill from the bank")
    assert probe.release(43) == packed and probe.retained == 0


def _columns(seed, n, chunk):
    """Sampled output columns, with both sides of every staging-chunk boundary."""
    pick = set(np.random.default_rng(seed).choice(n, 96, replace=False).tolist())
    for b in range(chunk, n, chunk):
        pick.update((b - 1, b))
    pick.update((0, n - 1))
    return np.array(sorted(pick))


# (encoding, in, out, rows per 16 MiB staging chunk): several chunks each, the last one
# partial; Q4_K and Q8_0 stream through the packed layout, Q3_K through plain rows.
STREAMED = [(Q4_K, 4096, 16000, 7280), (Q8_0, 4096, 8000, 3840), (Q3_K, 4096, 20000, 9532)]


@pytest.mark.parametrize("enc,n_in,n_out,chunk", STREAMED)
@pytest.mark.parametrize("rows", [3, 40])
def test_dense_gguf_source_streams_misses(probe, oracle, enc, n_in, n_out, chunk, rows):
    """A miss that is not retained is streamed in staging chunks (the reads of one chunk
    overlapping the upload, packing and product of the previous one): every row is read
    exactly once per call, nothing is banked, and the result is the exact product (the
    decode-time product at 3 rows, the prefill GEMM for the packed encodings at 40)."""
    w = synth.gguf_weights(enc, 0xF0 + enc, n_out, n_in)
    x = synth.normal(0xF1, rows, rows * n_in).reshape(rows, n_in)
    bias = synth.normal(0xF2, 1, n_out)
    res, y = probe.gguf(51, enc, w, x, n_out, bias=bias, retain=False)
    assert res == FINITE
    assert probe.reads == n_out and probe.retained == 0
    pick = _columns(enc + rows, n_out, chunk)
    want = oracle.gemv(enc, w[pick], x, n_in, len(pick)) + bias[None, pick]
    assert_close(y[:, pick], want, what=f"streamed enc={enc} rows={rows}")
    assert np.isfinite(y).all()
    res, y2 = probe.gguf(51, enc, w, x, n_out, bias=bias, retain=False)
    assert res == FINITE and probe.reads == 2 * n_out and np.array_equal(y, y2)


def test_weight_limit_refuses_and_streams(probe, oracle):
    """IW/include/kadan/device_weights.hpp:203-206: under a byte limit the bank admits
    misses until the next would pass it; later misses are streamed (read again on every
    call) while the admitted weights keep hitting, and nothing is evicted."""
    import kadan_amd
    n_in, n_out, rows = 512, 64, 2
    size = kadan_amd.lib().kdq_gguf_packed_bytes(Q4_K, n_in, n_out)
    probe.set_weight_limit(2 * size + size // 2)
    ws = {i: synth.gguf_weights(Q4_K, 0xF4 + i, n_out, n_in) for i in (1, 2, 3)}
    x = synth.normal(0xF8, rows, rows * n_in).reshape(rows, n_in)
    want = {i: oracle.gemv(Q4_K, w, x, n_in, n_out) for i, w in ws.items()}
    # (weight, rows read so far, weights banked): 1 and 2 admitted, 3 refused every time
    for ident, reads, banked in ((1, 64, 1), (2, 128, 2), (3, 192, 2), (1, 192, 2),
                                 (3, 256, 2), (2, 256, 2)):
        res, y = probe.gguf(60 + ident, Q4_K, ws[ident], x, n_out)
        assert res == FINITE
        assert_close(y, want[ident], what=f"limited bank weight {ident}")
        assert (probe.reads, probe.retained) == (reads, banked * size), ident
    assert probe.release(63) == 0  # never admitted
    assert probe.release(61) == size and probe.release(62) == size and probe.retained == 0
    probe.set_weight_limit(size // 2)  # below one weight: streamed, nothing evicted
    res, y = probe.gguf(61, Q4_K, ws[1], x, n_out)
    assert res == FINITE and probe.retained == 0
    assert_close(y, want[1], what="weight larger than the limit")


def test_streamed_prefill_fp16_range_fallback(probe, oracle):
    """A streamed GEMM chunk that flags the fp16 range (one block scale of 1000 in the
    second staging chunk) sends the call through the streamed decode-time product: every
    row is read twice and the result is still the exact product."""
    rows, n_in, n_out = 24, 4096, 8000
    w = synth.gguf_weights(Q8_0, 0xF9, n_out, n_in).reshape(n_out, -1).copy()
    big = np.array([1000.0], np.float16).view(np.uint16)[0]
    w[5000, 0], w[5000, 1] = big & 255, big >> 8
    x = synth.normal(0xFA, 1, rows * n_in).reshape(rows, n_in)
    res, y = probe.gguf(71, Q8_0, w, x, n_out, retain=False)
    assert res == FINITE and probe.reads == 2 * n_out and probe.retained == 0
    pick = np.union1d(_columns(0xFB, n_out, 3840), [5000])
    assert_close(y[:, pick], oracle.gemv(Q8_0, w[pick], x, n_in, len(pick)),
                 what="streamed fp16-range fallback")


def _f64_product(w, x, bias=None):
    y = x.astype(np.float64) @ w.astype(np.float64).T
    return y if bias is None else y + bias.astype(np.float64)


@pytest.mark.parametrize("rows", [1, 4, 8, 33])
def test_batch_f32_router_with_shared_gate_up(probe, oracle, rows):
    """MoeLayer::forward's first batch (IW/src/models/text/qwen_layers.cpp:383-389): an F32
    router job (no encoding: F32 rows from a byte source, IW/src/models/text/
    gguf_weights.cpp:456-466) and the Q8_0 shared gate and up, all on one input."""
    hidden, experts, shared_ff = 2048, 128, 768
    g = np.random.default_rng(0xF32 + rows)
    router = (g.standard_normal((experts, hidden)) * 0.05).astype(np.float32)
    wg = synth.gguf_weights(Q8_0, 0xF33, shared_ff, hidden)
    wu = synth.gguf_weights(Q8_0, 0xF34, shared_ff, hidden)
    x = synth.normal(0xF35, rows, rows * hidden).reshape(rows, hidden)
    rv = router.view(np.uint8).reshape(experts, -1)
    res, (logits, gate, up) = probe.batch([(900 + rows, 0, rv, x, experts),
                                           (910 + rows, Q8_0, wg, x, shared_ff),
                                           (920 + rows, Q8_0, wu, x, shared_ff)])
    assert res == UNVALIDATED
    want = _f64_product(router, x)
    rel = np.linalg.norm(logits - want) / np.linalg.norm(want)
    assert rel < 1e-6, rel  # the exact fp32 product, fp32 accumulation in a fixed order
    assert_close(gate, oracle.gemv(Q8_0, wg, x, hidden, shared_ff))
    assert_close(up, oracle.gemv(Q8_0, wu, x, hidden, shared_ff))
    # a second call finds all three in the bank
    before = probe.reads
    res, (logits2, _, _) = probe.batch([(900 + rows, 0, rv, x, experts),
                                        (910 + rows, Q8_0, wg, x, shared_ff),
                                        (920 + rows, Q8_0, wu, x, shared_ff)])
    assert probe.reads == before and np.array_equal(logits, logits2)


def test_batch_f32_nonfinite_weight_throws(probe):
    router = np.ones((16, 64), np.float32)
    router[3, 5] = np.inf
    x = np.ones((1, 64), np.float32)
    with pytest.raises(RuntimeError, match="kdq_nonfinite_weight"):
        probe.batch([(950, 0, router.view(np.uint8).reshape(16, -1), x, 16)])


def test_batch_f32_refusals_read_nothing(probe):
    # in % 8 != 0 (IW/include/kadan/gguf_batch_partition.hpp:35), on a mixed batch: the
    # whole batch is refused before any read or write
    x36 = np.ones((1, 36), np.float32)
    w = np.ones((4, 36), np.float32).view(np.uint8).reshape(4, -1)
    xq = np.ones((1, 256), np.float32)
    wq = synth.gguf_weights(Q8_0, 0xF36, 8, 256)
    res, (y0, y1) = probe.batch([(960, Q8_0, wq, xq, 8), (961, 0, w, x36, 4)])
    assert res == UNSUPPORTED and probe.reads == 0
    assert np.isnan(y0).all() and np.isnan(y1).all()


@pytest.mark.parametrize("n_in", [37, 256, 4100])
def test_dense_source_f32(probe, n_in):
    """dense_source (IW/include/kadan/dense_compute.hpp:239-249): F32 weights from a
    FloatWeightSource (element offsets), any width, bias, the bank shared across calls."""
    g = np.random.default_rng(n_in)
    n_out, rows = 96, 3
    w = g.standard_normal((n_out, n_in)).astype(np.float32)
    x = g.standard_normal((rows, n_in)).astype(np.float32)
    b = g.standard_normal(n_out).astype(np.float32)
    res, y = probe.dense_source(970 + n_in, w, x, b)
    assert res == FINITE
    want = _f64_product(w, x, b)
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 1e-6
    reads = probe.reads
    assert reads == n_out
    res, y2 = probe.dense_source(970 + n_in, w, x, b)
    assert probe.reads == reads and np.array_equal(y, y2)


def test_dense_source_nonfinite_weight_throws(probe):
    w = np.ones((8, 64), np.float32)
    w[7, 63] = np.nan
    with pytest.raises(RuntimeError, match="kdq_nonfinite_weight"):
        probe.dense_source(990, w, np.ones((1, 64), np.float32))


def test_precise_prefill_takes_the_exact_product(probe, oracle):
    """precise=true keeps fp32 operands at prefill row counts (the exact-decode product:
    fp32 weights as kdq_dequantize decodes them, fp32 fused multiply-adds), so it sits
    within fp32 rounding of the oracle's product, far inside the fp16 GEMM's error."""
    n_in, n_out, rows = 1024, 96, 40
    w = synth.gguf_weights(Q4_K, 0xF37, n_out, n_in)
    x = synth.normal(0xF38, rows, rows * n_in).reshape(rows, n_in)
    res, y = probe.gguf(995, Q4_K, w, x, n_out, precise=True)
    assert res == FINITE
    want = oracle.gemv(Q4_K, w, x, n_in, n_out)
    assert_close(y, want)
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    assert rel < 1e-6, rel

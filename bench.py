#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-weight matmul path (one GPU).

Headline (``value``): Q4_K GEMV weight throughput in GB/s at the Llama-3-8B FFN
decode shape gate/up 4096 -> 14336, batch 1 (the benchmark's configs[1]), with the inputs
resident in HBM in the library's tile-packed layout (kdq_gguf_pack, the form its weight
bank keeps).  A "step" is one GEMV over one weight copy (one kernel launch, one
kdq_gemv_packed_batch submission); the timed steps rotate over 16 distinct weight
copies (528 MB, twice the 256 MB Infinity Cache) so the cache cannot serve the weights.

The same line carries
  roofline      the GEMV kernel's algorithmic bytes / measured average launch time
                against the 8 TB/s HBM3E peak (traffic from profiles/traffic.json,
                the rocprofv3 FETCH_SIZE/WRITE_SIZE measurement, when present)
  cpu_baseline  the reference CPU path on this host: kadan::text::CpuMatvec over ggml's
                x86 quantize_row_q8_K + vec_dot_q4_K_q8_K (oracle/_ref, compiled from the
                reference sources), on the reference worker split (64-column units,
                clamp(cores/2, 1, 16) threads), on a bounded sample of the same workload
                rotating over 4 weight copies
  extra         the HBM read ceiling at the headline's size (kdq_hbm_read, timed the same
                way), the other benchmark configurations (C1 Q8_0 GEMV, C2 down, C3 Q4_0
                GEMM, C4 MoE at 1 and 256 tokens, C5 MoE at 2048 skewed tokens) and the
                prefill GEMMs, each timed with events over back-to-back launches (median
                of repetitions)

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-extra] [--skip-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0      # dense fp16/bf16 MFMA
FP4_PEAK_TFLOPS = 10100.0      # dense MXFP4 MFMA
Q4_K, Q8_0, Q4_0 = 12, 8, 2
Q3_K, Q6_K, IQ4_NL, IQ4_XS, BF16 = 11, 14, 20, 23, 30
IQ3_XXS, IQ3_S, IQ2_S = 18, 21, 22


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--skip-extra", action="store_true")
    p.add_argument("--skip-cpu", action="store_true")
    p.add_argument("--only", action="append", default=None,
                   help="run only these extra workloads (repeatable), e.g. c3_q4_0_gemm")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a 256 MiB device copy (reference for counter scaling)")
    return p.parse_args()


def rotated_copies(torch, base: np.ndarray, copies: int, keep: np.ndarray, seed: int):
    """`copies` distinct device copies of packed weights: copy 0 is `base`, copy c XORs
    every byte outside `keep` (the scale bytes) with a seeded byte stream, which keeps
    codes uniform and leaves the scale distribution unchanged."""
    dev = torch.device("cuda:0")
    first = torch.from_numpy(np.ascontiguousarray(base)).to(dev)
    out = [first]
    mask = torch.from_numpy(np.ascontiguousarray(~keep)).to(dev)
    g = torch.Generator(device=dev)
    for c in range(1, copies):
        g.manual_seed(seed * 1000 + c)
        noise = torch.randint(0, 256, first.shape, dtype=torch.uint8, device=dev, generator=g)
        out.append(torch.where(mask, first ^ noise, first))
    return out


def keep_mask(encoding: int, shape) -> np.ndarray:
    """True for the scale bytes of each packed row (d, dmin) that must stay as generated
    (BF16: every byte, so the copies stay the same finite values)."""
    rows, row_bytes = shape
    if encoding == BF16:
        return np.ones(shape, bool)
    keep = np.zeros(row_bytes, bool)
    block = {Q4_K: 144, Q8_0: 34, Q4_0: 18, Q3_K: 110, Q6_K: 210, IQ4_NL: 18, IQ4_XS: 136,
             IQ3_XXS: 98, IQ3_S: 110, IQ2_S: 82}[encoding]
    at, head = {Q4_K: (0, 4), Q3_K: (108, 2), Q6_K: (208, 2)}.get(encoding, (0, 2))
    for b in range(0, row_bytes, block):
        keep[b + at:b + at + head] = True
    return np.broadcast_to(keep, shape).copy()


def time_launches(torch, launch, count: int, reps: int = 1):
    """Average ms per launch over `count` back-to-back launches, events on the launch
    stream; median of `reps` repetitions."""
    stream = torch.cuda.current_stream()
    results = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for i in range(count):
            launch(i)
        stop.record(stream)
        stop.synchronize()
        results.append(start.elapsed_time(stop) / count)
    return statistics.median(results)


MIN_LAUNCHES = 1000      # launches timed per measurement, whatever --steps asks for
MIN_PER_REP = 100        # back-to-back launches inside each pair of events
MIN_WARMUP = 200         # untimed launches first, so the clocks leave their idle state


def timed_launches(steps: int) -> int:
    """Launches a measurement times: `steps`, raised to MIN_LAUNCHES so every one of the
    10 repetitions brackets at least MIN_PER_REP back-to-back launches (a pair of events
    around 2 launches of a 7 us kernel times the launch gap, not the kernel)."""
    return max(steps, MIN_LAUNCHES)


def time_steps(torch, submit, steps: int, reps: int = 10):
    """ms per step: timed_launches(steps) steps issued by `submit(n)` (which enqueues n
    steps), bracketed by synchronizations, split into `reps` back-to-back repetitions of
    at least MIN_PER_REP launches each (the last takes the remainder), each timed by its
    own pair of events on the launch stream; the median of the repetitions' per-step
    times."""
    stream = torch.cuda.current_stream()
    steps = timed_launches(steps)
    reps = max(1, min(reps, steps // MIN_PER_REP))
    counts = [steps // reps] * reps
    counts[-1] += steps - sum(counts)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    events[0].record(stream)
    for i, n in enumerate(counts):
        submit(n)
        events[i + 1].record(stream)
    events[-1].synchronize()
    torch.cuda.synchronize()
    return statistics.median(events[i].elapsed_time(events[i + 1]) / counts[i]
                             for i in range(reps))


def gemv_bytes(n_in: int, n_out: int, encoding: int) -> int:
    from kadan_amd import row_bytes
    return n_out * row_bytes(encoding, n_in) + 4 * n_in + 4 * n_out


def traffic_for(workload: str):
    """HBM bytes per launch of the workload's kernel from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE measurement (profiles/traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(workload)
    except (OSError, ValueError):
        return None
    return entry.get("bytes") if isinstance(entry, dict) else None


def cpu_baseline(seconds: float, copies: int = 4):
    """Reference CPU path on a bounded sample of the C2 gate/up workload, rotating over
    `copies` distinct weight copies (235 MB) so the host caches cannot hold them."""
    from kadan_amd import synth
    n_in, n_out = 4096, 14336
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    threads = max(1, min(16, affinity // 2))  # IW/src/models/text/gguf_weights.cpp:615-618
    base = synth.q4_k_weights(0xC2A, n_out, n_in)
    keep = keep_mask(Q4_K, base.shape)
    ws = [base]
    for c in range(1, copies):
        noise = synth.random_bytes(0xC2A, 100 + c, base.size).reshape(base.shape)
        ws.append(np.where(keep, base, base ^ noise))
    x = synth.normal(0xC2A, 50, n_in).reshape(1, n_in)
    import oracle
    if oracle.Reference.available():
        impl, kind = oracle.Reference(), "reference"
    else:
        impl, kind = oracle.Oracle(), "port"
    for w in ws:  # warm-up, one pass over every copy
        impl.cpu_matvec(Q4_K, w, x, n_in, n_out, threads)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        impl.cpu_matvec(Q4_K, ws[len(times) % copies], x, n_in, n_out, threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(gemv_bytes(n_in, n_out, Q4_K) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": kind,
        "cpu_model": cpu_model(),
        "sample": (f"{len(times)} runs (median) of the C2 gate/up Q4_K matvec 4096->14336, "
                   f"batch 1, over {copies} rotated weight copies: quantize_row_q8_K + "
                   f"vec_dot_q4_K_q8_K via CpuMatvec, 64-column units on {threads} threads "
                   f"of {affinity} available"),
    }


def cpu_thread_counts():
    """1 thread, the reference policy clamp(cores/2, 1, 16) (IW/src/models/text/
    gguf_weights.cpp:615-618), and every core this process may use (at most 16, the
    GPU box's share of one GPU)."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return cores, sorted({1, max(1, min(16, cores // 2)), max(1, min(16, cores))})


def timed_median(fn, seconds: float, least: int = 3):
    t0 = time.perf_counter()
    fn()  # warm-up; a run longer than the budget counts as the sample itself
    first = time.perf_counter() - t0
    if first > seconds:
        return first, 1
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < least:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baselines(seconds: float = 2.0):
    """The reference CPU path (oracle/_ref where built, else the oracle restatement) for
    C1, C2, C3, C4 and C5 at each thread count of cpu_thread_counts(), bounded samples of
    about `seconds` each; C3 and the MoE legs time a stated subset of rows or tokens.  The
    MoE layer runs twice: the exact flow (double accumulation, the reference's
    quantization::matvec semantics) and an AVX2 fp32 form (`*_f32`)."""
    from kadan_amd import synth
    import oracle
    cores, counts = cpu_thread_counts()
    ref = oracle.Reference() if oracle.Reference.available() else None
    impl = ref or oracle.Oracle()
    kind = "reference" if ref else "port"
    port = oracle.Oracle()
    out = {"cores_available": cores, "threads": counts, "cpu_model": cpu_model()}

    def gemv_leg(name, encoding, n_in, n_out, seed, copies=4):
        base = synth.gguf_weights(encoding, seed, n_out, n_in)
        keep = keep_mask(encoding, base.shape)
        ws = [base] + [np.where(keep, base, base ^ synth.random_bytes(seed, 100 + c, base.size)
                                .reshape(base.shape)) for c in range(1, copies)]
        x = synth.normal(seed, 50, n_in).reshape(1, n_in)
        nb = gemv_bytes(n_in, n_out, encoding)
        legs = {}
        for th in counts:
            state = {"i": 0}

            def run():
                impl.cpu_matvec(encoding, ws[state["i"] % copies], x, n_in, n_out, th)
                state["i"] += 1
            med, n = timed_median(run, seconds)
            legs[str(th)] = {"gbs": round(nb / med / 1e9, 2), "ms": round(med * 1e3, 3),
                             "runs": n}
        out[name] = {"kind": kind, "unit": "GB/s", "by_threads": legs,
                     "sample": f"whole matvec, {copies} weight copies"}

    gemv_leg("c1_q8_0_gemv_4096x4096", Q8_0, 4096, 4096, 0xC1)
    gemv_leg("c2_q4_k_gemv_4096_to_14336", Q4_K, 4096, 14336, 0xC2A)
    gemv_leg("c2_q4_k_gemv_14336_to_4096", Q4_K, 14336, 4096, 0xC2B)

    # C3: Q8_0-quantised activation rows x Q4_0 weights (CpuMatvec over the rows)
    n_out, k, rows = 14336, 4096, 32
    w = synth.gguf_weights(Q4_0, 0xC3, n_out, k)
    x16 = synth.normal(0xC3, 60, rows * k).astype(np.float16).astype(np.float32)
    x16 = x16.reshape(rows, k)
    legs = {}
    for th in counts:
        med, n = timed_median(lambda: impl.cpu_matvec(Q4_0, w, x16, k, n_out, th), seconds)
        legs[str(th)] = {"tflops": round(2.0 * rows * k * n_out / med / 1e12, 4),
                         "ms": round(med * 1e3, 2), "runs": n}
    out["c3_q4_0_gemm"] = {"kind": kind, "unit": "TFLOP/s", "by_threads": legs,
                           "sample": f"{rows} of 512 rows, all outputs"}

    # C4 and C5: the MoE layer flow with exact MXFP4 products (the oracle's composition:
    # the reference has no compiled MXFP4 MoeLayer)
    for experts, hot, seed, legs_of in ((32, 0, 0xC4, (("c4_moe_t1", 1, [0]),
                                                       ("c4_moe_t256", 256, [0, 1, 2, 3]))),
                                        (128, 8, 0xC5, (("c5_moe_t2048_skewed", 2048,
                                                         [0, 1]),))):
        (gb, gs), (ub, us), (db, ds) = synth.moe_weights(seed, experts, 2880, 2880)
        for name, tokens, sample in legs_of:
            xa, la = synth.moe_inputs(seed, tokens, 2880, experts, hot=hot)
            xa, la = xa[sample], la[sample]
            legs = {}
            for th in counts:
                med, n = timed_median(lambda: port.moe_forward(xa, la, 4, gb, gs, ub, us, db,
                                                               ds, threads=th),
                                      seconds, least=1)
                legs[str(th)] = {"tokens_per_s": round(len(sample) / med, 2),
                                 "ms": round(med * 1e3, 2), "runs": n}
            out[name] = {"kind": "port", "unit": "tokens/s", "by_threads": legs,
                         "sample": f"tokens {sample}" + (" (0 hot)" if hot else "")
                                   + ", exact double-accumulated products"}
            # the fast CPU form: fp32 products on AVX2 FMA, 64-row units over the threads
            fsample = list(range(min(tokens, 32 if experts == 32 else 64)))
            xf, lf = synth.moe_inputs(seed, tokens, 2880, experts, hot=hot)
            xf, lf = xf[fsample], lf[fsample]
            legs = {}
            for th in counts:
                med, n = timed_median(lambda: port.moe_forward_f32(xf, lf, 4, gb, gs, ub, us, db,
                                                                   ds, threads=th),
                                      seconds, least=1)
                legs[str(th)] = {"tokens_per_s": round(len(fsample) / med, 2),
                                 "ms": round(med * 1e3, 2), "runs": n}
            out[name + "_f32"] = {"kind": "port", "unit": "tokens/s", "by_threads": legs,
                                  "sample": f"tokens 0..{len(fsample) - 1}, AVX2 fp32 products"}
        del gb, gs, ub, us, db, ds
    return out


def cpu_model() -> dict:
    """The host CPU as lscpu reports it: model name, sockets, physical cores and logical
    CPUs of the machine, and the logical CPUs this process may run on."""
    info = {"model": "unknown", "sockets": None, "physical_cores": None,
            "logical_cpus": os.cpu_count()}
    try:
        import subprocess
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(line.split(":", 1) for line in text.splitlines() if ":" in line)
        fields = {k.strip(): v.strip() for k, v in fields.items()}
        info["model"] = fields.get("Model name", info["model"])
        parsable = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True,
                                  text=True, timeout=10).stdout
        rows = [r.split(",") for r in parsable.splitlines() if r and not r.startswith("#")]
        info["logical_cpus"] = len(rows)
        info["physical_cores"] = len({(r[2], r[1]) for r in rows})
        info["sockets"] = len({r[2] for r in rows})
    except (OSError, ValueError, IndexError):
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        info["model"] = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    try:
        info["allowed_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        info["allowed_cpus"] = info["logical_cpus"]
    return info


def bench_gemv(torch, encoding, n_in, n_out, steps, warmup, seed, copies=16, per_step=1,
               packed=True):
    """ms per step.  A step is one kdq_gemv_packed_batch submission (kdq_gemv_batch with
    packed=False) of `per_step` jobs over distinct weight copies (rotated through `copies`)
    that share one input and write separate outputs; the library runs a submission of one
    shape as one launch.  Packed weights are the resident form the host layer's bank
    keeps (kdq_gguf_pack, done once per copy outside the timed region).  The host
    enqueues submissions faster than the GPU retires them (a ctypes call and a launch
    take less than a kernel), so the events time the kernels rather than Python."""
    import ctypes
    import kadan_amd
    from kadan_amd import ops, synth
    w = synth.gguf_weights(encoding, seed, n_out, n_in)
    ws = rotated_copies(torch, w, copies, keep_mask(encoding, w.shape), seed)
    if packed:
        ws = [ops.gguf_pack(encoding, c, n_in) for c in ws]
        torch.cuda.synchronize()
    x = torch.from_numpy(synth.normal(seed, 50, n_in).reshape(1, n_in)).cuda()
    ys = [torch.empty(1, n_out, device="cuda") for _ in range(per_step)]
    tables = []
    for first in range(0, copies - per_step + 1, per_step):
        table = (kadan_amd.MatvecJob * per_step)()
        for k in range(per_step):
            wc = ws[first + k]
            table[k] = kadan_amd.MatvecJob(wc.data_ptr(), x.data_ptr(), ys[k].data_ptr(), 0,
                                           0 if packed else wc.shape[1], n_out, n_in, n_out,
                                           1, encoding)
        tables.append(table)
    addresses = [ctypes.addressof(t) for t in tables]
    fn = kadan_amd.lib().kdq_gemv_packed_batch if packed else kadan_amd.lib().kdq_gemv_batch
    stream = torch.cuda.current_stream().cuda_stream

    issued = [0]  # rotation continues across calls, so every copy is 15 launches old

    def submit(n):
        for _ in range(n):
            status = fn(addresses[issued[0] % len(addresses)], per_step, stream)
            issued[0] += 1
            if status:
                kadan_amd.check("kdq_gemv_packed_batch" if packed else "kdq_gemv_batch", status)

    submit(max(warmup, MIN_WARMUP))
    return time_steps(torch, submit, steps)


def bench_read_ceiling(torch, nbytes: int, steps: int, copies: int = 16,
                       shapes=((256, 1024), (256, 2048), (256, 4096), (1024, 256),
                               (1024, 512), (1024, 1024))):
    """The HBM read ceiling at the headline's size: kdq_hbm_read (a plain streaming read,
    16-byte non-temporal loads) over `copies` distinct buffers of `nbytes` each (the
    headline's per-launch bytes, rotated the same way), timed by time_steps exactly as
    the headline is, at several launch shapes, in both forms: every workgroup storing
    its fold (a kernel with output) and the read alone (no store on the critical path).
    The fastest shape of each form is its ceiling.  A single read of 64x the size gives
    the streaming rate without the per-launch cost.  kdq_hbm_read is the least a reader
    can do; ms/gbs are the form that stores a word per workgroup, as every kernel with
    output must, so the headline GEMV's time over that time is its distance from reading
    its bytes once and writing its result."""
    import kadan_amd
    from kadan_amd import ops
    nbytes = (nbytes + 15) // 16 * 16
    bufs = [torch.full((nbytes,), c, dtype=torch.uint8, device="cuda") for c in range(copies)]
    sink = torch.zeros(max(w for _, w in shapes), dtype=torch.int32, device="cuda")
    ops.hbm_read(bufs[0], sink, shapes[0][1], shapes[0][0])  # checked once through ops
    # launches as lean as the headline's (one ctypes call, arguments bound beforehand),
    # so the host enqueues faster than the kernels retire
    fn = kadan_amd.lib().kdq_hbm_read
    stream = torch.cuda.current_stream().cuda_stream
    pointers = [b.data_ptr() for b in bufs]
    sp = sink.data_ptr()
    never = 0x9E3779B9  # a constant-filled buffer folds to 0 or its fill word
    forms = {}
    for store_all in (1, 0):
        shape_ms = {}
        for threads, wg in shapes:
            issued = [0]

            def submit(n, wg=wg, threads=threads, store_all=store_all):
                for _ in range(n):
                    if fn(pointers[issued[0] % copies], nbytes, sp, wg, threads, store_all,
                          never, stream):
                        raise RuntimeError("kdq_hbm_read failed")
                    issued[0] += 1
            submit(MIN_WARMUP)
            shape_ms[f"{wg}x{threads}"] = time_steps(torch, submit, steps)
        best = min(shape_ms, key=shape_ms.get)
        gbs = nbytes / (shape_ms[best] * 1e-3) / 1e9
        forms["with_store" if store_all else "read_only"] = {
            "ms": round(shape_ms[best], 6), "gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "best_shape": best}
    del bufs
    big = torch.ones(64 * nbytes // 4, dtype=torch.int32, device="cuda")
    ops.hbm_read(big, sink, 4096)
    big_ms = time_launches(torch, lambda i: ops.hbm_read(big, sink, 4096), 10, 5)
    del big
    torch.cuda.empty_cache()
    store = forms["with_store"]
    return {"workload": f"HBM read ceiling, {nbytes} B/launch, {copies} buffers",
            "ms": store["ms"], "gbs": store["gbs"], "hbm_frac": store["hbm_frac"],
            "read_only": forms["read_only"], "best_shape": store["best_shape"],
            "streaming_gbs": round(64 * nbytes / (big_ms * 1e-3) / 1e9, 1)}


def calibrate_copy(torch, mib: int = 256, count: int = 5):
    """A plain device copy of known size, for scaling the FETCH_SIZE/WRITE_SIZE counters
    of a profiling run of this command (not part of the JSON line)."""
    src = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(count):  # an elementwise kernel that reads and writes `mib` MiB
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()


def bench_gemm(torch, reps=10, count=20, packed=True):
    from kadan_amd import ops, synth
    m, k, n = 512, 4096, 14336
    w = synth.q4_0_weights(0xC3, n, k)
    ws = rotated_copies(torch, w, 16, keep_mask(Q4_0, w.shape), 0xC3)
    if packed:  # the resident form the weight bank keeps (shared with the decode GEMV)
        ws = [ops.gguf_pack(Q4_0, wi, k) for wi in ws]
    x = torch.from_numpy(synth.normal(0xC3, 9, m * k).reshape(m, k).astype(np.float16)).cuda()
    y = torch.empty(m, n, dtype=torch.float16, device="cuda")
    if packed:
        launch = lambda i: ops.gemm_q4_0_packed(ws[i % 16], x, n, out=y)
    else:
        launch = lambda i: ops.gemm_q4_0(ws[i % 16], x, n, out=y)
    for i in range(5):
        launch(i)
    ms = time_launches(torch, launch, count, reps)
    flops = 2.0 * m * k * n
    tflops = flops / (ms * 1e-3) / 1e12
    layout = "tile-packed" if packed else "row-major"
    return {"workload": f"C3 Q4_0 GEMM M512 K4096 N14336, {layout}; quantize + GEMM",
            "ms": round(ms, 4), "tflops": round(tflops, 2),
            "mfma_frac": round(tflops / FP16_PEAK_TFLOPS, 4)}


def bench_gemm_gguf(torch, encoding, k, n, m=512, reps=10, count=20, copies=8):
    """Prefill GEMM for a kadan encoding (kdq_gemm_packed over the tile-packed bank copy):
    one 512-token chunk x fp32 [m, k] -> fp32 [m, n]; per launch the activation staging
    kernel and the GEMM."""
    from kadan_amd import ops, synth
    w = synth.gguf_weights(encoding, 0xD0 + encoding, n, k)
    ws = [ops.gguf_pack(encoding, wi, k)
          for wi in rotated_copies(torch, w, copies, keep_mask(encoding, w.shape), 0xD0)]
    x = torch.from_numpy(synth.normal(0xD0, 9, m * k).reshape(m, k)).cuda()
    y = torch.empty(m, n, dtype=torch.float32, device="cuda")
    launch = lambda i: ops.gemm_packed(encoding, ws[i % copies], x, n, out=y)
    for i in range(5):
        launch(i)
    ms = time_launches(torch, launch, count, reps)
    tflops = 2.0 * m * k * n / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "tflops": round(tflops, 2),
            "mfma_frac": round(tflops / FP16_PEAK_TFLOPS, 4)}


def bench_gemm_rows(torch, encoding, k, n, m=512, reps=10, count=20, copies=4):
    """Prefill GEMM over row-major GGUF rows (kdq_gemm_rows), the encodings that have no
    tile-packed form: one 512-token chunk x fp32 [m, k] -> fp32 [m, n]; per launch the
    activation staging kernel and the GEMM.  BF16 weights are random bits with a fixed
    exponent (the timing does not depend on the values; the seeded normal generator
    takes half a minute at this size)."""
    from kadan_amd import ops, synth
    if encoding == BF16:
        bits = synth.random_bytes(0xD0, 1, n * k * 2).view(np.uint16)
        w = ((bits & np.uint16(0x807F)) | np.uint16(0x3C00)).view(np.uint8).reshape(n, 2 * k)
    else:
        w = synth.gguf_weights(encoding, 0xD0 + encoding, n, k)
    ws = rotated_copies(torch, w, copies, keep_mask(encoding, w.shape), 0xD0)
    x = torch.from_numpy(synth.normal(0xD0, 9, m * k).reshape(m, k)).cuda()
    y = torch.empty(m, n, dtype=torch.float32, device="cuda")
    launch = lambda i: ops.gemm_rows(encoding, ws[i % copies], x, n, out=y)
    for i in range(5):
        launch(i)
    ms = time_launches(torch, launch, count, reps)
    tflops = 2.0 * m * k * n / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "tflops": round(tflops, 2),
            "mfma_frac": round(tflops / FP16_PEAK_TFLOPS, 4),
            "weight_gbps": round(gemv_bytes(k, n, encoding) / (ms * 1e-3) / 1e9, 1)}


def bench_moe_gguf(torch, rows, reps=10, count=64, resident=False):
    """The GGUF MoE layer (kdq_moe_gguf) at Qwen3-30B-A3B's geometry: hidden 2048, 128
    experts, top-8, expert ff 768, a 768-wide shared expert; Q4_K expert gate/up, Q6_K
    expert down, Q8_0 shared gate/up, Q4_K shared down, an fp32 router.  Each launch takes
    the next of 64 inputs and the next of 2 weight copies (392 MB of experts each), so the
    routed experts change between calls and the Infinity Cache cannot hold what they
    read.  resident: the copies' tile-packed forms are made once, outside the timed
    region, and every call reads them (kdq_moe_gguf_packed, as over a weight bank)."""
    from kadan_amd import ops, row_bytes, synth
    H, E, K, F, S = 2048, 128, 8, 768, 768
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    g = np.random.default_rng(0xE3)
    spec = dict(hidden=H, experts=E, top_k=K, ff=F, shared_ff=S,
                shared_gate=dev((g.standard_normal(H) * 0.05).astype(np.float32)),
                router=(0, dev((g.standard_normal((E, H)) * 0.1).astype(np.float32)
                               .view(np.uint8).reshape(E, -1))))
    encs = {"gate_exps": (Q4_K, (E, F, H)), "up_exps": (Q4_K, (E, F, H)),
            "down_exps": (Q6_K, (E, H, F)), "gate_shexp": (Q8_0, (S, H)),
            "up_shexp": (Q8_0, (S, H)), "down_shexp": (Q4_K, (H, S))}
    specs = [dict(spec), dict(spec)]
    for i, (name, (enc, shape)) in enumerate(encs.items()):
        w = synth.gguf_weights(enc, 0xE30 + i, int(np.prod(shape[:-1])), shape[-1])
        for c, wc in enumerate(rotated_copies(torch, w, 2, keep_mask(enc, w.shape), 0xE30 + i)):
            specs[c][name] = (enc, wc.reshape(*shape[:-1], -1))
    inputs = 64 if rows <= 8 else 4  # a prefill chunk touches every expert anyway
    xs = [dev(synth.normal(0xE4 + i, 1, rows * H).reshape(rows, H)) for i in range(inputs)]
    packs = [ops.moe_gguf_pack(sp) if resident else None for sp in specs]
    launch = lambda i: ops.moe_gguf(specs[i % 2], xs[i % inputs], packed=packs[i % 2])
    for i in range(5):
        launch(i)
    ms = time_launches(torch, launch, count, reps)
    per_call = np.mean([len(set(launch(i)[1].cpu().numpy().ravel().tolist()))
                        for i in range(inputs)])
    expert = 2 * F * row_bytes(Q4_K, H) + H * row_bytes(Q6_K, F)
    shared = 2 * S * row_bytes(Q8_0, H) + H * row_bytes(Q4_K, S)
    nbytes = per_call * expert + shared + E * H * 4 + H * 4 + 2 * rows * H * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    path = ("expert GEMVs" if rows <= 8 else
            "8-row items" if rows * 8 < 4 * 128 else "64-row GEMM tiles")
    if resident:
        path += ", resident"
    return {"workload": f"GGUF MoE Qwen3-30B-A3B rows={rows} ({path})",
            "ms": round(ms, 4), "experts_touched_per_call": round(float(per_call), 1),
            "algorithmic_bytes": int(nbytes), "gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def moe_bytes(tokens, hidden, inter, experts_touched):
    per_expert = 3 * inter * hidden // 2 + 3 * inter * hidden // 32
    return experts_touched * per_expert + tokens * hidden * 2 + tokens * hidden * 4


def bench_moe(torch, tokens, experts, hot, seed, copies, reps=10, count=10, inputs=1):
    """The MXFP4 MoE layer over `copies` resident weight sets.  With inputs > 1 the
    launches cycle through that many token batches whose routing is steered to disjoint
    expert groups (input i boosts experts [i * top_k, (i + 1) * top_k) mod experts), so
    consecutive decode calls touch different experts, as real decode steps do, and the
    weights they read (copies x experts x 13.2 MB) stay far beyond the 256 MB Infinity
    Cache.  Weights are packed once, outside the timed region; the products run on the
    scaled MFMA (FP4 E2M1 weights with their E8M0 scales as they lie, activations as FP8
    E4M3 terms with E8M0 block scales).  One token takes the two-launch single-token
    path; more take route, permute, gather, grouped gate/up and down GEMMs, combine."""
    from kadan_amd import ops, synth
    hidden = inter = 2880
    top_k = 4
    batches = []
    for i in range(inputs):
        x, logits = synth.moe_inputs(seed + i, tokens, hidden, experts, hot=hot)
        if inputs > 1:
            logits[:, [(i * top_k + j) % experts for j in range(top_k)]] += np.float32(8.0)
        batches.append((x, logits))
    (gb, gs), (ub, us), (db, ds) = synth.moe_weights(seed, experts, hidden, inter)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    sets = []  # resident weights: packed once, as the host layer's bank keeps them
    for c in range(copies):
        arrays = [dev(a) for a in (gb, gs, ub, us, db, ds)]
        if c:
            g = torch.Generator(device="cuda")
            g.manual_seed(seed + c)
            for i in (0, 2, 4):  # code bytes only; scales unchanged
                arrays[i] ^= torch.randint(0, 256, arrays[i].shape, dtype=torch.uint8,
                                           device="cuda", generator=g)
        sets.append([ops.moe_mxfp4_pack(arrays[0], arrays[1], experts, inter, hidden),
                     ops.moe_mxfp4_pack(arrays[2], arrays[3], experts, inter, hidden),
                     ops.moe_mxfp4_pack(arrays[4], arrays[5], experts, hidden, inter)])
        del arrays
    del gb, gs, ub, us, db, ds
    xbs = [dev(x).view(torch.bfloat16) for x, _ in batches]
    lgs = [dev(lg) for _, lg in batches]
    y = torch.empty(tokens, hidden, device="cuda")
    launch = lambda i: ops.moe_mxfp4_packed(xbs[i % inputs], lgs[i % inputs], top_k, inter,
                                            *sets[i % copies], out=y)
    for i in range(3):
        launch(i)
    ms = time_launches(torch, launch, count, reps)
    touched = np.mean([len(np.unique(_route_host(lg, top_k))) for _, lg in batches])
    nbytes = moe_bytes(tokens, hidden, inter, touched)
    flops = 2.0 * tokens * top_k * 3 * hidden * inter
    gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    del sets
    torch.cuda.empty_cache()
    cycle = "" if inputs == 1 else f", {inputs} inputs routed to disjoint experts"
    return {"workload": f"MXFP4 MoE H=I=2880 E={experts} top-4 T={tokens}"
                        + (" skewed" if hot else "") + f" ({copies} weight copies{cycle})",
            "ms": round(ms, 4), "tokens_per_s": round(tokens / (ms * 1e-3), 1),
            "experts_touched": round(float(touched), 2), "algorithmic_bytes": int(nbytes),
            "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tflops": round(tflops, 2),
            "fp4_mfma_frac": round(tflops / FP4_PEAK_TFLOPS, 5),
            "bf16_mfma_frac": round(tflops / FP16_PEAK_TFLOPS, 4)}


LAST_LINES = ("gemm_q4_k_prefill_4096x14336", "moe_gguf_t1_resident", "hbm_read_ceiling",
              "c1_q8_0_gemv_4096x4096", "c2_q4_k_gemv_14336_to_4096", "c3_q4_0_gemm",
              "c4_moe_t1", "c4_moe_t256", "c5_moe_t2048_skewed")


def _route_host(logits, top_k):
    """Experts touched by a routing (argsort on logits; only counts distinct experts)."""
    return np.argsort(-logits, axis=1, kind="stable")[:, :top_k]


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (the path runs on one "
                          "MI355X with no sharding); run with --gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    import kadan_amd
    kadan_amd.lib()

    if args.calibrate_copy:
        calibrate_copy(torch)
    n_in, n_out = 4096, 14336
    ms = bench_gemv(torch, Q4_K, n_in, n_out, args.steps, args.warmup, 0xC2A)
    nbytes = gemv_bytes(n_in, n_out, Q4_K)
    gbs = nbytes / (ms * 1e-3) / 1e9
    workload = "C2 Q4_K GEMV 4096->14336 batch 1"
    result = {
        "metric": "Q4_K GEMV weight GB/s (% HBM peak); MXFP4 MoE layer tokens/s (% MFMA peak)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "launches_timed": timed_launches(args.steps),
        "warmup_launches": max(args.warmup, MIN_WARMUP),
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x f32 (int8 MFMA on 16-bit block fixed-point activations, f32 accumulate)",
        "data": "synthetic (seeded SplitMix64 GGUF blocks, 16 rotated weight copies, "
                "resident in the tile-packed layout)",
        "config": {"workload": workload, "n_in": n_in, "n_out": n_out, "batch": 1,
                   "weight_copies": 16, "layout": "tile-packed (kdq_gguf_pack)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for(workload),
                     "algorithmic_bytes": nbytes},
        # the peaks every fraction in "extra" is taken against (mfma_frac: fp16 MFMA)
        "peaks": {"hbm_gbs": HBM_PEAK_GBS, "fp16_tflops": FP16_PEAK_TFLOPS,
                  "fp4_tflops": FP4_PEAK_TFLOPS},
    }
    if not args.skip_extra:
        extra = {}
        want = (lambda name: True) if not args.only else (lambda name: name in args.only)

        def gemv_line(name, enc, a, b, seed, steps, workload=None, **kw):
            if not want(name):
                return
            t = bench_gemv(torch, enc, a, b, steps, 20, seed, **kw)
            per = kw.get("per_step", 1)
            nb = per * gemv_bytes(a, b, enc) - (per - 1) * 4 * a  # one shared input
            line = {"ms": round(t, 6), "gbs": round(nb / (t * 1e-3) / 1e9, 1),
                    "hbm_frac": round(nb / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            if workload:
                line = {"workload": workload, **line}
            extra[name] = line

        if want("hbm_read_ceiling"):
            extra["hbm_read_ceiling"] = bench_read_ceiling(torch, nbytes, args.steps)
        # (name, encoding, in, out, seed, launches, note, options); "row-major" lines read
        # the GGUF rows in place (kdq_gemv_batch), the others the tile-packed bank copy
        gemv_line("c1_q8_0_gemv_4096x4096", Q8_0, 4096, 4096, 0xC1, 1000,
                  "C1 Q8_0 GEMV 4096x4096, tile-packed, 32 copies", copies=32)
        gemv_line("c2_q4_k_gemv_14336_to_4096", Q4_K, 14336, 4096, 0xC2B, 1000,
                  "C2 Q4_K GEMV 14336->4096, tile-packed, 16 copies")
        gemv_line("c2_q4_k_gemv_row_major", Q4_K, n_in, n_out, 0xC2A, 1000, "row-major",
                  packed=False)
        gemv_line("c2_q4_k_gate_up_pair", Q4_K, n_in, n_out, 0xC2C, 1000,
                  "gate+up in one launch", per_step=2)
        for enc, tag, a_, b_, packed in (
                (Q6_K, "q6_k", n_in, n_out, False), (Q6_K, "q6_k", n_in, n_out, True),
                (Q6_K, "q6_k", 14336, 4096, False), (IQ4_XS, "iq4_xs", n_in, n_out, False),
                (IQ4_NL, "iq4_nl", n_in, n_out, False), (Q3_K, "q3_k", n_in, n_out, False),
                (IQ3_XXS, "iq3_xxs", n_in, n_out, False), (IQ3_S, "iq3_s", n_in, n_out, False),
                (IQ2_S, "iq2_s", n_in, n_out, False)):
            name = (f"gemv_{tag}_4096x14336" if a_ == n_in else f"gemv_{tag}_14336_to_4096")
            gemv_line(name + ("_packed" if packed else ""), enc, a_, b_,
                      0xF0 + enc + (a_ != n_in), 1000, "packed" if packed else "row-major",
                      packed=packed, copies=8)
        gemv_line("gemv_bf16_4096x14336_exact", BF16, n_in, n_out, 0xF0 + BF16, 1000,
                  "row-major, exact-decode product", packed=False, copies=4)
        if want("c3_q4_0_gemm"):
            extra["c3_q4_0_gemm"] = bench_gemm(torch)
        for enc, tag in ((Q4_K, "q4_k"), (Q8_0, "q8_0"), (Q6_K, "q6_k")):
            for k_, n_ in ((4096, 14336), (14336, 4096)):
                name = f"gemm_{tag}_prefill_{k_}x{n_}"
                if want(name):
                    extra[name] = bench_gemm_gguf(torch, enc, k_, n_)
        for enc, tag in ((IQ4_XS, "iq4_xs"), (IQ4_NL, "iq4_nl"), (Q3_K, "q3_k"),
                         (IQ3_XXS, "iq3_xxs"), (IQ3_S, "iq3_s"), (IQ2_S, "iq2_s"),
                         (BF16, "bf16")):
            name = f"gemm_rows_{tag}_prefill_4096x14336"
            if want(name):
                extra[name] = bench_gemm_rows(torch, enc, 4096, 14336)
        if want("c3_q4_0_gemm_row_major"):
            extra["c3_q4_0_gemm_row_major"] = bench_gemm(torch, packed=False)
        if want("moe_gguf_t1"):
            extra["moe_gguf_t1"] = bench_moe_gguf(torch, 1)
        if want("moe_gguf_t4"):
            extra["moe_gguf_t4"] = bench_moe_gguf(torch, 4)
        if want("moe_gguf_t64"):
            extra["moe_gguf_t64"] = bench_moe_gguf(torch, 64, count=16)
        if want("moe_gguf_t1_resident"):
            extra["moe_gguf_t1_resident"] = bench_moe_gguf(torch, 1, resident=True)
        if want("moe_gguf_t4_resident"):
            extra["moe_gguf_t4_resident"] = bench_moe_gguf(torch, 4, resident=True)
        if want("moe_gguf_t64_resident"):
            extra["moe_gguf_t64_resident"] = bench_moe_gguf(torch, 64, count=16, resident=True)
        if want("moe_gguf_t512"):
            extra["moe_gguf_t512"] = bench_moe_gguf(torch, 512, reps=5, count=8)
        if want("moe_gguf_t512_resident"):
            extra["moe_gguf_t512_resident"] = bench_moe_gguf(torch, 512, reps=5, count=8,
                                                             resident=True)
        if want("c4_moe_t1"):
            extra["c4_moe_t1"] = bench_moe(torch, 1, 32, 0, 0xC4, copies=3, count=48,
                                           inputs=8)
        if want("c4_moe_t256"):
            extra["c4_moe_t256"] = bench_moe(torch, 256, 32, 0, 0xC4, copies=2)
        if want("c5_moe_t2048_skewed"):
            extra["c5_moe_t2048_skewed"] = bench_moe(torch, 2048, 128, 8, 0xC5, copies=1,
                                                     reps=5, count=5)
    if not args.skip_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        if not args.skip_extra:
            result["cpu_baselines"] = cpu_baselines()
    if not args.skip_extra:
        # the benchmark's own configurations and the read ceiling last, so a reader that
        # keeps only the end of the line still has them
        last = [k for k in LAST_LINES if k in extra]
        result["extra"] = {**{k: v for k, v in extra.items() if k not in last},
                           **{k: extra[k] for k in last}}
    print(json.dumps(result, separators=(",", ":")))


if __name__ == "__main__":
    main()

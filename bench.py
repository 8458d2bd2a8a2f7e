#!/usr/bin/env python3
"""Benchmark of the ipu-stack hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): fp16 GEMM C = A.B at
M = N = K = 8192, A, B ~ U[-1, 1] fp16, fp32 accumulation, fp16 output.  A
"step" is one such GEMM over inputs resident in HBM.  The other BASELINE
configurations are measured in the same run and reported under "results":
fp32 GEMM 4096^3, flash attention (causal S4096, non-causal S2048, B8 H16
D128), the memory chain (transpose, block-major 64x64, row reduce on
X[8192, 8192]), GELU on the MLP hidden [4096, 16384], the MLP graph through
build_package, and the 256^3 GEMM of configs[0].

Timing: the headline runs SETTLE_LAUNCHES untimed launches (the board's power
controller needs ~30-50 ms of load to settle), W warmups and a
synchronisation, then exactly K launches back to back between two HIP events
on the library's stream;
`value`, `ms_per_step` and `roofline.achieved` come from the region's time
over K (the average launch duration that rocprof's kernel trace reports for
the same run).  results{} adds the median of 5 such regions and the median
launch of K launches timed one by one (an event before each; both after
their own settle launches).  The other legs time 5 regions of back-to-back launches
between two events each and report the median region; the MFMA legs (fp32
GEMM, attention, MLP graph) run settle launches first as the headline does.
Bandwidth kernels rotate 3 buffer sets (768 MiB > the 256 MiB MALL).  One
JSON line on stdout.

Other modes turn rocprofv3 output of a bench run into the committed
summaries under profiles/ through the package's own rocprof ingestion
(ipu-stack_amd/profiling.py): --summarize-trace (kernel durations per kernel,
warmup launches excluded), --summarize-traffic (HBM bytes per launch from
FETCH_SIZE / WRITE_SIZE, scaled by the plain copy kernel's counters) and
--summarize-counters (shader clock and MFMA-pipe utilisation per kernel).
"""
from __future__ import annotations

import argparse
import glob
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

PEAK_FP16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 dense fp16 flop/clk/CU
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0
METRIC = "fp16 GEMM + flash-attn TFLOP/s (% MI355X peak), rearrange GB/s; 1 GPU"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Timing(dict):
    """Per-launch milliseconds of one timed region: median, mean, min, max."""

    @property
    def median(self) -> float:
        return self["median_ms"]

    @property
    def mean(self) -> float:
        return self["mean_ms"]


def timed(ctx, fn, steps: int, warmup: int, per_launch: bool = False,
          repeats: int = 5, settle: int = 0) -> Timing:
    """`warmup` untimed calls of `fn` (which enqueues on the stream) and a
    synchronisation, then timed calls on HIP events.  per_launch: `steps`
    calls with an event before each and after the last, so each call has its
    own duration.  Otherwise `repeats` regions of `steps` back-to-back calls
    between two events each (the headline: one region of exactly K steps),
    so short kernels carry no per-launch event gaps; the median is over the
    regions' per-call means.  `settle` untimed calls and a synchronisation
    come first (MFMA legs: the board's power controller needs ~30-50 ms of
    load after idle to settle; see SETTLE_LAUNCHES)."""
    for _ in range(settle):
        fn(0)
    ctx.sync()
    for _ in range(warmup):
        fn(0)
    ctx.sync()
    if per_launch:
        events = ctx.event_series(steps + 1)
        for i in range(steps):
            events.record(i)
            fn(i)
        events.record(steps)
        d = np.asarray(events.durations(), dtype=np.float64)
        ctx.sync()
        events.close()
        return Timing(median_ms=float(np.median(d)), mean_ms=float(d.mean()),
                      min_ms=float(d.min()), max_ms=float(d.max()), launches=int(d.size))
    regions = []
    for r in range(repeats):
        events = ctx.event_series(2)
        events.record(0)
        for i in range(steps):
            fn(r * steps + i)
        events.record(1)
        regions.append(events.durations()[0] / steps)
        ctx.sync()
        events.close()
    d = np.asarray(regions, dtype=np.float64)
    return Timing(median_ms=float(np.median(d)), mean_ms=float(d.mean()), min_ms=float(d.min()),
                  max_ms=float(d.max()), launches=steps * repeats)


def leg_entry(t: Timing, work: float, unit: str, peak: float) -> dict:
    """A results{} entry: rate from the median launch, its fraction of the
    spec peak, and the mean launch."""
    scale = 1e12 if unit == "tflops" else 1e9
    rate = work / (t.median * 1e-3) / scale
    return {"ms": round(t.median, 5), "ms_mean": round(t.mean, 5), unit: round(rate, 2),
            "frac_peak": round(rate / peak, 4)}


def gemm_scalars(n, m=None, k=None):
    m = m or n
    k = k or n
    return [1, m, n, k, 0, 0, 0, 0]


def bench_gemm_f16(ipus, ctx, n, steps, warmup, per_launch=False, repeats=5, settle=0,
                   tl=False, tr=False):
    """`settle` untimed launches and a synchronisation before timed()'s own
    warmups (the headline's settle phase); tl / tr: A and / or B stored
    transposed (the same bytes read as the other layout)."""
    a = ctx.upload(ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM))
    b = ctx.upload(ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM))
    c = ctx.alloc(n * n * 2)
    sc = [1, n, n, n, int(tl), int(tr), 0, 0]
    fn = lambda i: ctx.launch("ipu_stack_gemm_f16", c, [a, b], sc)  # noqa: E731
    ms = timed(ctx, fn, steps, warmup, per_launch=per_launch, repeats=repeats, settle=settle)
    for x in (a, b, c):
        x.free()
    return ms


def bench_gemm_f16_graph(ipus, ctx, n, steps, warmup, copies=64):
    """Device time of one n^3 fp16 GEMM without the host's per-launch cost:
    a package of `copies` independent one-op GEMMs (one shared weight, as
    configs[0] runs it: a one-op ComputeGraph) is captured once as a HIP
    graph, each timed call replays it, and the time per GEMM is the replay's
    over `copies`."""
    g = ipus.ComputeGraph()
    w = g.parameter("w", [n, n])
    g.set_outputs([g.gemm(g.host_input(f"x{i}", [n, n]), w) for i in range(copies)])
    pkg = ipus.build_package(g, ipus.PackageConfig())
    sess = pkg.session(ctx)
    sess.write("w", ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM).reshape(n, n))
    for i in range(copies):
        sess.write(f"x{i}", ipus.synth_f16(n * n, 2024, 10 + i, ipus.UNIFORM).reshape(n, n))
    sess.capture()
    t = timed(ctx, lambda i: sess.run(), steps, warmup)
    sess.close()
    return Timing(median_ms=t.median / copies, mean_ms=t.mean / copies,
                  min_ms=t["min_ms"] / copies, max_ms=t["max_ms"] / copies, launches=t["launches"])


def bench_gemm_f32(ipus, ctx, n, steps, warmup, settle=0):
    a = ctx.upload(ipus.synth_f32(n * n, 4096, 1, ipus.NORMAL))
    b = ctx.upload(ipus.synth_f32(n * n, 4096, 2, ipus.NORMAL))
    c = ctx.alloc(n * n * 4)
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_gemm_f32", c, [a, b], gemm_scalars(n)),
               steps, warmup, settle=settle)
    for x in (a, b, c):
        x.free()
    return ms


def bench_attention(ipus, ctx, s, causal, steps, warmup, streams=128, d=128, settle=0):
    n = streams * s * d
    q = ctx.upload(ipus.synth_f16(n, 5, 1, ipus.NORMAL))
    k = ctx.upload(ipus.synth_f16(n, 5, 2, ipus.NORMAL))
    v = ctx.upload(ipus.synth_f16(n, 5, 3, ipus.NORMAL))
    o = ctx.alloc(n * 4)
    sc = [streams, s, s, d, d, 0, int(causal), 0]
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_flash_attention_online_f16", o, [q, k, v], sc),
               steps, warmup, settle=settle)
    for x in (q, k, v, o):
        x.free()
    return ms


def bench_memory_chain(ipus, ctx, steps, warmup, n=8192, sets=3):
    """Transpose, block-major (64x64) and row reduce on X[8192, 8192] fp16."""
    x = [ctx.upload(ipus.synth_f16(n * n, 77, 10 + s, ipus.NORMAL)) for s in range(sets)]
    t = [ctx.alloc(n * n * 2) for _ in range(sets)]
    bm = [ctx.alloc(n * n * 2) for _ in range(sets)]
    r = ctx.alloc(n * 4)
    out = {}
    out["copy"] = timed(
        ctx, lambda i: ctx.launch("ipu_stack_copy", t[i % sets], [x[i % sets]], [n * n * 2]),
        steps, warmup)
    out["transpose"] = timed(
        ctx, lambda i: ctx.launch("ipu_stack_transpose_f16", t[i % sets], [x[i % sets]], [1, n, n]),
        steps, warmup)
    out["block_major"] = timed(
        ctx, lambda i: ctx.launch("ipu_stack_rearrange_row_major_f16", bm[i % sets], [t[i % sets]],
                                  [n, n, ipus.ORDER_BLOCK_MAJOR, n, n, 64, 64, 1]),
        steps, warmup)
    out["reduce_rows"] = timed(
        ctx, lambda i: ctx.launch("ipu_stack_reduce_rows_f16", r, [bm[i % sets]],
                                  [n, n, ipus.ORDER_BLOCK_MAJOR, 64, 64]),
        steps, warmup)
    out["reduce_rows_row_major"] = timed(
        ctx, lambda i: ctx.launch("ipu_stack_reduce_rows_f16", r, [x[i % sets]],
                                  [n, n, ipus.ORDER_ROW_MAJOR, 0, 0]),
        steps, warmup)
    for b in x + t + bm + [r]:
        b.free()
    return out


def bench_amp_layouts(ipus, ctx, steps, warmup, n=8192, sets=3):
    """The reference's AMP storage conversions on X[8192, 8192] fp16:
    row-major -> AMP-Left and -> AMP-TransposedRight (rearrange_amp_left_f16,
    rearrange_transposed_right_f16), and unpack of AMP-Output and
    AMP-TransposedLeft back to row-major (unpack_amp_f16)."""
    x = [ctx.upload(ipus.synth_f16(n * n, 79, 20 + s, ipus.NORMAL)) for s in range(sets)]
    y = [ctx.alloc(n * n * 2) for _ in range(sets)]
    out = {}
    for name, order in (("rearrange_amp_left", 0), ("rearrange_amp_transposed_right", 1)):
        out[name] = timed(
            ctx, lambda i, o=order: ctx.launch("ipu_stack_rearrange_row_major_f16", y[i % sets],
                                               [x[i % sets]], [n, n, o, n, n, 32, 16, 1]),
            steps, warmup)
    for name, source in (("unpack_amp_output", 0), ("unpack_amp_transposed_left", 1)):
        out[name] = timed(
            ctx, lambda i, src=source: ctx.launch("ipu_stack_unpack_amp_f16", y[i % sets],
                                                  [x[i % sets]], [1, n, n, n, n, src]),
            steps, warmup)
    for b in x + y:
        b.free()
    return out


def bench_gelu(ipus, ctx, steps, warmup, rows=4096, cols=16384, sets=3):
    n = rows * cols
    x = [ctx.upload(ipus.synth_f16(n, 88, s, ipus.NORMAL)) for s in range(sets)]
    y = [ctx.alloc(n * 2) for _ in range(sets)]
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_gelu_tanh_approx_f16", y[i % sets],
                                         [x[i % sets]], [n]), steps, warmup)
    for b in x + y:
        b.free()
    return ms


def bench_mlp_graph(ipus, ctx, steps, warmup, settle=0):
    """configs[3] through ComputeGraph + build_package + session."""
    g = ipus.ComputeGraph()
    xin = g.host_input("input", [4096, 4096])
    w1 = g.parameter("w1", [4096, 16384])
    w2 = g.parameter("w2", [16384, 4096])
    g.set_outputs([g.gemm(g.gelu(g.gemm(xin, w1)), w2)])
    pkg = ipus.build_package(g)
    sess = pkg.session(ctx)
    sess.write("input", ipus.synth_f16(4096 * 4096, 9, 1, ipus.NORMAL).reshape(4096, 4096))
    sess.write("w1", ipus.synth_f16(4096 * 16384, 9, 2, ipus.NORMAL, 0.02).reshape(4096, 16384))
    sess.write("w2", ipus.synth_f16(16384 * 4096, 9, 3, ipus.NORMAL, 0.02).reshape(16384, 4096))
    ms = timed(ctx, lambda i: sess.run(), steps, warmup, settle=settle)
    sess.close()
    return ms


def mfma_calibration(ipus, ctx, blocks=1024, iterations=4096):
    """Sustained MFMA rate and shader clock with register-resident operands
    (no memory traffic), after settle launches (~60 ms of load, as the
    headline gets): v_mfma_f32_32x32x16_f16 on fragments drawn like the
    headline's inputs (U[-1, 1] fp16) and on all-zero fragments, and
    v_mfma_f32_16x16x32_f16 -- the form the GEMM and attention kernels
    issue -- on U[-1, 1] fragments that change from one MFMA to the next.
    The clock under dense MFMA falls with operand entropy (power limit), and
    the 16 x 16 x 32 form draws less power per flop, so the last figure is
    the tightest ceiling for the headline GEMM on this board."""
    out = {}
    uniform = ipus.synth_f16(4096 * 8, 2024, 3, ipus.UNIFORM)
    forms = (("uniform", "ipus_calibrate_mfma_f16", 32 * 32 * 16, uniform, 25),
             ("zeros", "ipus_calibrate_mfma_f16", 32 * 32 * 16, np.zeros(4096 * 8, dtype=np.float16), 25),
             ("uniform_16x16x32", "ipus_calibrate_mfma_f16_16x16x32", 16 * 16 * 32, uniform, 50))
    for name, symbol, macs, frags, settle in forms:
        ops = ctx.upload(frags)
        res = ctx.alloc(16 + blocks * 256 * 4)
        sc = [4096, iterations, blocks]
        t = timed(ctx, lambda i: ctx.launch(symbol, res, [ops], sc), 5, 1, repeats=1, settle=settle)
        clocks = res.download(np.uint64)[:2]
        flops = blocks * 4 * 8 * iterations * macs * 2.0
        mhz = clocks[0] / (clocks[1] / 100.0) if clocks[1] else 0.0
        out[name] = {"tflops": round(flops / (t.median * 1e-3) / 1e12, 1),
                     "clock_mhz": round(mhz)}
        ops.free()
        res.free()
    return out


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (a C restatement of the reference's
# diagnostic::evaluate, oracle/) timed on the host's cores, on rank 0 only.
# ---------------------------------------------------------------------------
def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_seconds(fn, min_seconds: float, max_reps: int = 20) -> tuple:
    times = []
    while not times or (sum(times) < min_seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times), float(sum(times))


def cpu_baseline(ipus, n=8192, min_seconds=10.0):
    """The headline workload on the CPU evaluator: the full 8192^3 fp16 GEMM
    (fp16 -> fp32 operands, blocked AVX2 sgemm, one fp16 rounding) repeated
    until at least `min_seconds`, median reported; then the other configs on
    bounded samples (each labelled), and configs[0] single-threaded."""
    from oracle import oracle
    threads = oracle.threads()
    a = ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM)
    b = ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM)
    dt, reps, total = _median_seconds(lambda: oracle.gemm_f16(a, b, n, n, n, nthreads=threads),
                                      min_seconds)
    del a, b
    out = {
        "value": round(2.0 * n ** 3 / dt / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "model": cpu_model(),
        "sample": f"full 8192^3 fp16 GEMM x{reps} (fp16->fp32 operands, blocked AVX2 sgemm, "
                  f"fp16 rounding), median {dt:.2f} s, total {total:.1f} s",
    }
    out["configs"] = cpu_configs(ipus, oracle, threads)
    return out


def cpu_configs(ipus, oracle, threads):
    """CPU times of the other BASELINE configs on the oracle, each on a
    bounded sample of the same workload, labelled."""
    res = {}
    # 256^3 fp16 GEMM, one thread and all threads.
    m = 256
    a = ipus.synth_f16(m * m, 7, 1, ipus.UNIFORM)
    b = ipus.synth_f16(m * m, 7, 2, ipus.UNIFORM)
    for label, th in (("single_thread", 1), ("threads", threads)):
        dt, reps, _ = _median_seconds(lambda: oracle.gemm_f16(a, b, m, m, m, nthreads=th), 1.0, 200)
        res[f"gemm_f16_256_{label}"] = {"ms": round(dt * 1e3, 3), "threads": th,
                                        "gflops": round(2.0 * m ** 3 / dt / 1e9, 2),
                                        "sample": f"full 256^3, median of {reps}"}
    # fp32 GEMM 4096^3 (full).
    n = 4096
    af = ipus.synth_f32(n * n, 4096, 1, ipus.NORMAL)
    bf = ipus.synth_f32(n * n, 4096, 2, ipus.NORMAL)
    dt, reps, _ = _median_seconds(lambda: oracle.gemm_f32(af, bf, n, n, n, nthreads=threads), 2.0, 5)
    res["gemm_f32_4096"] = {"ms": round(dt * 1e3, 1), "tflops": round(2.0 * n ** 3 / dt / 1e12, 4),
                            "sample": f"full 4096^3, median of {reps}"}
    del af, bf
    # MLP 4096 x 4096 . 4096 x 16384 -> GELU -> . 16384 x 4096 (full).
    x = ipus.synth_f16(4096 * 4096, 9, 1, ipus.NORMAL)
    w1 = ipus.synth_f16(4096 * 16384, 9, 2, ipus.NORMAL, 0.02)
    w2 = ipus.synth_f16(16384 * 4096, 9, 3, ipus.NORMAL, 0.02)
    t0 = time.perf_counter()
    h = oracle.gelu_f16(oracle.gemm_f16(x, w1, 4096, 16384, 4096, nthreads=threads))
    oracle.gemm_f16(h, w2, 4096, 4096, 16384, nthreads=threads)
    dt = time.perf_counter() - t0
    res["mlp"] = {"ms": round(dt * 1e3, 1), "tflops": round(2 * 2.0 * 4096 * 4096 * 16384 / dt / 1e12, 4),
                  "sample": "full MLP once (two GEMMs and the GELU)"}
    del x, w1, w2, h
    # the memory chain on X[8192, 8192] (full).
    n = 8192
    xs = ipus.synth_f16(n * n, 77, 10, ipus.NORMAL)
    t0 = time.perf_counter()
    tr = oracle.transpose_u16(xs, 1, n, n)
    t1 = time.perf_counter()
    bm = oracle.rearrange_row_major_f16(tr, ipus.ORDER_BLOCK_MAJOR, 1, n, n, n, n, 64, 64)
    t2 = time.perf_counter()
    oracle.reduce_rows_block_major_f16(bm, 64, 64, n, n, nthreads=threads)
    t3 = time.perf_counter()
    for key, sec, nbytes in (("transpose", t1 - t0, 4 * n * n), ("block_major", t2 - t1, 4 * n * n),
                             ("reduce_rows", t3 - t2, 2 * n * n + 4 * n)):
        res[key] = {"ms": round(sec * 1e3, 1), "gbps": round(nbytes / sec / 1e9, 2),
                    "sample": "full 8192^2 once"}
    del xs, tr, bm
    # attention B8 H16 D128 on evenly spaced query rows of every
    # stream, extrapolated to all rows (labelled as such).
    streams, d = 128, 128
    for causal, s in ((True, 4096), (False, 2048)):
        nq = streams * s * d
        q = oracle.f16_to_f32(ipus.synth_f16(nq, 5, 1, ipus.NORMAL))
        k = oracle.f16_to_f32(ipus.synth_f16(nq, 5, 2, ipus.NORMAL))
        v = oracle.f16_to_f32(ipus.synth_f16(nq, 5, 3, ipus.NORMAL))
        per_stream = 8
        rows = np.array([st * s + r for st in range(streams)
                         for r in np.linspace(0, s - 1, per_stream).astype(np.int64)], np.uint32)
        t0 = time.perf_counter()
        oracle.attention(q, k, v, streams, s, s, d, d, causal, row_list=rows, nthreads=threads)
        dt = (time.perf_counter() - t0) * (streams * s) / rows.size
        fl = 4.0 * streams * d * (s * (s + 1) / 2 if causal else s * s)
        key = f"attention_{'causal' if causal else 'noncausal'}_s{s}"
        res[key] = {"ms": round(dt * 1e3, 1), "tflops": round(fl / dt / 1e12, 5),
                    "sample": f"{rows.size} evenly spaced query rows ({per_stream} per stream), "
                              f"time extrapolated x{streams * s // rows.size} to every row"}
        del q, k, v
    return res


# ---------------------------------------------------------------------------
# roofline.traffic: HBM bytes per launch from the committed rocprofv3 --pmc
# summary, used only when it was measured on the current kernel sources.
# ---------------------------------------------------------------------------
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "gemm_f16_8192_traffic.json")
GEMM_SOURCES = ("ipu-stack_amd/csrc/k_gemm_f16.hip", "ipu-stack_amd/csrc/device_common.h")


def source_digest(paths=GEMM_SOURCES) -> str:
    h = hashlib.sha256()
    for rel in paths:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def committed_traffic():
    """(bytes per launch, note): the traffic summary's figure if its kernel
    source digest equals the current sources', else (None, why)."""
    if not os.path.exists(TRAFFIC_JSON):
        return None, "no traffic summary"
    with open(TRAFFIC_JSON) as f:
        t = json.load(f)
    digest = source_digest()
    if t.get("kernel_source_digest") != digest:
        return None, (f"traffic summary measured on kernel sources {t.get('kernel_source_digest')}, "
                      f"current {digest}")
    return t.get("hbm_bytes_per_launch"), (
        f"profiles/gemm_f16_8192_traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of "
        f"the same kernel sources ({digest}), scaled by the copy kernel's counters")


def traffic_probe(ipus, ctx, n=8192, copy_bytes=256 << 20):
    """Untimed launches for the rocprofv3 --pmc passes that give
    roofline.traffic: the headline GEMM, then a plain 16-byte-vector copy of
    `copy_bytes` with ordinary loads and stores whose FETCH_SIZE / WRITE_SIZE
    calibrate the counters' unit (and the library's streaming copy, whose
    non-temporal accesses the counters weigh differently, for comparison)."""
    a = ctx.upload(ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM))
    b = ctx.upload(ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM))
    c = ctx.alloc(n * n * 2)
    for _ in range(3):
        ctx.launch("ipu_stack_gemm_f16", c, [a, b], gemm_scalars(n))
    ctx.sync()
    src, dst = ctx.alloc(copy_bytes), ctx.alloc(copy_bytes)
    ctx.memset(src, 1)
    for symbol in ("ipus_calibrate_copy", "ipu_stack_copy"):
        for _ in range(3):
            ctx.launch(symbol, dst, [src], [copy_bytes])
    ctx.sync()
    for x in (a, b, c, src, dst):
        x.free()
    log(f"traffic probe: 3x gemm_f16 {n}^3, 3x plain copy and 3x streaming copy of "
        f"{copy_bytes} B")


# ---------------------------------------------------------------------------
# Summaries of rocprofv3 output through the package's ProfileReport ingestion
# ---------------------------------------------------------------------------
def _profiling():
    __graft_entry__.import_package()
    import ipu_stack_amd.profiling as prof
    return prof


def _timed_phases(report, skip_per_kernel: int) -> frozenset:
    """Dispatch phases left after dropping each kernel's first
    `skip_per_kernel` dispatches (the warmups)."""
    seen = {}
    keep = set()
    for tile in report.tiles:
        for sample in sorted(tile.samples, key=lambda x: x.step.phase):
            k = sample.step.kernel
            seen[k] = seen.get(k, 0) + 1
            if seen[k] > skip_per_kernel:
                keep.add(sample.step.phase)
    return frozenset(keep)


def summarize_trace(directory: str, skip: int, command: str) -> str:
    prof = _profiling()
    report = prof.from_rocprof(directory)
    keep = _timed_phases(report, skip)
    q = prof.query(report, prof.Query(group_by=prof.GroupBy.KERNEL, phases=keep, shared_clock=True))
    lines = [f"Command (from the repository root, `export TMPDIR=/tmp`):", "",
             f"    {command}", "",
             f"Summary: `python bench.py --summarize-trace <trace dir> --skip {skip}` "
             f"(ipu-stack_amd/profiling.py: rocprofv3 kernel trace -> ProfileReport -> query "
             f"grouped by kernel); each kernel's first {skip} dispatches (warmups) are excluded.",
             "", "| kernel | dispatches | mean ns | p50 ns | p95 ns | max ns |",
             "|---|---|---|---|---|---|"]
    for g in q.groups:
        lines.append(f"| `{g.name}` | {g.sample_count} | {g.mean_cycles:.0f} | {g.p50_cycles} | "
                     f"{g.p95_cycles} | {g.maximum_cycles} |")
    return "\n".join(lines) + "\n"


def summarize_traffic(fetch_dir: str, write_dir: str, kernel: str, copy_kernel: str,
                      copy_bytes: int, algorithmic: float, skip: int, commands: list) -> dict:
    """HBM bytes per launch of `kernel` from FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by the factor that makes the copy kernel's counter
    equal its known bytes."""
    prof = _profiling()

    def per_kernel(directory, counter):
        report = prof.from_rocprof(counter_csv=directory)
        keep = _timed_phases(report, skip)
        vals = {}
        for tile in report.tiles:
            for smp in tile.samples:
                if smp.step.phase not in keep:
                    continue
                md = {m.name: m.value for m in smp.step.metadata}
                v = md.get(prof.COUNTER_PREFIX + counter)
                if v is not None:
                    vals.setdefault(smp.step.kernel, []).append(float(v) * 1024.0)
        return {k: float(np.mean(v)) for k, v in vals.items()}

    fetch = per_kernel(fetch_dir, "FETCH_SIZE")
    write = per_kernel(write_dir, "WRITE_SIZE")
    pick = lambda table, name: next(v for k, v in table.items() if k.startswith(name))  # noqa: E731
    f_scale = copy_bytes / pick(fetch, copy_kernel)
    w_scale = copy_bytes / pick(write, copy_kernel)
    fb, wb = pick(fetch, kernel) * f_scale, pick(write, kernel) * w_scale
    return {
        "kernel": kernel, "kernel_source_digest": source_digest(),
        "fetch_bytes_per_launch": round(fb), "write_bytes_per_launch": round(wb),
        "hbm_bytes_per_launch": round(fb + wb),
        "algorithmic_bytes_per_launch": algorithmic,
        "traffic_over_algorithmic": round((fb + wb) / algorithmic, 3),
        "counter_scale": {"FETCH_SIZE": round(f_scale, 4), "WRITE_SIZE": round(w_scale, 4),
                          "calibration": f"{copy_kernel} of {copy_bytes} bytes read and written"},
        "raw_bytes_per_dispatch": {"FETCH_SIZE": {k: round(v) for k, v in fetch.items()},
                                   "WRITE_SIZE": {k: round(v) for k, v in write.items()}},
        "commands": commands,
        "summary": "python bench.py --summarize-traffic <FETCH_SIZE dir> <WRITE_SIZE dir>",
    }


def summarize_traffic_table(fetch_dir: str, write_dir: str, skip: int, command: str,
                            copy_kernel: str = "copy_bytes_kernel",
                            copy_bytes: int = 8192 * 8192 * 2) -> str:
    """HBM bytes per dispatch of every kernel of a FETCH_SIZE and a WRITE_SIZE
    pass (KiB per dispatch, medians after each kernel's first `skip`
    dispatches), each scaled by the factor that makes `copy_kernel` (which
    reads and writes `copy_bytes`) read and write exactly its bytes."""
    prof = _profiling()

    def medians(directory, counter):
        report = prof.from_rocprof(counter_csv=directory)
        keep = _timed_phases(report, skip)
        vals = {}
        for tile in report.tiles:
            for smp in tile.samples:
                if smp.step.phase not in keep:
                    continue
                md = {m.name: m.value for m in smp.step.metadata}
                v = md.get(prof.COUNTER_PREFIX + counter)
                if v is not None:
                    vals.setdefault(smp.step.kernel, []).append(float(v))
        return {k: float(np.median(v)) for k, v in vals.items()}

    fetch, write = medians(fetch_dir, "FETCH_SIZE"), medians(write_dir, "WRITE_SIZE")
    f_scale = copy_bytes / (fetch[copy_kernel] * 1024.0)
    w_scale = copy_bytes / (write[copy_kernel] * 1024.0)
    lines = ["Commands (from the repository root, `export TMPDIR=/tmp`):", ""]
    lines += [f"    {c}" for c in command.split(" ;; ") if c]
    lines += ["", f"Summary: `python bench.py --summarize-traffic-table <FETCH_SIZE dir> "
              f"<WRITE_SIZE dir> --skip {skip}` (ipu-stack_amd/profiling.py's rocprof "
              f"ingestion); medians over each kernel's dispatches after its first {skip}.  "
              f"Scales from `{copy_kernel}` ({copy_bytes} bytes read and written): FETCH_SIZE "
              f"x {f_scale:.3f}, WRITE_SIZE x {w_scale:.3f}.", "",
              "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read MB | HBM write MB |",
              "|---|---|---|---|---|"]
    for k in sorted(set(fetch) & set(write)):
        lines.append(f"| `{k}` | {fetch[k]:.1f} | {write[k]:.1f} | "
                     f"{fetch[k] * 1024 * f_scale / 1e6:.2f} | {write[k] * 1024 * w_scale / 1e6:.2f} |")
    return "\n".join(lines) + "\n"


def summarize_counters(directory: str, skip: int, command: str, xcds: int = 8,
                       simds: int = 1024) -> str:
    """MFMA-pipe utilisation and shader clock per kernel from one rocprofv3
    --pmc pass holding SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE (and any
    other counters, reported as medians).  GRBM_GUI_ACTIVE is summed over the
    XCDs, so the shader clock is GRBM_GUI_ACTIVE / xcds / duration;
    SQ_VALU_MFMA_BUSY_CYCLES counts the matrix pipes' busy cycles over all
    SIMDs (16 per v_mfma_f32_16x16x32_f16, 32 per v_mfma_f32_32x32x16_f16),
    so the utilisation is that over shader cycles x SIMDs."""
    prof = _profiling()
    report = prof.from_rocprof(counter_csv=directory)
    keep = _timed_phases(report, skip)
    rows = {}
    for tile in report.tiles:
        for smp in tile.samples:
            if smp.step.phase not in keep:
                continue
            md = {m.name[len(prof.COUNTER_PREFIX):]: float(m.value) for m in smp.step.metadata
                  if m.name.startswith(prof.COUNTER_PREFIX)}
            md["ns"] = float((smp.end_cycle - smp.start_cycle) % (1 << 32))
            rows.setdefault(smp.step.kernel, []).append(md)
    names = sorted({c for v in rows.values() for r in v for c in r} - {"ns"})
    lines = ["Command (from the repository root, `export TMPDIR=/tmp`):", "", f"    {command}", "",
             f"Summary: `python bench.py --summarize-counters <pmc dir> --skip {skip}` "
             f"(ipu-stack_amd/profiling.py: rocprofv3 counter collection -> ProfileReport); "
             f"medians over each kernel's dispatches after its first {skip}.  Shader clock = "
             f"GRBM_GUI_ACTIVE / {xcds} XCDs / duration; MFMA-pipe utilisation = "
             f"SQ_VALU_MFMA_BUSY_CYCLES / (shader cycles x {simds} SIMDs).", "",
             "| kernel | dispatches | median ns | " + " | ".join(names) +
             " | shader clock | MFMA-pipe utilisation |",
             "|---|---|---|" + "---|" * len(names) + "---|---|"]
    for kernel, v in sorted(rows.items()):
        med = {c: float(np.median([r[c] for r in v if c in r])) for c in names + ["ns"]
               if any(c in r for r in v)}
        ns = med["ns"]
        cycles = med.get("GRBM_GUI_ACTIVE", 0.0) / xcds
        clock = f"{cycles / ns:.2f} GHz" if cycles and ns else "-"
        busy = med.get("SQ_VALU_MFMA_BUSY_CYCLES")
        util = f"{busy / (cycles * simds):.0%}" if busy is not None and cycles else "-"
        cells = [f"{med[c]:.4g}" if c in med else "-" for c in names]
        lines.append(f"| `{kernel}` | {len(v)} | {ns:.0f} | " + " | ".join(cells) +
                     f" | {clock} | {util} |")
    return "\n".join(lines) + "\n"


def device_name(info: dict) -> str:
    """The HIP device name; where the runtime leaves it empty, the product
    name the amdgpu driver exposes in sysfs."""
    if info.get("name"):
        return info["name"]
    for path in sorted(glob.glob("/sys/class/drm/card*/device/product_name")):
        try:
            with open(path) as f:
                text = f.read().strip()
            if text:
                return text
        except OSError:
            continue
    return f"AMD GPU {info.get('arch', '').split(':')[0]} ({info.get('compute_units')} CUs)"


# Untimed headline GEMMs (~45 ms) before the W warmups: from idle, the first
# 20 back-to-back 8192^3 launches average ~1300 TFLOP/s and the next 20 ~1470
# while the board's power controller settles; from the fourth region of 20 on
# they hold 1,500-1,550 for as long as measured (1.2 s).
SETTLE_LAUNCHES = 60
# The same for the attention legs (0.27-0.57 ms a launch; from idle the
# causal S4096 rate climbs from ~900 to ~1,040 TFLOP/s over ~60 launches).
ATTENTION_SETTLE_LAUNCHES = 200

LEGS = ("mfma_calibration", "gemm_f16_layouts", "gemm_f32_4096", "attention_causal_s4096",
        "attention_noncausal_s2048", "memory_chain", "amp_layouts", "gelu_4096x16384",
        "mlp_graph", "off_fast_path", "gemm_f16_256")


def bench_off_fast_path(ipus, ctx, steps):
    """Shapes no BASELINE config uses, on the kernels' other paths: fp16 /
    fp32 GEMMs whose pitches are not multiples of 8 / 4 (element-gathering
    tile kernels), attention at width 256 (the fast kernel's 256-wide
    tiles), at value width 64 beside query width 128 (its separate K and V
    tiles) and at width 132, not a multiple of 8 (the MFMA kernel for other
    widths)."""
    out = {}

    def gemm(name, m, n, k, f32):
        synth = ipus.synth_f32 if f32 else ipus.synth_f16
        a = ctx.upload(synth(m * k, 7, 1, ipus.UNIFORM))
        b = ctx.upload(synth(k * n, 7, 2, ipus.UNIFORM))
        c = ctx.alloc(m * n * (4 if f32 else 2))
        sym = "ipu_stack_gemm_f32" if f32 else "ipu_stack_gemm_f16"
        t = timed(ctx, lambda i: ctx.launch(sym, c, [a, b], [1, m, n, k, 0, 0, 0, 0]), steps, 2,
                  repeats=3, settle=10)
        out[name] = leg_entry(t, 2.0 * m * n * k, "tflops",
                              PEAK_FP32_TFLOPS if f32 else PEAK_FP16_TFLOPS)
        for x in (a, b, c):
            x.free()

    def attention(name, streams, s, d, dv):
        q = ctx.upload(ipus.synth_f16(streams * s * d, 5, 1, ipus.NORMAL))
        k = ctx.upload(ipus.synth_f16(streams * s * d, 5, 2, ipus.NORMAL))
        v = ctx.upload(ipus.synth_f16(streams * s * dv, 5, 3, ipus.NORMAL))
        o = ctx.alloc(streams * s * dv * 4)
        sc = [streams, s, s, d, dv, 0, 0, 0]
        t = timed(ctx, lambda i: ctx.launch("ipu_stack_flash_attention_online_f16", o, [q, k, v], sc),
                  steps, 2, repeats=3, settle=10)
        out[name] = leg_entry(t, 2.0 * streams * s * s * (d + dv), "tflops", PEAK_FP16_TFLOPS)
        for x in (q, k, v, o):
            x.free()

    gemm("gemm_f16_4096x4096x4100", 4096, 4096, 4100, False)
    gemm("gemm_f32_4096x4096x4097", 4096, 4096, 4097, True)
    attention("attention_16x2048_d256", 16, 2048, 256, 256)
    attention("attention_16x2048_d128_dv64", 16, 2048, 128, 64)
    attention("attention_16x2048_d132", 16, 2048, 132, 132)
    return out


def secondary_legs(ipus, ctx, args, headline_tflops=None, only=None):
    """The other BASELINE configurations (results{} of the JSON line); `only`
    restricts the run to the named legs (for profiling one kernel)."""
    def want(name):
        return only is None or name in only

    n = 8192
    results = {}
    sub_steps = max(5, args.steps // 2)
    if want("mfma_calibration"):
        cal = mfma_calibration(ipus, ctx)
        if headline_tflops:
            cal["headline_frac_of_uniform"] = round(headline_tflops / cal["uniform"]["tflops"], 4)
            cal["headline_frac_of_uniform_16x16x32"] = round(
                headline_tflops / cal["uniform_16x16x32"]["tflops"], 4)
        results["mfma_calibration"] = cal
        log(f"mfma calibration: {cal}")
    if want("gemm_f16_layouts"):
        # The headline GEMM with B, A or both stored transposed (NN is the
        # headline itself): the same kernel template reads K-contiguous rows
        # with ds_read_b128 and MN-contiguous ones with ds_read_b64_tr_b16.
        for name, tl, tr in (("nt", False, True), ("tn", True, False), ("tt", True, True)):
            t = bench_gemm_f16(ipus, ctx, n, sub_steps, 2, settle=SETTLE_LAUNCHES, tl=tl, tr=tr)
            results[f"gemm_f16_8192_{name}"] = leg_entry(t, 2.0 * n ** 3, "tflops",
                                                         PEAK_FP16_TFLOPS)
            log(f"gemm_f16 8192^3 {name.upper()}: {results[f'gemm_f16_8192_{name}']}")
    if want("gemm_f32_4096"):
        t = bench_gemm_f32(ipus, ctx, 4096, sub_steps, 2, settle=SETTLE_LAUNCHES)
        results["gemm_f32_4096"] = leg_entry(t, 2.0 * 4096 ** 3, "tflops", PEAK_FP32_TFLOPS)
        log(f"gemm_f32 4096^3: {results['gemm_f32_4096']}")
    for causal, s in ((True, 4096), (False, 2048)):
        key = f"attention_{'causal' if causal else 'noncausal'}_s{s}"
        if not want(key):
            continue
        t = bench_attention(ipus, ctx, s, causal, sub_steps, 2, settle=ATTENTION_SETTLE_LAUNCHES)
        fl = 4.0 * 128 * 128 * (s * (s + 1) / 2 if causal else s * s)
        results[key] = leg_entry(t, fl, "tflops", PEAK_FP16_TFLOPS)
        log(f"{key}: {results[key]}")
    if want("off_fast_path"):
        results["off_fast_path"] = bench_off_fast_path(ipus, ctx, 5)
        log(f"off the fast paths: {results['off_fast_path']}")
    if want("memory_chain"):
        chain = bench_memory_chain(ipus, ctx, args.steps, 3)
        bytes_rw = {"copy": 2 * n * n * 2, "transpose": 2 * n * n * 2, "block_major": 2 * n * n * 2,
                    "reduce_rows": n * n * 2 + n * 4, "reduce_rows_row_major": n * n * 2 + n * 4}
        for k, t in chain.items():
            results[k] = leg_entry(t, bytes_rw[k], "gbps", PEAK_HBM_GBPS)
            log(f"{k}: {results[k]}")
    if want("amp_layouts"):
        for k, t in bench_amp_layouts(ipus, ctx, args.steps, 3).items():
            results[k] = leg_entry(t, 2 * n * n * 2, "gbps", PEAK_HBM_GBPS)
            log(f"{k}: {results[k]}")
    if want("gelu_4096x16384"):
        t = bench_gelu(ipus, ctx, args.steps, 3)
        results["gelu_4096x16384"] = leg_entry(t, 2 * 4096 * 16384 * 2, "gbps", PEAK_HBM_GBPS)
        log(f"gelu: {results['gelu_4096x16384']}")
    if want("mlp_graph"):
        t = bench_mlp_graph(ipus, ctx, args.steps, 3, settle=SETTLE_LAUNCHES)
        results["mlp_graph"] = leg_entry(t, 2 * 2.0 * 4096 * 4096 * 16384, "tflops",
                                         PEAK_FP16_TFLOPS)
        log(f"mlp graph: {results['mlp_graph']}")
    # Last: once a HIP graph has been replayed, the block-major row reduce (a
    # 512-workgroup kernel) runs at ~4.6 instead of ~6.2 TB/s for the rest of
    # the process, in that context or a new one; other kernels are unaffected.
    if want("gemm_f16_256"):
        t = bench_gemm_f16(ipus, ctx, 256, 50, 5)
        results["gemm_f16_256"] = leg_entry(t, 2.0 * 256 ** 3, "tflops", PEAK_FP16_TFLOPS)
        results["gemm_f16_256"]["note"] = ("back-to-back ipus_launch calls; one 256 x 256 "
                                           "tile, so one workgroup on one of the 256 CUs")
        t = bench_gemm_f16_graph(ipus, ctx, 256, 10, 2)
        results["gemm_f16_256_graph"] = leg_entry(t, 2.0 * 256 ** 3, "tflops", PEAK_FP16_TFLOPS)
        results["gemm_f16_256_graph"]["note"] = ("64 one-op GEMM packages' steps captured as "
                                                 "one HIP graph and replayed: no host cost per "
                                                 "launch, so the kernel itself sets the time")
        log(f"gemm_f16 256^3: {results['gemm_f16_256']} graph {results['gemm_f16_256_graph']}")
    return results


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the headline GEMM and a calibration copy (for --pmc)")
    ap.add_argument("--leg", action="append", choices=LEGS,
                    help="run only these secondary legs (no headline; for profiling)")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="markdown summary of a rocprofv3 --kernel-trace output directory")
    ap.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="JSON traffic summary of two rocprofv3 --pmc runs of --traffic-probe")
    ap.add_argument("--summarize-traffic-table", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="markdown HBM bytes per kernel of a FETCH_SIZE and a WRITE_SIZE pass")
    ap.add_argument("--summarize-counters", metavar="DIR",
                    help="markdown MFMA-utilisation / clock summary of a rocprofv3 --pmc pass")
    ap.add_argument("--skip", type=int, default=5, help="warmup dispatches per kernel to drop")
    ap.add_argument("--command", default="", help="command line recorded in a summary")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.skip, args.command), end="")
        return 0
    if args.summarize_traffic_table:
        print(summarize_traffic_table(args.summarize_traffic_table[0],
                                      args.summarize_traffic_table[1], args.skip, args.command),
              end="")
        return 0
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.skip, args.command), end="")
        return 0
    if args.summarize_traffic:
        n = 8192
        out = summarize_traffic(args.summarize_traffic[0], args.summarize_traffic[1],
                                "gemm_f16_256_kernel", "copy_plain_kernel", 256 << 20,
                                3.0 * n * n * 2, args.skip,
                                [c for c in args.command.split(" ;; ") if c])
        print(json.dumps(out, indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); run with --gpus 1.", file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))

    ipus = __graft_entry__.import_package()
    ipus.load_library()
    ctx = ipus.Context(0)
    info = ctx.device_info()
    name = device_name(info)
    log(f"device: {name} {info['arch']} CUs={info['compute_units']} "
        f"clock={info['clock_khz'] / 1e3:.0f} MHz")

    if args.traffic_probe:
        traffic_probe(ipus, ctx)
        ctx.close()
        return 0
    if args.leg:
        legs = secondary_legs(ipus, ctx, args, only=set(args.leg))
        ctx.close()
        print(json.dumps({"legs": legs}), flush=True)
        return 0

    n = 8192
    flops = 2.0 * n ** 3
    log(f"headline: gemm_f16 8192^3 ({SETTLE_LAUNCHES} settle launches, then the W warmups)")
    # The timed region: settle launches, W warmups and a synchronisation,
    # then exactly K launches back to back between two events.
    t = bench_gemm_f16(ipus, ctx, n, args.steps, args.warmup, repeats=1, settle=SETTLE_LAUNCHES)
    tflops = flops / (t.mean * 1e-3) / 1e12
    log(f"  {t.mean:.4f} ms/step ({tflops:.1f} TFLOP/s)")

    results = {"gemm_f16_8192": leg_entry(t, flops, "tflops", PEAK_FP16_TFLOPS)}
    if not args.only_headline:
        # The same region repeated (median of 5), and the median launch of K
        # launches timed one by one (an event before each; the events add a
        # few microseconds between launches).  Each re-uploads its inputs,
        # so each runs its own settle launches first.
        rep = bench_gemm_f16(ipus, ctx, n, args.steps, 1, repeats=5, settle=SETTLE_LAUNCHES)
        results["gemm_f16_8192_regions"] = dict(
            leg_entry(rep, flops, "tflops", PEAK_FP16_TFLOPS),
            note=f"5 regions of {args.steps} back-to-back launches, median region")
        per = bench_gemm_f16(ipus, ctx, n, args.steps, 1, per_launch=True,
                             settle=SETTLE_LAUNCHES)
        results["gemm_f16_8192_per_launch"] = dict(
            leg_entry(per, flops, "tflops", PEAK_FP16_TFLOPS),
            min_ms=round(per["min_ms"], 5), max_ms=round(per["max_ms"], 5),
            note=f"{args.steps} launches with an event before each and after the last: "
                 "median launch")
        log(f"  regions median {rep.median:.4f} ms, per-launch median {per.median:.4f} ms")
        results.update(secondary_legs(ipus, ctx, args, tflops))

    traffic, traffic_note = committed_traffic()
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t.mean, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "gemm_f16 M=N=K=8192, A,B ~ U[-1,1] fp16, fp32 accumulate, "
                               "fp16 out (BASELINE configs[1])",
                   "M": n, "N": n, "K": n, "parallelism": "single GPU",
                   "statistic": "value, ms_per_step and roofline.achieved: the K timed "
                                "launches back to back between two HIP events, region time / K "
                                "(rocprof's average launch duration for the same run)",
                   "settle_launches": SETTLE_LAUNCHES,
                   "settle": "untimed launches before the W warmups: from idle, the board's "
                             "power controller takes ~30-50 ms of load to settle (launches 3-6 "
                             "run ~25% slower than the steady state)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_note,
                     "kernel": "gemm_f16_256_kernel<false, false, 0, false, false>",
                     "ms_mean": round(t.mean, 5)},
        "results": results,
        "device": {"name": name, "arch": info["arch"], "cus": info["compute_units"]},
    }
    ctx.close()
    if rank == 0 and not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        line["cpu_baseline"] = cpu_baseline(ipus)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

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

Timing: HIP events recorded on the library's stream around K launches after
W warmups; bandwidth kernels rotate 3 buffer sets (768 MiB > the 256 MiB
MALL).  One JSON line on stdout.
"""
from __future__ import annotations

import argparse
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


def timed(ctx, fn, steps: int, warmup: int) -> float:
    """Average milliseconds per call of `fn` (which enqueues on the stream)."""
    for _ in range(warmup):
        fn(0)
    ctx.sync()
    timer = ctx.timer()
    timer.start()
    for i in range(steps):
        fn(i)
    ms = timer.stop()
    ctx.sync()
    timer.close()
    return ms / steps


def gemm_scalars(n, m=None, k=None):
    m = m or n
    k = k or n
    return [1, m, n, k, 0, 0, 0, 0]


def bench_gemm_f16(ipus, ctx, n, steps, warmup):
    a = ctx.upload(ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM))
    b = ctx.upload(ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM))
    c = ctx.alloc(n * n * 2)
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_gemm_f16", c, [a, b], gemm_scalars(n)),
               steps, warmup)
    for x in (a, b, c):
        x.free()
    return ms


def bench_gemm_f32(ipus, ctx, n, steps, warmup):
    a = ctx.upload(ipus.synth_f32(n * n, 4096, 1, ipus.NORMAL))
    b = ctx.upload(ipus.synth_f32(n * n, 4096, 2, ipus.NORMAL))
    c = ctx.alloc(n * n * 4)
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_gemm_f32", c, [a, b], gemm_scalars(n)),
               steps, warmup)
    for x in (a, b, c):
        x.free()
    return ms


def bench_attention(ipus, ctx, s, causal, steps, warmup, streams=128, d=128):
    n = streams * s * d
    q = ctx.upload(ipus.synth_f16(n, 5, 1, ipus.NORMAL))
    k = ctx.upload(ipus.synth_f16(n, 5, 2, ipus.NORMAL))
    v = ctx.upload(ipus.synth_f16(n, 5, 3, ipus.NORMAL))
    o = ctx.alloc(n * 4)
    sc = [streams, s, s, d, d, 0, int(causal), 0]
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_flash_attention_online_f16", o, [q, k, v], sc),
               steps, warmup)
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


def bench_gelu(ipus, ctx, steps, warmup, rows=4096, cols=16384, sets=3):
    n = rows * cols
    x = [ctx.upload(ipus.synth_f16(n, 88, s, ipus.NORMAL)) for s in range(sets)]
    y = [ctx.alloc(n * 2) for _ in range(sets)]
    ms = timed(ctx, lambda i: ctx.launch("ipu_stack_gelu_tanh_approx_f16", y[i % sets],
                                         [x[i % sets]], [n]), steps, warmup)
    for b in x + y:
        b.free()
    return ms


def bench_mlp_graph(ipus, ctx, steps, warmup):
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
    ms = timed(ctx, lambda i: sess.run(), steps, warmup)
    sess.close()
    return ms


def mfma_calibration(ipus, ctx, blocks=1024, iterations=4096):
    """Sustained v_mfma_f32_32x32x16_f16 rate and shader clock with register-
    resident operands: once with fragments drawn like the headline's inputs
    (U[-1, 1] fp16) and once with all-zero fragments.  The clock under dense
    MFMA falls with operand entropy (power limit), so the first figure is the
    ceiling the headline GEMM can reach on this board."""
    out = {}
    for name, frags in (("uniform", ipus.synth_f16(4096 * 8, 2024, 3, ipus.UNIFORM)),
                        ("zeros", np.zeros(4096 * 8, dtype=np.float16))):
        ops = ctx.upload(frags)
        res = ctx.alloc(16 + blocks * 256 * 4)
        sc = [4096, iterations, blocks]
        ms = timed(ctx, lambda i: ctx.launch("ipus_calibrate_mfma_f16", res, [ops], sc), 3, 1)
        clocks = res.download(np.uint64)[:2]
        flops = blocks * 4 * 8 * iterations * 32 * 32 * 16 * 2.0
        mhz = clocks[0] / (clocks[1] / 100.0) if clocks[1] else 0.0
        out[name] = {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "clock_mhz": round(mhz)}
        ops.free()
        res.free()
    return out


def cpu_baseline(ipus, n=8192, min_seconds=10.0):
    """The repo's CPU evaluator (oracle/, a C restatement of the reference's
    diagnostic::evaluate GEMM) on the headline workload itself: the full
    8192^3 fp16 GEMM, repeated until at least `min_seconds` of CPU work; the
    reported rate is the median over the repetitions."""
    from oracle import oracle
    threads = oracle.threads()
    a = ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM)
    b = ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM)
    times = []
    while not times or (sum(times) < min_seconds and len(times) < 20):
        t0 = time.perf_counter()
        oracle.gemm_f16(a, b, n, n, n, nthreads=threads)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    return {
        "value": round(2.0 * n ** 3 / dt / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full 8192^3 fp16 GEMM x{len(times)} (fp16->fp32 operands, blocked AVX2 "
                  f"sgemm, fp16 rounding), median {dt:.2f} s, total {sum(times):.1f} s",
    }


def traffic_probe(ipus, ctx, n=8192, copy_bytes=256 << 20):
    """Untimed launches for the rocprofv3 --pmc passes that give
    roofline.traffic: the headline GEMM, then a plain 16-byte-vector copy of
    `copy_bytes` whose FETCH_SIZE / WRITE_SIZE calibrate the counters' unit."""
    a = ctx.upload(ipus.synth_f16(n * n, 2024, 1, ipus.UNIFORM))
    b = ctx.upload(ipus.synth_f16(n * n, 2024, 2, ipus.UNIFORM))
    c = ctx.alloc(n * n * 2)
    for _ in range(3):
        ctx.launch("ipu_stack_gemm_f16", c, [a, b], gemm_scalars(n))
    ctx.sync()
    src, dst = ctx.alloc(copy_bytes), ctx.alloc(copy_bytes)
    ctx.memset(src, 1)
    for _ in range(3):
        ctx.launch("ipu_stack_copy", dst, [src], [copy_bytes])
    ctx.sync()
    for x in (a, b, c, src, dst):
        x.free()
    log(f"traffic probe: 3x gemm_f16 {n}^3, 3x copy {copy_bytes} B")


def committed_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/gemm_f16_8192_traffic.json)."""
    path = os.path.join(ROOT, "profiles", "gemm_f16_8192_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


LEGS = ("mfma_calibration", "gemm_f32_4096", "gemm_f16_256", "attention_causal_s4096",
        "attention_noncausal_s2048", "memory_chain", "gelu_4096x16384", "mlp_graph")


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
        results["mfma_calibration"] = cal
        log(f"mfma calibration: {cal}")
    if want("gemm_f32_4096"):
        ms32 = bench_gemm_f32(ipus, ctx, 4096, sub_steps, 2)
        t32 = 2.0 * 4096 ** 3 / (ms32 * 1e-3) / 1e12
        results["gemm_f32_4096"] = {"ms": round(ms32, 5), "tflops": round(t32, 2),
                                    "frac_peak": round(t32 / PEAK_FP32_TFLOPS, 4)}
        log(f"gemm_f32 4096^3: {ms32:.4f} ms {t32:.1f} TFLOP/s")
    if want("gemm_f16_256"):
        ms256 = bench_gemm_f16(ipus, ctx, 256, 50, 5)
        results["gemm_f16_256"] = {"ms": round(ms256, 5),
                                   "tflops": round(2.0 * 256 ** 3 / (ms256 * 1e-3) / 1e12, 3)}
    for causal, s in ((True, 4096), (False, 2048)):
        key = f"attention_{'causal' if causal else 'noncausal'}_s{s}"
        if not want(key):
            continue
        msa = bench_attention(ipus, ctx, s, causal, sub_steps, 2)
        fl = 4.0 * 128 * 128 * (s * (s + 1) / 2 if causal else s * s)
        ta = fl / (msa * 1e-3) / 1e12
        results[key] = {"ms": round(msa, 5), "tflops": round(ta, 2),
                        "frac_peak": round(ta / PEAK_FP16_TFLOPS, 4)}
        log(f"{key}: {msa:.4f} ms {ta:.1f} TFLOP/s")
    if want("memory_chain"):
        chain = bench_memory_chain(ipus, ctx, args.steps, 3)
        bytes_rw = {"copy": 2 * n * n * 2, "transpose": 2 * n * n * 2, "block_major": 2 * n * n * 2,
                    "reduce_rows": n * n * 2 + n * 4, "reduce_rows_row_major": n * n * 2 + n * 4}
        for k, v in chain.items():
            gbps = bytes_rw[k] / (v * 1e-3) / 1e9
            results[k] = {"ms": round(v, 5), "gbps": round(gbps, 1),
                          "frac_peak": round(gbps / PEAK_HBM_GBPS, 4)}
            log(f"{k}: {v * 1e3:.1f} us {gbps:.0f} GB/s")
    if want("gelu_4096x16384"):
        msg = bench_gelu(ipus, ctx, args.steps, 3)
        gg = 2 * 4096 * 16384 * 2 / (msg * 1e-3) / 1e9
        results["gelu_4096x16384"] = {"ms": round(msg, 5), "gbps": round(gg, 1),
                                      "frac_peak": round(gg / PEAK_HBM_GBPS, 4)}
        log(f"gelu: {msg * 1e3:.1f} us {gg:.0f} GB/s")
    if want("mlp_graph"):
        msm = bench_mlp_graph(ipus, ctx, 5, 1)
        tm = 2 * 2.0 * 4096 * 4096 * 16384 / (msm * 1e-3) / 1e12
        results["mlp_graph"] = {"ms": round(msm, 5), "tflops": round(tm, 2),
                                "frac_peak": round(tm / PEAK_FP16_TFLOPS, 4)}
        log(f"mlp graph: {msm:.3f} ms {tm:.1f} TFLOP/s")
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
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); run with --gpus 1.", file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))

    ipus = __graft_entry__.import_package()
    ipus.load_library()
    ctx = ipus.Context(0)
    info = ctx.device_info()
    log(f"device: {info['name']} {info['arch']} CUs={info['compute_units']} "
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
    log("headline: gemm_f16 8192^3")
    ms = bench_gemm_f16(ipus, ctx, n, args.steps, args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"  {ms:.4f} ms/step  {tflops:.1f} TFLOP/s")

    results = {"gemm_f16_8192": {"ms": round(ms, 5), "tflops": round(tflops, 2),
                                 "frac_peak": round(tflops / PEAK_FP16_TFLOPS, 4)}}
    if not args.only_headline:
        results.update(secondary_legs(ipus, ctx, args, tflops))

    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "gemm_f16 M=N=K=8192, A,B ~ U[-1,1] fp16, fp32 accumulate, "
                               "fp16 out (BASELINE configs[1])",
                   "M": n, "N": n, "K": n, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": committed_traffic()},
        "results": results,
        "device": {"name": info["name"], "arch": info["arch"], "cus": info["compute_units"]},
    }
    ctx.close()
    if rank == 0 and not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        line["cpu_baseline"] = cpu_baseline(ipus)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

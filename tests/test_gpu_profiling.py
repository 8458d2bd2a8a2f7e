"""rocprof ingestion on a real device run (crates/ipu-profile/src/lib.rs:440-585
query semantics): a package runs under `rocprofv3 --kernel-trace` in a child
process, and the trace, read back through `profiling.from_rocprof` with the
package's step symbols as operations, answers the reference's queries."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNS = 3

CHILD = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    import numpy as np
    import __graft_entry__
    ipus = __graft_entry__.import_package()
    ipus.load_library()
    g = ipus.ComputeGraph()
    x = g.host_input("x", [256, 512])
    w = g.parameter("w", [512, 256])
    g.set_outputs([g.gelu(g.gemm(x, w)), g.transpose(x)])
    pkg = ipus.build_package(g, ipus.PackageConfig())
    with ipus.Context(0) as ctx:
        sess = pkg.session(ctx)
        rng = np.random.default_rng(5)
        sess.write("x", rng.standard_normal((256, 512)).astype(np.float16))
        sess.write("w", rng.standard_normal((512, 256)).astype(np.float16))
        for _ in range({runs}):
            sess.run()
        ctx.sync()
        sess.close()
    print("steps", " ".join(s[0] for s in pkg.steps))
    print("done", flush=True)
""")


@pytest.mark.gpu
def test_rocprof_trace_of_a_package_run_answers_queries(ipus, tmp_path):
    exe = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(exe):
        pytest.skip("rocprofv3 is not installed")
    import ipu_stack_amd.profiling as prof
    script = tmp_path / "run_package.py"
    script.write_text(CHILD.format(root=ROOT, runs=RUNS))
    trace = tmp_path / "trace"
    env = dict(os.environ, TMPDIR=str(tmp_path))
    print(f"rocprofv3 kernel trace of {script}", flush=True)
    r = subprocess.run([exe, "--kernel-trace", "--output-format", "csv", "-d", str(trace),
                        "-o", "run", "--", sys.executable, str(script)],
                       cwd=str(tmp_path), env=env, capture_output=True, text=True, timeout=180)
    # The profiled program must have finished; rocprofv3 itself may end with
    # a non-zero status after writing complete results.
    assert "done" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    steps = next(l for l in r.stdout.splitlines() if l.startswith("steps ")).split()[1:]
    assert steps, "the package plans at least one step"

    report = prof.from_rocprof(str(trace), operations=steps,
                               kernel_filter=lambda k: not k.startswith("__amd"))
    samples = [s for t in report.tiles for s in t.samples]
    assert len(samples) == RUNS * len(steps)
    # Dispatch order follows the package's steps, run after run.
    assert [s.step.operation for s in sorted(samples, key=lambda s: s.step.phase)] == steps * RUNS

    by_op = prof.query(report, prof.Query(group_by=prof.GroupBy.OPERATION))
    counts = {g.name: g.sample_count for g in by_op.groups}
    for sym in set(steps):
        assert counts[sym] == RUNS * steps.count(sym)
    by_kernel = prof.query(report, prof.Query(group_by=prof.GroupBy.KERNEL))
    assert sum(g.sample_count for g in by_kernel.groups) == RUNS * len(steps)
    for g in by_kernel.groups:
        assert 0 < g.p50_cycles <= g.p95_cycles <= g.maximum_cycles
    # A profile database calibrated from the report serialises and reloads.
    text = report.to_json()
    again = prof.ProfileReport.from_json(text)
    assert sum(len(t.samples) for t in again.tiles) == len(samples)

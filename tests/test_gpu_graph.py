"""GPU runs of compiled packages (build_package + session) against the CPU
oracle, and the fused GEMM+GELU launch against its two-launch form.

Each graph is built with the ComputeGraph API, compiled, bound and run on
cuda:0; the expected values come from the oracle's restatement of the
reference's per-operator evaluation (crates/ipu-tests/src/diagnostic.rs:
411-847) applied step by step in the same precisions.  Bars as in
test_gpu_kernels.py: bit-exact for rearranges and for the fusion against the
unfused launches, normwise max-rel <= 1e-2 for fp16 results.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import fp16_close, max_rel

pytestmark = pytest.mark.gpu

FP16_TOL = 1e-2


def synth(ipus, n, seed, tensor, dist=1, scale=1.0):
    return ipus.synth_f16(n, seed, tensor, dist, scale)


def run_package(ipus, ctx, graph, feeds, config=None):
    pkg = ipus.build_package(graph, config)
    sess = pkg.session(ctx)
    for name, array in feeds.items():
        sess.write(name, array)
    sess.run_sync()
    outs = [sess.read(t.name) for t in pkg.outputs]
    sess.close()
    return pkg, outs


def test_mlp_package_matches_oracle_and_fusion_is_exact(ipus, oracle, ctx):
    # configs[3]'s structure at a small size: X . W1 -> GELU -> . W2.
    m, d, h = 256, 256, 1024
    g = ipus.ComputeGraph()
    x = g.host_input("x", [m, d])
    w1 = g.parameter("w1", [d, h])
    w2 = g.parameter("w2", [h, d])
    g.set_outputs([g.gemm(g.gelu(g.gemm(x, w1)), w2)])
    xs = synth(ipus, m * d, 31, 1).reshape(m, d)
    w1s = synth(ipus, d * h, 31, 2, scale=0.05).reshape(d, h)
    w2s = synth(ipus, h * d, 31, 3, scale=0.05).reshape(h, d)
    pkg, (y,) = run_package(ipus, ctx, g, {"x": xs, "w1": w1s, "w2": w2s})
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16"]
    hidden = oracle.gelu_f16(oracle.gemm_f16(xs, w1s, m, h, d)).reshape(m, h)
    want = oracle.f16_to_f32(oracle.gemm_f16(hidden, w2s, m, d, h)).reshape(m, d)
    assert fp16_close(oracle.f16_to_f32(y), want, FP16_TOL)
    # The fused launch equals GEMM then GELU bit for bit.
    bx, b1 = ctx.upload(xs), ctx.upload(w1s)
    fused, plain, act = ctx.alloc(m * h * 2), ctx.alloc(m * h * 2), ctx.alloc(m * h * 2)
    sc = [1, m, h, d, 0, 0, 0, 0]
    ctx.launch("ipu_stack_gemm_f16_gelu", fused, [bx, b1], sc)
    ctx.launch("ipu_stack_gemm_f16", plain, [bx, b1], sc)
    ctx.launch("ipu_stack_gelu_tanh_approx_f16", act, [plain], [m * h])
    assert np.array_equal(fused.download(np.uint16), act.download(np.uint16))
    for b in (bx, b1, fused, plain, act):
        b.free()


@pytest.mark.parametrize("h,plan", [
    (8608, ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16_split", "ipu_stack_reduce_splits_f16"]),
    (4304, ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16_gelu"])])
def test_split_k_mlp_package_matches_oracle(ipus, oracle, ctx, h, plan):
    """The reference's SigLIP MLP at one image (729 tokens, width 1152,
    hidden 4304): both GEMMs run unsplit on the small-tile kernel with GELU
    fused; with the hidden width doubled the second GEMM (K = 8608) is
    planned split-K with GELU fused into the reduction."""
    m, d = 729, 1152
    g = ipus.ComputeGraph()
    x = g.host_input("x", [m, d])
    w1 = g.parameter("w1", [d, h])
    w2 = g.parameter("w2", [h, d])
    g.set_outputs([g.gelu(g.gemm(g.gelu(g.gemm(x, w1)), w2))])
    xs = synth(ipus, m * d, 33, 1).reshape(m, d)
    w1s = synth(ipus, d * h, 33, 2, scale=0.05).reshape(d, h)
    w2s = synth(ipus, h * d, 33, 3, scale=0.05).reshape(h, d)
    pkg, (y,) = run_package(ipus, ctx, g, {"x": xs, "w1": w1s, "w2": w2s})
    assert [s[0] for s in pkg.steps] == plan
    hidden = oracle.gelu_f16(oracle.gemm_f16(xs, w1s, m, h, d)).reshape(m, h)
    want = oracle.f16_to_f32(oracle.gelu_f16(oracle.gemm_f16(hidden, w2s, m, d, h))).reshape(m, d)
    assert fp16_close(oracle.f16_to_f32(y), want, FP16_TOL)


@pytest.mark.parametrize("M,N,K,tl,tr,splits,batches,shared", [
    (729, 1152, 4304, 0, 0, 8, 1, ""), (729, 1152, 4304, 0, 1, 8, 1, ""),
    (264, 136, 3000, 0, 1, 5, 2, ""), (200, 264, 2048, 1, 0, 4, 1, ""),
    (256, 256, 4096, 0, 0, 16, 1, ""), (264, 136, 3000, 0, 1, 5, 3, "right"),
    (136, 264, 2560, 1, 1, 3, 2, "left")])
def test_split_k_gemm_matches_oracle(ipus, oracle, ctx, M, N, K, tl, tr, splits, batches, shared):
    """Split partials summed by the reduction equal the one-launch GEMM's
    semantics (fp32 accumulation, one fp16 rounding) to the fp16 bar, and the
    GELU variant of the reduction is GELU of the plain reduction bit for bit.
    `shared` names an operand broadcast over the batch (batch stride 0)."""
    lbs = 0 if shared == "left" else M * K
    rbs = 0 if shared == "right" else K * N
    a = synth(ipus, (1 if lbs == 0 else batches) * M * K, 34, 1)
    b = synth(ipus, (1 if rbs == 0 else batches) * K * N, 34, 2, scale=0.2)
    ba, bb = ctx.upload(a), ctx.upload(b)
    parts = ctx.alloc(splits * batches * M * N * 4)
    out, act, fused = (ctx.alloc(batches * M * N * 2) for _ in range(3))
    ctx.launch("ipu_stack_gemm_f16_split", parts, [ba, bb],
               [batches, M, N, K, tl, tr, lbs, rbs, splits])
    ctx.launch("ipu_stack_reduce_splits_f16", out, [parts], [splits, batches * M * N, 0])
    ctx.launch("ipu_stack_reduce_splits_f16", fused, [parts], [splits, batches * M * N, 1])
    ctx.launch("ipu_stack_gelu_tanh_approx_f16", act, [out], [batches * M * N])
    got = oracle.f16_to_f32(out.download(np.uint16))
    want = oracle.f16_to_f32(oracle.gemm_f16(a, b, M, N, K, bool(tl), bool(tr), batches,
                                             lbs, rbs))
    assert fp16_close(got, want, FP16_TOL)
    assert np.array_equal(fused.download(np.uint16), act.download(np.uint16))
    for buf in (ba, bb, parts, out, act, fused):
        buf.free()


def test_split_k_rejects_empty_splits(ipus, ctx):
    buf = ctx.alloc(4096)
    # K = 2048 in 3 splits of 704 k: ceil(2048 / 704) = 3, fine; 40 splits of
    # 64 k leave 8 splits without work.
    with pytest.raises(ipus.IpusError) as e:
        ctx.launch("ipu_stack_gemm_f16_split", buf, [buf, buf], [1, 8, 8, 2048, 0, 0, 0, 0, 40])
    assert e.value.status == ipus.ERROR_INVALID_ARGUMENT
    buf.free()


@pytest.mark.parametrize("M,N,K,tl,tr", [(256, 512, 128, 0, 0), (512, 256, 192, 1, 1),
                                         (100, 60, 40, 0, 0), (64, 96, 48, 0, 1),
                                         (66, 68, 129, 1, 0), (130, 132, 260, 0, 0)])
def test_gemm_gelu_fusion_bit_exact(ipus, ctx, M, N, K, tl, tr):
    a = synth(ipus, M * K, 32, 1)
    b = synth(ipus, K * N, 32, 2, scale=0.2)
    ba, bb = ctx.upload(a), ctx.upload(b)
    fused, plain, act = ctx.alloc(M * N * 2), ctx.alloc(M * N * 2), ctx.alloc(M * N * 2)
    sc = [1, M, N, K, tl, tr, 0, 0]
    ctx.launch("ipu_stack_gemm_f16_gelu", fused, [ba, bb], sc)
    ctx.launch("ipu_stack_gemm_f16", plain, [ba, bb], sc)
    ctx.launch("ipu_stack_gelu_tanh_approx_f16", act, [plain], [M * N])
    assert np.array_equal(fused.download(np.uint16), act.download(np.uint16))
    for buf in (ba, bb, fused, plain, act):
        buf.free()


def test_attention_package_matches_oracle(ipus, oracle, ctx):
    # Projections, head split and causal attention (graph.rs:338-362).
    b, s, d, heads = 2, 128, 256, 2
    g = ipus.ComputeGraph()
    x = g.host_input("x", [b, s, d])
    wq = g.parameter("wq", [d, d])
    wk = g.parameter("wk", [d, d])
    wv = g.parameter("wv", [d, d])
    q = g.split_heads(g.gemm(x, wq), heads)
    k = g.split_heads(g.gemm(x, wk), heads)
    v = g.split_heads(g.gemm(x, wv), heads)
    g.set_outputs([g.flash_attention_with_options(q, k, v, causal=True)])
    xs = synth(ipus, b * s * d, 33, 1).reshape(b, s, d)
    ws = {n: synth(ipus, d * d, 33, i + 2, scale=0.08).reshape(d, d)
          for i, n in enumerate(("wq", "wk", "wv"))}
    pkg, (o,) = run_package(ipus, ctx, g, {"x": xs, **ws})
    assert o.dtype == np.float32 and o.shape == (b * heads, s, d // heads)
    proj = {n: oracle.f16_to_f32(oracle.gemm_f16(xs.reshape(b * s, d), ws[n], b * s, d, d))
            .reshape(b, s, d) for n in ws}
    qh, kh, vh = (oracle.split_heads(proj[n], heads) for n in ("wq", "wk", "wv"))
    want = oracle.attention(qh, kh, vh, b * heads, s, s, d // heads, d // heads, causal=True)
    assert fp16_close(o.reshape(-1, d // heads), want, FP16_TOL)


def test_memory_chain_package_bit_exact(ipus, oracle, ctx):
    n = 512
    g = ipus.ComputeGraph()
    x = g.host_input("x", [n, n])
    t = g.transpose(x)
    bm = g.rearrange(t, ipus.ORDER_BLOCK_MAJOR, 64, 64)
    r = g.reduce_rows(bm)
    g.set_outputs([t, bm, r])
    xs = synth(ipus, n * n, 34, 1).reshape(n, n)
    _, (tg, bmg, rg) = run_package(ipus, ctx, g, {"x": xs})
    tw = oracle.transpose_u16(xs, 1, n, n).reshape(n, n)
    assert np.array_equal(tg, tw)
    bmw = oracle.rearrange_row_major_f16(tw, 2, 1, n, n, n, n, 64, 64)
    assert np.array_equal(bmg.reshape(-1), bmw.reshape(-1))
    rw = oracle.reduce_rows_f16(tw, n, n)
    assert np.abs(rg - rw).max() <= 1e-5 * max(1.0, np.abs(rw).max())


def test_add_broadcast_and_f32_compute_package(ipus, oracle, ctx):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [4, 64, 32])
    bias = g.parameter("bias", [32])
    w = g.parameter("w", [32, 48])
    y = g.gemm(g.add(x, bias), w)
    g.set_outputs([y])
    xs = synth(ipus, 4 * 64 * 32, 35, 1).reshape(4, 64, 32)
    bs = synth(ipus, 32, 35, 2).reshape(32)
    wsr = synth(ipus, 32 * 48, 35, 3, scale=0.2).reshape(32, 48)
    # fp32 compute: host tensors are fp32 (PackageConfig compute precision)
    cfg = ipus.PackageConfig(compute_precision="f32")
    xf, bf, wf = (oracle.f16_to_f32(a) for a in (xs, bs, wsr))
    _, (yf,) = run_package(ipus, ctx, g, {"x": xf, "bias": bf, "w": wf}, cfg)
    want = oracle.add_f32(xf, bf).reshape(-1, 32) @ wf.astype(np.float64)
    assert np.abs(yf.reshape(-1, 48) - want).max() <= 1e-5 * np.abs(want).max()
    # fp16 compute: the add rounds to fp16 before the GEMM
    _, (yh,) = run_package(ipus, ctx, g, {"x": xs, "bias": bs, "w": wsr})
    added = oracle.f32_to_f16(oracle.add_f32(xf, bf)).reshape(-1, 32)
    want16 = oracle.f16_to_f32(oracle.gemm_f16(added, wsr, 4 * 64, 48, 32)).reshape(4, 64, 48)
    assert fp16_close(oracle.f16_to_f32(yh), want16, FP16_TOL)


def test_repeat_package_matches_unrolled_oracle(ipus, oracle, ctx):
    # x <- x + x . W_i for i in 0..3 (graph.rs:382-472, diagnostic.rs:466-522)
    g = ipus.ComputeGraph()
    x = g.host_input("x", [64, 64])
    ws = [g.parameter(f"w{i}", [64, 64]) for i in range(4)]
    seq = g.value_sequence("layers", ws)
    out = g.repeat(4, [x], [], [seq],
                   lambda body, a: [body.add(a.carried[0], body.gemm(a.carried[0], a.iterated[0]))])
    g.set_outputs(out)
    xs = synth(ipus, 64 * 64, 36, 1).reshape(64, 64)
    wv = [synth(ipus, 64 * 64, 36, i + 2, scale=0.05).reshape(64, 64) for i in range(4)]
    _, (y,) = run_package(ipus, ctx, g, {"x": xs, **{f"w{i}": wv[i] for i in range(4)}})
    cur = xs
    for w in wv:
        prod = oracle.gemm_f16(cur, w, 64, 64, 64).reshape(64, 64)
        cur = oracle.f32_to_f16(oracle.f16_to_f32(cur) + oracle.f16_to_f32(prod)).reshape(64, 64)
    assert fp16_close(oracle.f16_to_f32(y), oracle.f16_to_f32(cur), FP16_TOL)


def _mlp_graph(ipus, m, d, h):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [m, d])
    w1 = g.parameter("w1", [d, h])
    w2 = g.parameter("w2", [h, d])
    g.set_outputs([g.gemm(g.gelu(g.gemm(x, w1)), w2)])
    return g, {"x": (m * d, 1.0), "w1": (d * h, 0.05), "w2": (h * d, 0.05)}


def _memory_graph(ipus, n):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [n, n])
    t = g.transpose(x)
    bm = g.rearrange(t, ipus.ORDER_BLOCK_MAJOR, 64, 64)
    g.set_outputs([t, bm, g.reduce_rows(bm)])
    return g, {"x": (n * n, 1.0)}


@pytest.mark.parametrize("which", ["mlp", "memory"])
def test_captured_session_replays_match_eager(ipus, ctx, which):
    # A captured session replays its HIP graph on each run; every replay,
    # with fresh inputs written and an eager session run in between, must
    # equal the eager session bit for bit.
    g, feeds = _mlp_graph(ipus, 256, 256, 512) if which == "mlp" else _memory_graph(ipus, 512)
    pkg = ipus.build_package(g)
    eager, graph = pkg.session(ctx), pkg.session(ctx)
    graph.capture()
    graph.capture()  # second call is a no-op
    try:
        for replay in range(4):
            for i, (name, (count, scale)) in enumerate(feeds.items()):
                a = synth(ipus, count, 40 + replay, i + 1, scale=scale)
                eager.write(name, a)
                graph.write(name, a)
            eager.run_sync()
            graph.run_sync()
            eager.run_sync()  # eager work between replays
            for t in pkg.outputs:
                want, got = eager.read(t.name), graph.read(t.name)
                assert np.array_equal(want.view(np.uint8), got.view(np.uint8)), (replay, t.name)
    finally:
        eager.close()
        graph.close()


def test_mlp_package_full_size_configs3(ipus, oracle, ctx):
    """BASELINE configs[3] at its full size: X[4096, 4096] ~ N(0, 1),
    W1[4096, 16384] and W2[16384, 4096] ~ N(0, 0.02), X . W1 -> GELU -> . W2.
    Row i of Y depends only on row i of X, so 24 sampled rows (every stream
    of 256-row tiles, both edges) are checked against the oracle:
    y_i = f16(f16(gelu(f16(x_i . W1))) . W2)."""
    m, d, h = 4096, 4096, 16384
    g = ipus.ComputeGraph()
    x = g.host_input("x", [m, d])
    w1 = g.parameter("w1", [d, h])
    w2 = g.parameter("w2", [h, d])
    g.set_outputs([g.gemm(g.gelu(g.gemm(x, w1)), w2)])
    xs = synth(ipus, m * d, 2024, 1)
    w1s = synth(ipus, d * h, 2024, 2, scale=0.02)
    w2s = synth(ipus, h * d, 2024, 3, scale=0.02)
    pkg, (y,) = run_package(ipus, ctx, g, {"x": xs.reshape(m, d), "w1": w1s.reshape(d, h),
                                          "w2": w2s.reshape(h, d)})
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16"]
    rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 1],
                                     np.linspace(2, m - 2, 19).astype(np.int64)]))
    xr = xs.reshape(m, d)[rows]
    hidden = oracle.gelu_f16(oracle.f32_to_f16(
        oracle.gemm_f16_rows(xr, w1s, len(rows), h, d, np.arange(len(rows)))))
    want = oracle.f16_to_f32(oracle.f32_to_f16(
        oracle.gemm_f16_rows(hidden, w2s, len(rows), d, h, np.arange(len(rows)))))
    got = oracle.f16_to_f32(y.reshape(m, d)[rows])
    assert np.all(np.isfinite(got))
    assert fp16_close(got, want, FP16_TOL), max_rel(got, want)


def test_injected_launch_failure_propagates_and_releases_everything(ipus, oracle, ctx):
    """A launch that fails inside ipus_session_run or ipus_session_capture
    surfaces as that call's error (the first failing step's status and
    message), leaves the stream usable, and every buffer is released by
    session and context teardown (the role of the reference's failure path,
    crates/ipu-tests/src/main.rs:985-1006; the failure is injected on the
    host, so no kernel faults)."""
    status = -1000 - 700  # IPUS_ERROR_HIP_BASE - hipErrorIllegalAddress
    base = ctx.live_buffers()
    m, d, h = 128, 128, 512
    g = ipus.ComputeGraph()
    x = g.host_input("x", [m, d])
    w1 = g.parameter("w1", [d, h])
    w2 = g.parameter("w2", [h, d])
    g.set_outputs([g.gelu(g.add(g.gemm(g.gelu(g.gemm(x, w1)), w2), x))])
    pkg = ipus.build_package(g)
    assert len(pkg.steps) == 3
    feeds = {"x": synth(ipus, m * d, 51, 1).reshape(m, d),
             "w1": synth(ipus, d * h, 51, 2, scale=0.05).reshape(d, h),
             "w2": synth(ipus, h * d, 51, 3, scale=0.05).reshape(h, d)}
    sess = pkg.session(ctx)
    assert ctx.live_buffers()[0] > base[0]
    for name, array in feeds.items():
        sess.write(name, array)
    sess.run_sync()
    want = sess.read("output.0")
    # Eager run: the second step fails; nothing after it runs.
    ctx.inject_launch_failure(1, status)
    with pytest.raises(ipus.IpusError) as err:
        sess.run()
    assert err.value.status == status and "injected" in err.value.message
    ctx.sync()
    sess.run_sync()
    assert np.array_equal(sess.read("output.0"), want)
    # Capture: the failing launch ends the capture with the error and no
    # graph; eager runs and a later capture work.
    ctx.inject_launch_failure(0, status)
    with pytest.raises(ipus.IpusError) as err:
        sess.capture()
    assert err.value.status == status
    sess.run_sync()
    assert np.array_equal(sess.read("output.0"), want)
    sess.capture()
    for _ in range(2):
        sess.run_sync()
        assert np.array_equal(sess.read("output.0"), want)
    sess.close()
    assert ctx.live_buffers() == base
    # Context.close with a session still open after a failure releases the
    # session, its buffers and the context.
    c2 = ipus.Context(0)
    s2 = pkg.session(c2)
    extra = c2.alloc(4096)
    c2.inject_launch_failure(0, status)
    with pytest.raises(ipus.IpusError):
        s2.run()
    c2.close()
    assert s2.handle is None and extra.ptr == 0
    with pytest.raises(ipus.IpusError):
        s2.run()


# ---------------------------------------------------------------------------
# Declared input formats: reference-layout bytes in, row-major results out
# ---------------------------------------------------------------------------
from test_graph import FORMAT_CASES, oracle_layout_args  # noqa: E402


@pytest.mark.parametrize("name,shape,make", FORMAT_CASES, ids=[c[0] for c in FORMAT_CASES])
def test_declared_format_unshards_bit_exact(ipus, oracle, ctx, name, shape, make):
    """Every layout of the CPU plan tests: the oracle packs random fp16 data
    into the format's host bytes, the package's unshard launch rebuilds the
    tensor, which the graph returns unchanged (bit-exact)."""
    layout = make(ipus.Layout)
    g = ipus.ComputeGraph()
    x = g.host_input("x", shape)
    g.set_outputs([x])
    cfg = ipus.PackageConfig().with_input(x, ipus.TensorFormat(ipus.PRECISION_F16, layout))
    n = int(np.prod(shape))
    data = synth(ipus, n, 71, len(name))
    packed = oracle.pack_tiled(data, shape, **oracle_layout_args(ipus, layout))
    pkg, (y,) = run_package(ipus, ctx, g, {"x": packed}, cfg)
    assert "ipu_stack_unshard" in [s[0] for s in pkg.steps]
    assert np.array_equal(y.reshape(-1), data)


@pytest.mark.parametrize("batch,tiles", [(1, 8), (3, 8), (3, 5)])
def test_reference_gemm_smoke_from_reference_layout_bytes(ipus, oracle, ctx, batch, tiles):
    """The reference's GEMM smoke graph (crates/ipu-tests/src/main.rs:595-613):
    left [batch, tiles, 64] in amp_left(64, tiles), right [1, 64, 64 tiles] in
    block_major_matrix(64, tiles), bytes built as run_gemm builds them
    (one-hot left selecting inner (7 b + t) % 64, right = gemm_right_value,
    main.rs:1079-1105, 2133-2136).  Every output is exact."""
    L = ipus.Layout
    g = ipus.ComputeGraph()
    left = g.host_input("left", [batch, tiles, 64])
    right = g.parameter("right", [1, 64, tiles * 64])
    g.set_outputs([g.gemm(left, right)])
    lf, rf = L.amp_left(64, tiles), L.block_major_matrix(64, tiles)
    cfg = (ipus.PackageConfig()
           .with_input(left, ipus.TensorFormat(ipus.PRECISION_F16, lf))
           .with_input(right, ipus.TensorFormat(ipus.PRECISION_F16, rf)))
    levels = np.array([0xBC00, 0xB800, 0x0000, 0x3800, 0x3C00], dtype=np.uint16)
    b, t = np.meshgrid(np.arange(batch), np.arange(tiles), indexing="ij")
    selected = (b * 7 + t) % 64
    lx = np.zeros((batch, tiles, 64), dtype=np.uint16)
    lx[b, t, selected] = 0x3C00
    inner, col = np.meshgrid(np.arange(64), np.arange(tiles * 64), indexing="ij")
    rx = levels[(inner * 3 + col) % 5].reshape(1, 64, tiles * 64)
    feeds = {"left": oracle.pack_tiled(lx, lx.shape, **oracle_layout_args(ipus, lf)),
             "right": oracle.pack_tiled(rx, rx.shape, **oracle_layout_args(ipus, rf))}
    pkg, (y,) = run_package(ipus, ctx, g, feeds, cfg)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_unshard", "ipu_stack_unshard",
                                         "ipu_stack_gemm_f16"]
    want = rx[0][selected]                               # [batch, tiles, 64 tiles]
    assert np.array_equal(y.reshape(batch, tiles, tiles * 64), want)


def test_reference_mlp_smoke_from_reference_layout_bytes(ipus, oracle, ctx):
    """The reference's MLP smoke (main.rs:614-634): left [tiles, 64] in
    amp_left(64, tiles), both [64, 64] weights in block_major_matrix(64,
    tiles) (tile 0 holds the whole weight, the other slices are empty),
    GEMM -> GELU -> GEMM -> GELU; checked against the oracle at the fp16 bar
    and the reference's own 0.02 bound (main.rs:1929-2033)."""
    tiles = 16
    L = ipus.Layout
    g = ipus.ComputeGraph()
    left = g.host_input("left", [tiles, 64])
    r0 = g.parameter("right.0", [64, 64])
    r1 = g.parameter("right.1", [64, 64])
    g.set_outputs([g.gelu(g.gemm(g.gelu(g.gemm(left, r0)), r1))])
    lf, rf = L.amp_left(64, tiles), L.block_major_matrix(64, tiles)
    cfg = (ipus.PackageConfig().with_input(left, ipus.TensorFormat(ipus.PRECISION_F16, lf))
           .with_input(r0, ipus.TensorFormat(ipus.PRECISION_F16, rf))
           .with_input(r1, ipus.TensorFormat(ipus.PRECISION_F16, rf)))
    x = synth(ipus, tiles * 64, 72, 1, scale=1.0)
    w0 = synth(ipus, 64 * 64, 72, 2, scale=0.125)
    w1 = synth(ipus, 64 * 64, 72, 3, scale=0.125)
    args_l, args_r = oracle_layout_args(ipus, lf), oracle_layout_args(ipus, rf)
    feeds = {"left": oracle.pack_tiled(x, [tiles, 64], **args_l),
             "right.0": oracle.pack_tiled(w0, [64, 64], **args_r),
             "right.1": oracle.pack_tiled(w1, [64, 64], **args_r)}
    assert feeds["right.0"].size == 64 * 64            # 15 empty slices
    pkg, (y,) = run_package(ipus, ctx, g, feeds, cfg)
    h = oracle.gelu_f16(oracle.gemm_f16(x, w0, tiles, 64, 64))
    want = oracle.f16_to_f32(oracle.gelu_f16(oracle.gemm_f16(h, w1, tiles, 64, 64)))
    got = oracle.f16_to_f32(y).reshape(-1)
    assert fp16_close(got, want, FP16_TOL)
    assert np.max(np.abs(got - want)) <= 0.02


def test_reference_attention_smoke_from_reference_layout_bytes(ipus, oracle, ctx):
    """The reference's attention smoke (main.rs:671-701, 1305-1505): Q
    [4, 17, 72] in attention_output(4, query_partitions), K and V [4, 19, 72]
    in attention_output(4, 1), N(0, 0.25); the fp32 output within the
    smoke's max 0.012 and rms 0.003 of the oracle."""
    heads, qr, kr, d = 4, 17, 19, 72
    active_tiles = 64
    qparts = min(qr, active_tiles // heads)
    kparts = -(-kr // 64)
    L = ipus.Layout
    g = ipus.ComputeGraph()
    q = g.host_input("query", [heads, qr, d])
    k = g.host_input("key", [heads, kr, d])
    v = g.host_input("value", [heads, kr, d])
    g.set_outputs([g.flash_attention(q, k, v)])
    qf, kf = L.attention_output(heads, qparts), L.attention_output(heads, kparts)
    cfg = (ipus.PackageConfig().with_input(q, ipus.TensorFormat(ipus.PRECISION_F16, qf))
           .with_input(k, ipus.TensorFormat(ipus.PRECISION_F16, kf))
           .with_input(v, ipus.TensorFormat(ipus.PRECISION_F16, kf)))
    qs = synth(ipus, heads * qr * d, 73, 1, scale=0.25)
    ks = synth(ipus, heads * kr * d, 73, 2, scale=0.25)
    vs = synth(ipus, heads * kr * d, 73, 3, scale=0.25)
    feeds = {"query": oracle.pack_tiled(qs, [heads, qr, d], **oracle_layout_args(ipus, qf)),
             "key": oracle.pack_tiled(ks, [heads, kr, d], **oracle_layout_args(ipus, kf)),
             "value": oracle.pack_tiled(vs, [heads, kr, d], **oracle_layout_args(ipus, kf))}
    pkg, (y,) = run_package(ipus, ctx, g, feeds, cfg)
    want = oracle.attention(oracle.f16_to_f32(qs), oracle.f16_to_f32(ks), oracle.f16_to_f32(vs),
                            heads, qr, kr, d, d)
    err = np.abs(y.reshape(-1) - want.reshape(-1))
    assert float(err.max()) <= 0.012 and float(np.sqrt(np.mean(err ** 2))) <= 0.003


def test_residual_and_bias_packages_fuse_and_match_two_launches(ipus, oracle, ctx):
    """x + x . W and x . W + bias plan one accumulate launch each; the fused
    package equals the GEMM and Add kernels run one after the other."""
    g = ipus.ComputeGraph()
    x = g.host_input("x", [2, 300, 256])
    w = g.parameter("w", [256, 256])
    bias = g.parameter("bias", [256])
    g.set_outputs([g.add(x, g.gemm(x, w)), g.add(g.gemm(x, w), bias)])
    pkg = ipus.build_package(g)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16_accumulate"] * 2
    xs = synth(ipus, 2 * 300 * 256, 53, 1).reshape(2, 300, 256)
    ws = synth(ipus, 256 * 256, 53, 2, scale=0.05).reshape(256, 256)
    bs = synth(ipus, 256, 53, 3)
    _, (res, biased) = run_package(ipus, ctx, g, {"x": xs, "w": ws, "bias": bs})
    n = 2 * 300 * 256
    dx, dw, db = ctx.upload(xs), ctx.upload(ws), ctx.upload(bs)
    prod, want = ctx.alloc(n * 2), ctx.alloc(n * 2)
    ctx.launch("ipu_stack_gemm_f16", prod, [dx, dw], [2, 300, 256, 256, 0, 0, 300 * 256, 0])
    ctx.launch("ipu_stack_add_f16", want, [dx, prod], [n, n, n])
    assert np.array_equal(res.reshape(-1), want.download(np.uint16))
    ctx.launch("ipu_stack_add_f16", want, [prod, db], [n, n, 256])
    assert np.array_equal(biased.reshape(-1), want.download(np.uint16))
    for b in (dx, dw, db, prod, want):
        b.free()

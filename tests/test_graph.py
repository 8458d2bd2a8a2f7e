"""CPU tests of the ComputeGraph surface and build_package's launch plan.

The randomized shape tests restate crates/ipu-codegen/src/graph.rs:806-966
(same case construction, own seeds); the error tests follow GraphError
(graph.rs:221-245)."""
from __future__ import annotations

import math
import random

import numpy as np
import pytest

RANDOM_CASES = 256


def dimension(rng):
    return rng.randint(1, 128)


def broadcast_batch(rng):
    rank = rng.randint(0, 4)
    left, right, out = [], [], []
    for _ in range(rank):
        extent = dimension(rng)
        kind = rng.randint(0, 2)
        l, r = (extent, extent) if kind == 0 else ((1, extent) if kind == 1 else (extent, 1))
        left.append(l)
        right.append(r)
        out.append(extent)
    return left, right, out


def test_randomized_batched_gemm_preserves_matrix_axes_and_broadcasts_batch(ipus):
    rng = random.Random(0x6A656D6D)
    for case in range(RANDOM_CASES):
        left, right, expected = broadcast_batch(rng)
        rows, inner, cols = dimension(rng), dimension(rng), dimension(rng)
        tl, tr = rng.random() < 0.5, rng.random() < 0.5
        left += [inner, rows] if tl else [rows, inner]
        right += [cols, inner] if tr else [inner, cols]
        expected += [rows, cols]
        g = ipus.ComputeGraph()
        l = g.host_input("left", left)
        r = g.parameter("right", right)
        out = g.gemm_with_options(l, r, tl, tr)
        assert g.value_shape(out) == tuple(expected), f"case {case}"


def test_randomized_attention_preserves_query_and_value_axes(ipus):
    rng = random.Random(0x6174746E)
    for case in range(RANDOM_CASES):
        qb, kb, expected = broadcast_batch(rng)
        qr, kr, kc, vc = dimension(rng), dimension(rng), dimension(rng), dimension(rng)
        g = ipus.ComputeGraph()
        q = g.host_input("q", qb + [qr, kc])
        k = g.host_input("k", kb + [kr, kc])
        v = g.host_input("v", kb + [kr, vc])
        causal = rng.random() < 0.5
        scale = None if rng.random() < 0.5 else rng.random() + 0.01
        out = g.flash_attention_with_options(q, k, v, causal, scale)
        assert g.value_shape(out) == tuple(expected + [qr, vc]), f"case {case}"


def test_randomized_split_heads_preserves_every_projection_element(ipus):
    rng = random.Random(0x73706C69745F6864)
    for _ in range(RANDOM_CASES):
        batch, rows = rng.randint(1, 8), rng.randint(1, 256)
        heads, width = rng.randint(1, 32), rng.randint(1, 128)
        g = ipus.ComputeGraph()
        x = g.host_input("projection", [batch, rows, heads * width])
        out = g.split_heads(x, heads)
        assert g.value_shape(out) == (batch * heads, rows, width)


def test_randomized_attention_rejects_nonpositive_or_nonfinite_scales(ipus):
    rng = random.Random(0x7363616C)
    for case in range(RANDOM_CASES):
        scale = [0.0, -rng.random() - 1e-6, float("inf"), float("nan")][rng.randint(0, 3)]
        g = ipus.ComputeGraph()
        q, k, v = (g.host_input(n, [4, 8]) for n in "qkv")
        with pytest.raises(ipus.GraphError):
            g.flash_attention_with_options(q, k, v, rng.random() < 0.5, scale)


def test_graph_errors(ipus):
    g = ipus.ComputeGraph()
    with pytest.raises(ipus.GraphError, match="graph name must not be empty"):
        g.host_input("", [1])
    x = g.host_input("x", [4, 8])
    with pytest.raises(ipus.GraphError, match="is not available"):
        g.gelu(12345)
    with pytest.raises(ipus.GraphError, match="inner dimensions do not match"):
        g.gemm(x, x)
    with pytest.raises(ipus.GraphError, match="rank at least two"):
        g.gemm(g.host_input("v", [8]), x)
    with pytest.raises(ipus.GraphError, match="cannot be broadcast"):
        g.add(x, g.host_input("y", [3, 8]))
    with pytest.raises(ipus.GraphError, match="divisible by heads"):
        g.split_heads(g.host_input("p", [1, 4, 10]), 3)
    with pytest.raises(ipus.GraphError, match="nonzero heads"):
        g.split_heads(x, 2)
    with pytest.raises(ipus.GraphError, match="head or sequence"):
        g.flash_attention(x, g.host_input("k", [4, 7]), x)


def test_repeat_semantics_and_errors(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("input", [1, 64])
    weights = [g.parameter(f"layer.{i}.weight", [64, 64]) for i in range(3)]
    seq = g.value_sequence("layer weights", weights)
    out = g.repeat(3, [x], [], [seq],
                   lambda body, a: [body.add(a.carried[0], body.gemm(a.carried[0], a.iterated[0]))])
    assert g.value_shape(out[0]) == (1, 64)
    g.set_outputs(out)
    with pytest.raises(ipus.GraphError, match="repeat count must be nonzero"):
        g.repeat(0, [x], [], [], lambda b, a: [a.carried[0]])
    with pytest.raises(ipus.GraphError, match="entries for 4 iterations"):
        g.repeat(4, [x], [], [seq], lambda b, a: [a.carried[0]])
    with pytest.raises(ipus.GraphError, match="yielded 0 values for 1 carried"):
        g.repeat(1, [x], [], [], lambda b, a: [])
    with pytest.raises(ipus.GraphError, match="does not have the shape"):
        g.repeat(1, [x], [weights[0]], [], lambda b, a: [a.invariants[0]])
    with pytest.raises(ipus.GraphError, match="different shape from its first entry"):
        g.value_sequence("bad", [weights[0], x])
    # body values do not escape the region
    captured = []

    def body(b, a):
        captured.append(b.gelu(a.carried[0]))
        return [captured[-1]]

    g.repeat(1, [x], [], [], body)
    with pytest.raises(ipus.GraphError, match="is not available"):
        g.gelu(captured[0])
    # a failing body leaves the graph usable
    with pytest.raises(ipus.GraphError):
        g.repeat(1, [x], [], [], lambda b, a: [b.gemm(a.carried[0], a.carried[0])])
    g.gelu(x)


def test_build_package_mlp_plan(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("input", [4096, 4096])
    w1 = g.parameter("w1", [4096, 16384])
    w2 = g.parameter("w2", [16384, 4096])
    y = g.gemm(g.gelu(g.gemm(x, w1)), w2)
    g.set_outputs([y])
    pkg = ipus.build_package(g)
    # The GELU of the first GEMM's result is fused into its epilogue.
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16"]
    assert pkg.steps[0][2][:4] == (1, 4096, 16384, 4096)
    assert [t.name for t in pkg.inputs] == ["input", "w1", "w2"]
    assert pkg.outputs[0].name == "output.0" and pkg.outputs[0].shape == (4096, 4096)
    # only gelu(hidden) (128 MiB) lives in the arena
    assert pkg.arena_bytes == 4096 * 16384 * 2


def test_split_k_plan_for_few_tiles_and_long_k(ipus):
    """The reference's SigLIP MLP shape at one image (729 tokens) with a
    doubled hidden width: its second GEMM has 3 x 5 output tiles and K =
    8608, so it is split over K into fp32 partials (an arena value) and
    summed; GELU after the first GEMM fuses into that GEMM, a GELU after a
    split GEMM into the reduction."""
    g = ipus.ComputeGraph()
    x = g.host_input("x", [729, 1152])
    w1 = g.parameter("w1", [1152, 8608])
    w2 = g.parameter("w2", [8608, 1152])
    g.set_outputs([g.gelu(g.gemm(g.gelu(g.gemm(x, w1)), w2))])
    pkg = ipus.build_package(g)
    syms = [s[0] for s in pkg.steps]
    assert syms == ["ipu_stack_gemm_f16_gelu", "ipu_stack_gemm_f16_split",
                    "ipu_stack_reduce_splits_f16"]
    split, reduce = pkg.steps[1][2], pkg.steps[2][2]
    assert split[:4] == (1, 729, 1152, 8608)
    splits = split[8]
    assert 2 <= splits <= 16
    assert reduce == (splits, 729 * 1152, 1)  # GELU fused into the reduction
    # Enough work per tile, or short K: no split.
    g2 = ipus.ComputeGraph()
    a = g2.host_input("a", [4096, 1024])
    b = g2.parameter("b", [1024, 4096])
    g2.set_outputs([g2.gemm(a, b)])
    assert [s[0] for s in ipus.build_package(g2).steps] == ["ipu_stack_gemm_f16"]
    g3 = ipus.ComputeGraph()
    a = g3.host_input("a", [256, 512])
    b = g3.parameter("b", [512, 256])
    g3.set_outputs([g3.gemm(a, b)])
    assert [s[0] for s in ipus.build_package(g3).steps] == ["ipu_stack_gemm_f16"]


def _single_gemm_package(ipus, m, n, k, config=None):
    g = ipus.ComputeGraph()
    a = g.host_input("a", [m, k])
    b = g.parameter("b", [k, n])
    g.set_outputs([g.gemm(a, b)])
    return ipus.build_package(g, config) if config else ipus.build_package(g)


@pytest.mark.parametrize("m,n,k,splits", [
    # tiles = ceil(m/256) * ceil(n/256); splits = ceil(k / c) with
    # c = 64 * ceil(ceil(k / want) / 64), want = min(16, k // 1024, 64 // tiles).
    (729, 1152, 8608, 4),   # 15 tiles: want 4, c = 2176
    (729, 1152, 4304, 1),   # k < 6144: the small-tile kernel, one launch
    (256, 256, 8192, 8),    # 1 tile: want 8, c = 1024
    (1024, 1024, 8192, 4),  # 16 tiles: want 4, c = 2048
    (64, 64, 40000, 16),    # 1 tile: want 16, c = 2560, 15.6 -> 16
    (2048, 2048, 8192, 1),  # 64 tiles: want 1, one launch
    (729, 1152, 1960, 1),   # k < 6144: one launch
    (729, 1152, 8604, 1),   # k not a multiple of 8: one launch
    (729, 1150, 8608, 1),   # n not a multiple of 8: one launch
])
def test_split_k_plan_counts(ipus, m, n, k, splits):
    """The planner's split count for few-tile, long-K GEMMs, and the arena
    room for the fp32 partials when it splits."""
    pkg = _single_gemm_package(ipus, m, n, k)
    syms = [s[0] for s in pkg.steps]
    if splits == 1:
        assert syms[0] != "ipu_stack_gemm_f16_split"
        assert "ipu_stack_reduce_splits_f16" not in syms
        return
    assert syms == ["ipu_stack_gemm_f16_split", "ipu_stack_reduce_splits_f16"]
    assert pkg.steps[0][2][8] == splits
    assert pkg.steps[1][2] == (splits, m * n, 0)
    assert pkg.arena_bytes >= splits * m * n * 4


def test_split_k_not_planned_for_f32(ipus):
    pkg = _single_gemm_package(ipus, 729, 1152, 4304, ipus.PackageConfig(compute_precision="f32"))
    syms = [s[0] for s in pkg.steps]
    assert "ipu_stack_gemm_f32" in syms and "ipu_stack_gemm_f16_split" not in syms


def test_gemm_gelu_fusion_needs_a_private_result(ipus):
    # The GEMM result is also an output: both launches stay.
    g = ipus.ComputeGraph()
    x = g.host_input("x", [256, 256])
    w = g.parameter("w", [256, 256])
    h = g.gemm(x, w)
    g.set_outputs([g.gelu(h), h])
    assert [s[0] for s in ipus.build_package(g).steps][:2] == [
        "ipu_stack_gemm_f16", "ipu_stack_gelu_tanh_approx_f16"]
    # The GEMM result has a second reader.
    g = ipus.ComputeGraph()
    x = g.host_input("x", [256, 256])
    w = g.parameter("w", [256, 256])
    h = g.gemm(x, w)
    g.set_outputs([g.add(g.gelu(h), h)])
    steps = [s[0] for s in ipus.build_package(g).steps]
    assert steps[:2] == ["ipu_stack_gemm_f16", "ipu_stack_gelu_tanh_approx_f16"]
    # fp32 compute: the GEMM result is cast before the GELU, no fusion.
    g = ipus.ComputeGraph()
    x = g.host_input("x", [256, 256])
    w = g.parameter("w", [256, 256])
    g.set_outputs([g.gelu(g.gemm(x, w))])
    steps = [s[0] for s in ipus.build_package(g, ipus.PackageConfig(compute_precision="f32")).steps]
    assert "ipu_stack_gemm_f16_gelu" not in steps


def test_gemm_add_fusion_plans(ipus):
    """A Gemm read only by the Add after it becomes one accumulate launch
    (C = addend + A . B) when the addend broadcasts as whole rows or
    matrices; otherwise both launches stay."""
    def steps(build, config=None):
        g = ipus.ComputeGraph()
        g.set_outputs([build(g)])
        pkg = ipus.build_package(g, config) if config else ipus.build_package(g)
        return [(s[0], s[2]) for s in pkg.steps]

    # residual x + x . W per Repeat layer: one launch a layer (graph.rs:12-33)
    g = ipus.ComputeGraph()
    x = g.host_input("x", [64, 64])
    seq = g.value_sequence("layers", [g.parameter(f"w{i}", [64, 64]) for i in range(4)])
    g.set_outputs(g.repeat(4, [x], [], [seq], lambda b, a: [
        b.add(a.carried[0], b.gemm(a.carried[0], a.iterated[0]))]))
    pkg = ipus.build_package(g)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16_accumulate"] * 4
    assert all(s[1] == 3 and s[2][8:] == (0, 64) for s in pkg.steps)
    # bias over the rows, either operand order
    for order in (0, 1):
        def bias(g, order=order):
            y = g.gemm(g.host_input("x", [128, 256]), g.parameter("w", [256, 512]))
            b = g.parameter("b", [512])
            return g.add(y, b) if order == 0 else g.add(b, y)
        assert steps(bias) == [("ipu_stack_gemm_f16_accumulate",
                                (1, 128, 512, 256, 0, 0, 0, 0, 0, 0))]
    # batched product and a batched residual
    def batched(g):
        x = g.host_input("x", [2, 3, 64, 64])
        return g.add(g.gemm(x, g.parameter("w", [64, 32])), g.host_input("r", [2, 3, 64, 32]))
    assert steps(batched) == [("ipu_stack_gemm_f16_accumulate",
                               (6, 64, 32, 64, 0, 0, 4096, 0, 2048, 32))]
    # the addend broadcast over the batch
    def shared(g):
        x = g.host_input("x", [2, 3, 64, 64])
        return g.add(g.gemm(x, g.parameter("w", [64, 32])), g.host_input("r", [64, 32]))
    assert steps(shared)[0][1][8:] == (0, 32)
    # not expressible: a column broadcast, a partial batch broadcast
    def column(g):
        y = g.gemm(g.host_input("x", [64, 64]), g.parameter("w", [64, 64]))
        return g.add(y, g.host_input("c", [64, 1]))
    assert [s[0] for s in steps(column)] == ["ipu_stack_gemm_f16", "ipu_stack_add_broadcast_f16"]
    def partial(g):
        y = g.gemm(g.host_input("x", [2, 3, 64, 64]), g.parameter("w", [64, 64]))
        return g.add(y, g.host_input("r", [2, 1, 64, 64]))
    assert [s[0] for s in steps(partial)] == ["ipu_stack_gemm_f16", "ipu_stack_add_broadcast_f16"]
    # the product also read elsewhere, and fp32 compute: no fusion
    def shared_product(g):
        y = g.gemm(g.host_input("x", [64, 64]), g.parameter("w", [64, 64]))
        return g.add(g.add(y, g.host_input("r", [64, 64])), y)
    assert steps(shared_product)[0][0] == "ipu_stack_gemm_f16"
    def plain(g):
        y = g.gemm(g.host_input("x", [64, 64]), g.parameter("w", [64, 64]))
        return g.add(y, g.host_input("r", [64, 64]))
    assert "ipu_stack_gemm_f16_accumulate" not in [
        s[0] for s in steps(plain, ipus.PackageConfig(compute_precision="f32"))]
    # a split-K GEMM fuses into its reduction
    def split(g):
        y = g.gemm(g.host_input("x", [729, 8608]), g.parameter("w", [8608, 1152]))
        return g.add(g.host_input("r", [729, 1152]), y)
    (s0, _), (s1, sc) = steps(split)
    assert s0 == "ipu_stack_gemm_f16_split" and s1 == "ipu_stack_reduce_splits_accumulate_f16"
    assert sc[1:] == (1, 729, 1152, 0, 1152)


def _projected_attention(ipus, b=2, s=128, d=256, heads=2):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [b, s, d])
    proj = [g.gemm(x, g.parameter(n, [d, d])) for n in ("wq", "wk", "wv")]
    q, k, v = (g.split_heads(p, heads) for p in proj)
    return g, proj, (q, k, v)


def test_split_heads_feeding_attention_is_a_strided_view(ipus):
    # graph.rs:338-362 structure: the three head splits become the heads
    # layout of one attention launch, and their buffers leave the arena.
    g, proj, (q, k, v) = _projected_attention(ipus)
    g.set_outputs([g.flash_attention_with_options(q, k, v, causal=True)])
    pkg = ipus.build_package(g)
    syms = [s[0] for s in pkg.steps]
    assert "ipu_stack_split_heads" not in syms
    assert syms[-1] == "ipu_stack_flash_attention_heads_f16"
    assert pkg.steps[-1][2][8:] == (2, 2, 2)  # query, key, value heads
    assert pkg.steps[-1][2][:5] == (4, 128, 128, 128, 128)
    # only the three projections (2 * 128 * 256 fp16 each) are in the arena
    assert pkg.arena_bytes == 3 * 2 * 128 * 256 * 2


def test_split_heads_with_another_reader_is_copied(ipus):
    # The split K is also a graph output: its copy stays and only Q and V
    # are read through the view.
    g, proj, (q, k, v) = _projected_attention(ipus)
    g.set_outputs([g.flash_attention_with_options(q, k, v, causal=False), k])
    pkg = ipus.build_package(g)
    syms = [s[0] for s in pkg.steps]
    assert syms.count("ipu_stack_split_heads") == 1
    att = [s for s in pkg.steps if s[0].startswith("ipu_stack_flash_attention")]
    assert att[0][0] == "ipu_stack_flash_attention_heads_f16" and att[0][2][8:] == (2, 1, 2)
    # fp32 compute: the split result is cast before attention, no view
    g, proj, (q, k, v) = _projected_attention(ipus)
    g.set_outputs([g.flash_attention_with_options(q, k, v, causal=False)])
    pkg = ipus.build_package(g, ipus.PackageConfig(compute_precision="f32"))
    syms = [s[0] for s in pkg.steps]
    assert syms.count("ipu_stack_split_heads") == 3
    assert "ipu_stack_flash_attention_online_f16" in syms


def test_build_package_arena_reuses_dead_values(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [1024, 1024])
    v = x
    for _ in range(6):
        v = g.gelu(v)
    g.set_outputs([v])
    pkg = ipus.build_package(g)
    # a chain only ever needs two intermediates alive at once
    assert pkg.arena_bytes == 2 * 1024 * 1024 * 2


def test_build_package_precisions_and_casts(ipus):
    g = ipus.ComputeGraph()
    q = g.host_input("q", [2, 64, 64])
    att = g.flash_attention_with_options(q, q, q, causal=True)
    w = g.parameter("w", [64, 64])
    out = g.gemm(att, w)
    g.set_outputs([out, att])
    pkg = ipus.build_package(g)
    assert pkg.precision(att) == ipus.PRECISION_F32   # mid.rs:2064-2067
    assert pkg.precision(out) == ipus.PRECISION_F16
    symbols = [s[0] for s in pkg.steps]
    assert symbols[:3] == ["ipu_stack_flash_attention_online_f16", "ipu_stack_cast_f32_f16",
                           "ipu_stack_gemm_f16"]
    assert pkg.outputs[1].precision == ipus.PRECISION_F32
    pkg16 = ipus.build_package(g, ipus.PackageConfig(attention_output_f16=True))
    assert "ipu_stack_cast_f32_f16" not in [s[0] for s in pkg16.steps]


def test_build_package_memory_chain_plan(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [8192, 8192])
    t = g.transpose(x)
    bm = g.rearrange(t, ipus.ORDER_BLOCK_MAJOR, 64, 64)
    r = g.reduce_rows(bm)
    g.set_outputs([bm, r])
    pkg = ipus.build_package(g)
    assert [s[0] for s in pkg.steps] == [
        "ipu_stack_transpose_f16", "ipu_stack_rearrange_row_major_f16",
        "ipu_stack_reduce_rows_f16"]
    assert pkg.steps[2][2] == (8192, 8192, ipus.ORDER_BLOCK_MAJOR, 64, 64)
    assert pkg.outputs[0].order == ipus.ORDER_BLOCK_MAJOR
    assert pkg.outputs[1].shape == (8192,) and pkg.outputs[1].precision == ipus.PRECISION_F32


def test_build_package_repeat_unrolls_with_iterated_weights(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("input", [1, 64])
    ws = [g.parameter(f"w{i}", [64, 64]) for i in range(4)]
    seq = g.value_sequence("weights", ws)
    out = g.repeat(4, [x], [], [seq], lambda b, a: [b.gemm(a.carried[0], a.iterated[0])])
    g.set_outputs(out)
    pkg = ipus.build_package(g)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f16"] * 4


def test_build_package_output_of_input_is_copied(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [16])
    g.set_outputs([x, x])
    pkg = ipus.build_package(g)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_copy", "ipu_stack_copy"]


def test_build_package_f32_compute(ipus):
    g = ipus.ComputeGraph()
    a = g.host_input("a", [4096, 4096])
    b = g.parameter("b", [4096, 4096])
    g.set_outputs([g.gemm(a, b)])
    pkg = ipus.build_package(g, ipus.PackageConfig(compute_precision="f32"))
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gemm_f32"]
    assert pkg.inputs[0].precision == ipus.PRECISION_F32


@pytest.mark.parametrize("build", [
    lambda ipus, g: g.gemm(g.host_input("x", [0, 4096]), g.parameter("w", [4096, 256])),
    lambda ipus, g: g.gemm(g.host_input("x", [256, 4096]), g.parameter("w", [4096, 0])),
    lambda ipus, g: g.gemm(g.host_input("x", [0, 256, 4096]), g.parameter("w", [0, 4096, 256])),
    lambda ipus, g: g.gemm(g.host_input("x", [256, 0]), g.parameter("w", [0, 256])),
    lambda ipus, g: g.transpose(g.host_input("x", [0, 64])),
    lambda ipus, g: g.transpose(g.host_input("x", [3, 64, 0])),
    lambda ipus, g: g.rearrange(g.host_input("x", [0, 64]), ipus.ORDER_BLOCK_MAJOR, 64, 64),
    lambda ipus, g: g.reduce_rows(g.host_input("x", [64, 0])),
    lambda ipus, g: g.reduce_rows(g.host_input("x", [0, 64])),
    lambda ipus, g: g.gelu(g.host_input("x", [0, 7])),
    lambda ipus, g: g.flash_attention(g.host_input("q", [2, 0, 64]), g.host_input("k", [2, 5, 64]),
                                      g.host_input("v", [2, 5, 64])),
    lambda ipus, g: g.flash_attention(g.host_input("q", [2, 5, 64]), g.host_input("k", [2, 0, 64]),
                                      g.host_input("v", [2, 0, 64])),
])
def test_build_package_zero_extents(ipus, build):
    """Zero extents are legal graph values (graph.rs shape inference accepts
    them); the plan must build without dividing by a zero matrix size."""
    g = ipus.ComputeGraph()
    g.set_outputs([build(ipus, g)])
    pkg = ipus.build_package(g)
    out = pkg.outputs[0]
    assert out.nbytes == math.prod(out.shape) * (4 if out.precision == ipus.PRECISION_F32 else 2)
    for symbol, _inputs, scalars in pkg.steps:
        assert all(0 <= s <= 0xFFFFFFFF for s in scalars), symbol


def test_build_package_rejects_empty_batch_broadcast_to_one(ipus):
    """graph.rs:755-777 broadcasts extents 0 and 1 to 1 (the larger), so a
    GEMM or Add result can be non-empty while an operand holds no data: the
    plan refuses instead of reading past an empty buffer."""
    g = ipus.ComputeGraph()
    out = g.gemm(g.host_input("x", [0, 256, 64]), g.parameter("w", [64, 256]))
    assert g.value_shape(out) == (1, 256, 256)
    g.set_outputs([out])
    with pytest.raises(ipus.PackageBuildError):
        ipus.build_package(g)
    g = ipus.ComputeGraph()
    out = g.add(g.host_input("x", [0, 8]), g.host_input("y", [1, 8]))
    assert g.value_shape(out) == (1, 8)
    g.set_outputs([out])
    with pytest.raises(ipus.PackageBuildError):
        ipus.build_package(g)


def test_build_package_splits_u32_element_counts(ipus):
    """Values of 2^32 elements and more fit in HBM: element-wise steps whose
    count scalar would overflow u32 are split into launches of at most 2^30
    elements instead of being truncated."""
    shape = [65536, 65538]
    n = 65536 * 65538                       # 2^32 + 2^17 elements
    g = ipus.ComputeGraph()
    x = g.host_input("x", shape)
    g.set_outputs([g.gelu(x), x])
    pkg = ipus.build_package(g)
    gelu = [s for s in pkg.steps if s[0] == "ipu_stack_gelu_tanh_approx_f16"]
    assert [s[2][0] for s in gelu] == [1 << 30] * 4 + [1 << 17]
    copies = [s for s in pkg.steps if s[0] == "ipu_stack_copy"]
    assert sum(s[2][0] for s in copies) == 2 * n and max(s[2][0] for s in copies) == 1 << 30
    # An fp32 graph value of 2^32 + 2^17 elements cast for GELU (F32 compute).
    g = ipus.ComputeGraph()
    x = g.host_input("x", shape)
    g.set_outputs([g.gelu(x)])
    pkg = ipus.build_package(g, ipus.PackageConfig(compute_precision="f32"))
    casts = [s for s in pkg.steps if s[0] == "ipu_stack_cast_f32_f16"]
    assert sum(s[2][0] for s in casts) == n and len(casts) == 5


def test_build_package_batched_gemm_with_u32_overflowing_stride(ipus):
    """A batched operand whose matrix holds 2^32 elements or more cannot pass
    its batch stride as a u32 scalar: the plan launches per batch."""
    g = ipus.ComputeGraph()
    x = g.host_input("x", [2, 65536, 65544])
    w = g.parameter("w", [65544, 8])
    g.set_outputs([g.gemm(x, w)])
    pkg = ipus.build_package(g)
    gemms = [s for s in pkg.steps if s[0] == "ipu_stack_gemm_f16"]
    assert len(gemms) == 2 and all(s[2][0] == 1 and s[2][6] == 0 for s in gemms)


# ---------------------------------------------------------------------------
# Declared input formats (PipelineConfig::with_input, config.rs:310-320)
# ---------------------------------------------------------------------------
def oracle_layout_args(ipus, layout):
    """The oracle's packer arguments for a product Layout (test glue)."""
    kinds = {ipus.ORDER_ROW_MAJOR: (0, 0), ipus.ORDER_AMP_LEFT: (1, 0),
             ipus.ORDER_AMP_TRANSPOSED_LEFT: (1, 1), ipus.ORDER_AMP_TRANSPOSED_RIGHT: (1, 2),
             ipus.ORDER_AMP_OUTPUT: (1, 3), ipus.ORDER_AMP_TRANSPOSED_OUTPUT: (1, 4),
             ipus.ORDER_BLOCK_MAJOR: (2, 0), ipus.ORDER_BLOCK_MAJOR_TRANSPOSED: (2, 1)}
    kind, variant = kinds[layout.order]
    axes = [dict(axis=("end" if a.axis.from_end else "start", a.axis.index),
                 partitions=a.partitions, block_size=a.block_size,
                 padding_groups=a.padding_groups,
                 padding_multiple=a.padding_multiple or a.block_size,
                 shard_padding_multiple=a.shard_padding_multiple,
                 zero_padding=a.padding == ipus.PADDING_ZERO,
                 tile_stride=a.tile_stride or None) for a in layout.axes]
    return dict(kind=kind, variant=variant, tile_count=layout.tile_count,
                replicas=layout.replicas, axes=axes, row_block=layout.row_block,
                column_block=layout.column_block)


FORMAT_CASES = [
    ("amp_left", [3, 4, 64], lambda L: L.amp_left(64, 4)),
    ("amp_left_padded", [2, 5, 40], lambda L: L.amp_left(64, 5)),
    ("block_major", [1, 64, 256], lambda L: L.block_major_matrix(64, 4)),
    ("block_major_empty_shards", [64, 64], lambda L: L.block_major_matrix(64, 4)),
    ("attention_output", [4, 17, 72], lambda L: L.attention_output(4, 5)),
    ("attention_key", [4, 19, 72], lambda L: L.attention_key(4, 1)),
    ("attention_query", [4, 17, 72], lambda L: L.attention_query(4, 3)),
    ("attention_block_major_kv", [4, 130, 72], lambda L: L.attention_block_major_key_value(4, 3)),
    ("amp_output", [6, 40], lambda L: L.amp_output(3)),
    ("transposed_block_major", [100, 64], lambda L: L.transposed_block_major_matrix_storage(
        64, 64, 2, 1, 1)),
    ("block_major_copies", [64, 128], lambda L: L.block_major_matrix_storage(64, 64, 2, 1, 2)),
]


@pytest.mark.parametrize("name,shape,make", FORMAT_CASES, ids=[c[0] for c in FORMAT_CASES])
def test_declared_input_format_plans_one_unshard(ipus, oracle, name, shape, make):
    """A with_input format makes the input binding hold the shards' bytes
    (the oracle's packing of the same layout has the same size) and plans
    one ipu_stack_unshard step ahead of the consumer."""
    layout = make(ipus.Layout)
    g = ipus.ComputeGraph()
    x = g.host_input("x", shape)
    g.set_outputs([g.gelu(x)])
    cfg = ipus.PackageConfig().with_input(x, ipus.TensorFormat(ipus.PRECISION_F16, layout))
    pkg = ipus.build_package(g, cfg)
    n = int(np.prod(shape))
    packed = oracle.pack_tiled(np.ones(n, np.uint16), shape, **oracle_layout_args(ipus, layout))
    assert pkg.inputs[0].nbytes == packed.nbytes
    assert pkg.inputs[0].shards == layout.tile_count
    assert [s[0] for s in pkg.steps][:2] == ["ipu_stack_unshard", "ipu_stack_gelu_tanh_approx_f16"]


def test_declared_row_major_identity_needs_no_conversion(ipus):
    """Row-sharded row-major data without padding is already the tensor."""
    g = ipus.ComputeGraph()
    x = g.host_input("x", [8, 64])
    g.set_outputs([g.gelu(x)])
    cfg = ipus.PackageConfig().with_input(
        x, ipus.TensorFormat(ipus.PRECISION_F16, ipus.Layout.row_sharded(4)))
    pkg = ipus.build_package(g, cfg)
    assert [s[0] for s in pkg.steps] == ["ipu_stack_gelu_tanh_approx_f16"]
    assert pkg.inputs[0].nbytes == 8 * 64 * 2


def test_automatic_input_fixes_precision_and_casts(ipus):
    """with_automatic_input(value, F32): the host writes fp32 row-major and
    the plan casts to the fp16 compute precision."""
    g = ipus.ComputeGraph()
    x = g.host_input("x", [64, 64])
    w = g.parameter("w", [64, 64])
    g.set_outputs([g.gemm(x, w)])
    cfg = ipus.PackageConfig().with_automatic_input(x, ipus.PRECISION_F32)
    pkg = ipus.build_package(g, cfg)
    assert pkg.inputs[0].precision == ipus.PRECISION_F32 and pkg.inputs[0].nbytes == 64 * 64 * 4
    assert [s[0] for s in pkg.steps] == ["ipu_stack_cast_f32_f16", "ipu_stack_gemm_f16"]


@pytest.mark.parametrize("shape,make,message", [
    ([4, 40], lambda L: L.row_major(2, [ipus_axis(1, 2, 16)]), "multiple"),  # Reject, 40 % 16
    ([3, 4, 64], lambda L: replace_tiles(L.amp_left(64, 4), 5), "tile count"),
    ([4, 64], lambda L: L.row_major(4, [ipus_axis(2, 2, 1).with_tile_stride(1),
                                        ipus_axis(1, 2, 1).with_tile_stride(1)]), "strides"),
])
def test_declared_input_format_errors(ipus, shape, make, message):
    import re
    g = ipus.ComputeGraph()
    x = g.host_input("x", shape)
    g.set_outputs([g.gelu(x)])
    cfg = ipus.PackageConfig().with_input(x, ipus.TensorFormat(ipus.PRECISION_F16,
                                                               make(ipus.Layout)))
    with pytest.raises(ipus.PackageBuildError) as err:
        ipus.build_package(g, cfg)
    assert re.search(message, err.value.message)


def ipus_axis(from_end, partitions, block):
    import importlib
    m = importlib.import_module("ipu_stack_amd")
    return m.AxisTiling(m.TensorAxis(from_end), partitions, block)


def replace_tiles(layout, tiles):
    import dataclasses
    return dataclasses.replace(layout, tile_count=tiles)


def test_input_format_for_a_non_input_is_rejected(ipus):
    g = ipus.ComputeGraph()
    x = g.host_input("x", [16, 16])
    y = g.gelu(x)
    g.set_outputs([y])
    cfg = ipus.PackageConfig().with_automatic_input(y, ipus.PRECISION_F16)
    with pytest.raises(ipus.PackageBuildError):
        ipus.build_package(g, cfg)

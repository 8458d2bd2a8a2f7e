"""Pins the CPU oracle before it is trusted as the GPU checker.

The reference ships no golden-vector files (its tests are seeded property
tests and hardware known-answer runs), so each oracle function is pinned by
(a) the reference's own known-answer designs restated here, (b) independent
expressions of the same layout taken from the reference's DEVICE code
(device/*.S, device/*.cpp) where the oracle follows storage.rs, (c) library
routines (numpy's IEEE float16, float64 matmul, broadcasting) and (d)
closed-form invariants chosen so a dropped term, wrong sign/index or swapped
operand fails.  Fixtures in tests/golden/ are checked too."""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------------------
# binary16 conversion (half 2.7.1 semantics: IEEE round to nearest even)
# ---------------------------------------------------------------------------
def test_f16_to_f32_every_pattern_matches_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0x16)
    raw = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8,
                         2.9802322e-08, 6.1035156e-05, 6.0975552e-05, np.inf, -np.inf, 1.0,
                         1.0009765625, 1.00048828125, 1.00146484375, 2049.0, 2051.0],
                        dtype=np.float32)
    values = np.concatenate([raw.view(np.float32), specials])
    ours = oracle.f32_to_f16(values)
    with np.errstate(over="ignore"):  # values beyond fp16 range round to inf by design
        ref = values.astype(np.float16).view(np.uint16)
    nan = np.isnan(values)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))


# ---------------------------------------------------------------------------
# Storage maps (storage.rs) against the device code's own address arithmetic
# ---------------------------------------------------------------------------
def test_block_major_64x16_matches_assembly_address_formula(oracle):
    """device/rearrange_block_major_f16.S:69-104: byte address
    (c/16)*2048 + (r/16)*512 + (r%16)*2 + (c%16)*32 for a 64 x N shard."""
    N = 48
    for r in range(64):
        for c in range(N):
            byte = (c // 16) * 2048 + (r // 16) * 512 + (r % 16) * 2 + (c % 16) * 32
            assert oracle.block_major_matrix_index(0, 64, 16, oracle.F16, 64, N, r, c) * 2 == byte


def test_block_major_matches_rearrange_cpp_target_2(oracle):
    """device/rearrange_f16.cpp:129-151 (TARGET_ORDER 2) for several blocks."""
    inner = 16
    for rb, cb, R, C in [(64, 16, 128, 64), (64, 64, 64, 128), (32, 32, 96, 64)]:
        for r in range(R):
            for c in range(C):
                panel = ((r // rb) * (C // cb) * (rb // inner) + (c // cb) * (rb // inner)
                         + (r % rb) // inner)
                dest = panel * inner * cb + r % inner + (c % cb) * inner
                assert oracle.block_major_matrix_index(0, rb, cb, oracle.F16, R, C, r, c) == dest


def test_transposed_right_matches_rearrange_cpp_target_1_and_asm(oracle):
    """device/rearrange_f16.cpp:76-90 (TARGET_ORDER 1) and, for a 64x16 shard,
    the plain row copy of device/rearrange_transposed_right_f16.S:27-55."""
    R, C = 64, 48
    for r in range(R):
        for c in range(C):
            panel = (r // 16) * (C // 16) + c // 16
            dest = panel * 256 + (r % 16) * 16 + c % 16
            assert oracle.amp_matrix_index(oracle.AMP_TRANSPOSED_RIGHT, oracle.F16, R, C, r, c) == dest
    for r in range(64):
        for c in range(16):
            assert oracle.amp_matrix_index(oracle.AMP_TRANSPOSED_RIGHT, oracle.F16, 64, 16, r, c) == r * 16 + c


def test_amp_left_matches_rearrange_amp_left_asm(oracle):
    """device/rearrange_amp_left_f16.S / rearrange_f16.cpp:98-100 (TARGET 0):
    (c/16)*PR*16 + r*16 + c%16."""
    PR, C = 37, 64
    for r in range(PR):
        for c in range(C):
            assert oracle.amp_matrix_index(oracle.AMP_LEFT, oracle.F16, PR, C, r, c) == \
                (c // 16) * PR * 16 + r * 16 + c % 16


def test_unpack_sources_match_unpack_cpp(oracle):
    """device/unpack_amp_f16.cpp:61-70 for both source orders."""
    PR, PC = 32, 48
    for r in range(PR):
        for c in range(PC):
            lp = c % 16 // 2
            pp = lp % 4 * 2 + lp // 4
            out_idx = (c // 16) * PR * 16 + r * 16 + pp * 2 + c % 2
            assert oracle.amp_matrix_index(oracle.AMP_OUTPUT, oracle.F16, PR, PC, r, c) == out_idx
            tl = (r // 16) * PC * 16 + c * 16 + r % 16
            assert oracle.amp_matrix_index(oracle.AMP_TRANSPOSED_LEFT, oracle.F16, PR, PC, r, c) == tl


def _unpack_vertex(source_order, matrices, lr, pr, lc, pc, source):
    """device/unpack_amp_f16.cpp:40-80 restated word for word: a pass over the
    physical rows of every matrix writes 32-bit words of two fp16 columns at
    matrixBase + row * physicalColumns + column; a word whose row or first
    column lies past the logical extent is 0, and so is a second lane past
    the logical columns.  Source and destination share matrixBase =
    matrix * physicalRows * physicalColumns."""
    words = source.astype(np.uint32)
    out = np.full(matrices * pr * pc // 2, 0xDEADBEEF, dtype=np.uint32)
    matrix_elements = pr * pc
    for matrix_row in range(matrices * pr):
        matrix, row = divmod(matrix_row, pr)
        base = matrix * matrix_elements
        for column in range(0, pc, 2):
            packed = 0
            if row < lr and column < lc:
                for lane in range(2):
                    c = column + lane
                    if c >= lc:
                        continue
                    if source_order == 0:
                        logical_pair = c % 16 // 2
                        physical_pair = logical_pair % 4 * 2 + logical_pair // 4
                        physical = (c // 16) * pr * 16 + row * 16 + physical_pair * 2 + c % 2
                    else:
                        physical = (row // 16) * pc * 16 + c * 16 + row % 16
                    packed |= int(words[base + physical]) << (lane * 16)
            out[(base + row * pc + column) // 2] = packed
    return out.view(np.uint16)


@pytest.mark.parametrize("source_order", [0, 1])
@pytest.mark.parametrize("matrices,lr,pr,lc,pc", [
    (1, 16, 16, 16, 16),    # one micro-panel, no padding
    (2, 30, 32, 40, 48),    # padding on both axes, two matrices
    (3, 17, 32, 33, 48),    # odd logical columns: a word with one real lane
    (2, 32, 32, 31, 32),    # column padding only
    (1, 5, 16, 64, 64),     # row padding only, four column panels
])
def test_unpack_to_row_major_matches_unpack_vertex(oracle, source_order, matrices, lr, pr, lc,
                                                   pc):
    """Pins or_unpack_to_row_major_f16's matrix base, destination pitch and zero
    padding against the vertex loop, with a source whose every element is
    distinct and nonzero (so a wrong base, pitch or pad rule shows)."""
    src = (np.arange(matrices * pr * pc, dtype=np.uint32) % 65535 + 1).astype(np.uint16)
    want = _unpack_vertex(source_order, matrices, lr, pr, lc, pc, src)
    got = oracle.unpack_to_row_major_f16(src, source_order, matrices, lr, pr, lc, pc)
    assert np.array_equal(got, want)
    # Padding is zero and every logical element appears once.
    got3 = got.reshape(matrices, pr, pc)
    assert not np.any(got3[:, lr:, :]) and not np.any(got3[:, :, lc:])
    assert np.unique(got3[:, :lr, :lc]).size == matrices * lr * lc


def test_amp_output_pair_permutation_matches_gelu_reorder_table(oracle):
    """crates/ipu-tests/src/diagnostic.rs:910-946: AMP-Output word s of a
    16-column group holds the logical pair permutation[s] of AMP-Left."""
    permutation = [0, 4, 1, 5, 2, 6, 3, 7]
    rows, cols = 5, 32
    for base in range(0, rows * cols // 2, 8):
        for s, d in enumerate(permutation):
            for lane in range(2):
                src = oracle.amp_matrix_coordinates(oracle.AMP_OUTPUT, oracle.F16, rows, cols,
                                                    (base + s) * 2 + lane)
                dst = oracle.amp_matrix_coordinates(oracle.AMP_LEFT, oracle.F16, rows, cols,
                                                    (base + d) * 2 + lane)
                assert src == dst


@pytest.mark.parametrize("role", [0, 1, 2, 3, 4])
def test_amp_maps_are_bijections(oracle, role):
    """storage.rs:822-895 style: index and coordinates are inverse bijections."""
    rng = np.random.default_rng(role)
    for _ in range(12):
        rows = int(rng.integers(1, 5)) * 16
        cols = int(rng.integers(1, 5)) * 16
        seen = set()
        for r in range(rows):
            for c in range(cols):
                idx = oracle.amp_matrix_index(role, oracle.F16, rows, cols, r, c)
                assert 0 <= idx < rows * cols
                assert oracle.amp_matrix_coordinates(role, oracle.F16, rows, cols, idx) == (r, c)
                seen.add(idx)
        assert len(seen) == rows * cols


@pytest.mark.parametrize("transposed", [0, 1])
def test_block_major_maps_are_bijections(oracle, transposed):
    for rb, cb, R, C in [(64, 16, 128, 32), (64, 64, 64, 128), (16, 8, 48, 24)]:
        if transposed:
            R, C = C, R
        seen = set()
        for r in range(R):
            for c in range(C):
                idx = oracle.block_major_matrix_index(transposed, rb, cb, oracle.F16, R, C, r, c)
                assert oracle.block_major_matrix_coordinates(transposed, rb, cb, oracle.F16, R, C,
                                                             idx) == (r, c)
                seen.add(idx)
        assert len(seen) == R * C


def test_block_major_64x64_blocks_are_contiguous(oracle):
    """storage.rs:428-527: with a 64-column block every 64x64 block is one
    contiguous 4096-element span."""
    R, C = 128, 192
    for br in range(R // 64):
        for bc in range(C // 64):
            idx = {oracle.block_major_matrix_index(0, 64, 64, oracle.F16, R, C, br * 64 + r,
                                                   bc * 64 + c)
                   for r in range(64) for c in range(64)}
            assert max(idx) - min(idx) == 4095 and min(idx) % 4096 == 0


@pytest.mark.parametrize("order", [0, 1, 2])
def test_rearrange_places_every_element_and_zero_pads(oracle, order):
    m, lr, pr, lc, pc = 2, 30, 32, 40, 48
    src = np.arange(m * lr * lc, dtype=np.uint16) + 1
    out = oracle.rearrange_row_major_f16(src, order, m, lr, pr, lc, pc, 32, 16)
    assert not np.any(out == 0xFFFF)            # every position written
    assert np.count_nonzero(out) == src.size    # padding is zero
    s3 = src.reshape(m, lr, lc)
    for mm in range(m):
        for r in range(0, lr, 7):
            for c in range(0, lc, 5):
                if order == 0:
                    idx = oracle.amp_matrix_index(0, oracle.F16, m * pr, pc, mm * pr + r, c)
                elif order == 1:
                    idx = mm * pr * pc + oracle.amp_matrix_index(2, oracle.F16, pr, pc, r, c)
                else:
                    idx = mm * pr * pc + oracle.block_major_matrix_index(0, 32, 16, oracle.F16,
                                                                         pr, pc, r, c)
                assert out[idx] == s3[mm, r, c]


def test_transpose_is_numpy_transpose(oracle):
    x = np.arange(3 * 5 * 7, dtype=np.uint16)
    assert np.array_equal(oracle.transpose_u16(x, 3, 5, 7),
                          x.reshape(3, 5, 7).transpose(0, 2, 1).reshape(-1))


# ---------------------------------------------------------------------------
# GEMM (diagnostic.rs:533-654)
# ---------------------------------------------------------------------------
def test_randomized_gemm_f32_matches_float64(oracle):
    """diagnostic.rs:855-907 restated: random shapes and transposes."""
    rng = np.random.default_rng(0x424C4153)
    for _ in range(128):
        M, K, N = (int(x) for x in rng.integers(1, 40, size=3))
        tl, tr = bool(rng.integers(2)), bool(rng.integers(2))
        A = rng.random((K, M) if tl else (M, K), dtype=np.float32) - 0.5
        B = rng.random((N, K) if tr else (K, N), dtype=np.float32) - 0.5
        got = oracle.gemm_f32(A, B, M, N, K, tl, tr).reshape(M, N)
        want = (A.T if tl else A).astype(np.float64) @ (B.T if tr else B).astype(np.float64)
        assert np.max(np.abs(got - want)) <= 2e-5


def test_gemm_f32_large_blocked_path(oracle):
    rng = np.random.default_rng(7)
    M, K, N = 300, 700, 1100   # crosses the MC/KC/NC blocking and edge tiles
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = rng.standard_normal((K, N), dtype=np.float32)
    got = oracle.gemm_f32(A, B, M, N, K).reshape(M, N)
    want = A.astype(np.float64) @ B.astype(np.float64)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= 1e-6


def test_gemm_batched_broadcast(oracle):
    rng = np.random.default_rng(8)
    A = rng.random((3, 20, 30), dtype=np.float32)
    B = rng.random((30, 10), dtype=np.float32)
    got = oracle.gemm_f32(A, B, 20, 10, 30, batches=3, left_batch_stride=600,
                          right_batch_stride=0).reshape(3, 20, 10)
    assert np.allclose(got, A.astype(np.float64) @ B.astype(np.float64), atol=1e-5)


def test_gemm_f16_one_hot_kat(oracle):
    """main.rs:1079-1105 with 2133-2136: one-hot rows select a 5-level right
    operand; the result is exact."""
    levels = np.array([0xBC00, 0xB800, 0x0000, 0x3800, 0x3C00], dtype=np.uint16)
    M, K, N = 64, 64, 128
    left = np.zeros((M, K), dtype=np.uint16)
    sel = (np.arange(M) * 7 + 3) % 64
    left[np.arange(M), sel] = 0x3C00
    right = levels[(np.arange(K)[:, None] * 3 + np.arange(N)[None, :]) % 5]
    got = oracle.gemm_f16(left, right, M, N, K).reshape(M, N)
    assert np.array_equal(got, right[sel])


def test_gemm_f16_constant_kat(oracle):
    """main.rs:1590-1591, 1788-1798: all-ones x 0.25 gives K * 0.25 exactly."""
    M, K, N = 8, 1024, 8
    got = oracle.gemm_f16(np.full(M * K, 0x3C00, np.uint16), np.full(K * N, 0x3400, np.uint16),
                          M, N, K)
    assert np.all(oracle.f16_to_f32(got) == K * 0.25)


def test_gemm_f16_is_quantized_fp32_product(oracle):
    rng = np.random.default_rng(9)
    M, K, N = 33, 65, 47
    a = (rng.random((M, K)) * 2 - 1).astype(np.float16)
    b = (rng.random((K, N)) * 2 - 1).astype(np.float16)
    got = oracle.gemm_f16(a.view(np.uint16), b.view(np.uint16), M, N, K).view(np.float16)
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float16).reshape(-1)
    ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulps.max() <= 1 and np.mean(ulps == 0) > 0.95


def test_gemm_f16_rows_matches_full(oracle):
    rng = np.random.default_rng(10)
    n = 96
    a = (rng.random(n * n) - 0.5).astype(np.float16).view(np.uint16)
    b = (rng.random(n * n) - 0.5).astype(np.float16).view(np.uint16)
    rows = np.array([0, 5, 95], dtype=np.uint32)
    full = oracle.gemm_f32(oracle.f16_to_f32(a), oracle.f16_to_f32(b), n, n, n).reshape(n, n)
    assert np.allclose(oracle.gemm_f16_rows(a, b, n, n, n, rows), full[rows], atol=1e-5)


# ---------------------------------------------------------------------------
# Attention (diagnostic.rs:711-780)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_attention_identity_values_expose_softmax(oracle, causal):
    """With V = I the output is the probability matrix itself: rows sum to 1,
    the causal upper triangle is 0 (diagnostic.rs:741-745), and ratios are
    exp(scale * (s_ij - s_ik)) of the raw scores."""
    rng = np.random.default_rng(11)
    S, D = 24, 16
    q = rng.standard_normal((S, D)).astype(np.float32)
    k = rng.standard_normal((S, D)).astype(np.float32)
    v = np.eye(S, dtype=np.float32)
    p = oracle.attention(q, k, v, 1, S, S, D, S, causal)
    assert np.allclose(p.sum(axis=1), 1.0, atol=1e-5)
    if causal:
        assert np.all(np.triu(p, 1) == 0)
    scores = (q.astype(np.float64) @ k.T.astype(np.float64)) / math.sqrt(D)
    i = S - 1
    for j in range(1, S):
        assert math.isclose(p[i, j] / p[i, 0], math.exp(scores[i, j] - scores[i, 0]),
                            rel_tol=1e-4)


def test_attention_zero_keys_give_prefix_means(oracle):
    """K = 0 makes every allowed key equally likely: O[i] = mean(V[0..i]) when
    causal, mean(V) otherwise."""
    rng = np.random.default_rng(12)
    S, D = 40, 8
    q = rng.standard_normal((S, D)).astype(np.float32)
    v = rng.standard_normal((S, D)).astype(np.float32)
    k = np.zeros((S, D), np.float32)
    causal = oracle.attention(q, k, v, 1, S, S, D, D, True)
    prefix = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    assert np.allclose(causal, prefix, atol=1e-5)
    full = oracle.attention(q, k, v, 1, S, S, D, D, False)
    assert np.allclose(full, v.mean(axis=0, dtype=np.float64), atol=1e-5)


def test_attention_scale_and_row_sampling(oracle):
    rng = np.random.default_rng(13)
    st, S, D = 3, 20, 8
    q = rng.standard_normal((st, S, D)).astype(np.float32)
    k = rng.standard_normal((st, S, D)).astype(np.float32)
    v = rng.standard_normal((st, S, D)).astype(np.float32)
    full = oracle.attention(q, k, v, st, S, S, D, D, False, scale=0.3)
    rows = [0, 7, 59]
    assert np.array_equal(oracle.attention(q, k, v, st, S, S, D, D, False, scale=0.3,
                                           row_list=rows), full[rows])
    # an explicit scale of 1/sqrt(D) equals the default (diagnostic.rs:733-736)
    assert np.allclose(oracle.attention(q, k, v, st, S, S, D, D, True, scale=1 / math.sqrt(D)),
                       oracle.attention(q, k, v, st, S, S, D, D, True), atol=1e-6)


def test_attention_single_key_is_that_value(oracle):
    rng = np.random.default_rng(14)
    q = rng.standard_normal((5, 8)).astype(np.float32)
    k = rng.standard_normal((1, 8)).astype(np.float32)
    v = rng.standard_normal((1, 6)).astype(np.float32)
    out = oracle.attention(q, k, v, 1, 5, 1, 8, 6, False)
    assert np.allclose(out, np.broadcast_to(v, (5, 6)), atol=1e-6)


# ---------------------------------------------------------------------------
# GELU (main.rs:1985-1987), reductions, add, split_heads
# ---------------------------------------------------------------------------
def test_gelu_special_values(oracle):
    assert oracle.gelu_reference(0.0) == 0.0
    for x in (10.0, 20.0, 100.0):
        assert oracle.gelu_reference(x) == pytest.approx(x, rel=1e-6)
    for x in (-10.0, -20.0):
        assert abs(oracle.gelu_reference(x)) < 1e-6
    # the tanh approximation, not the erf form: they differ at x = 1 in the 4th digit
    exact_tanh = 0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * (1 + 0.044715)))
    assert oracle.gelu_reference(1.0) == pytest.approx(exact_tanh, abs=1e-6)
    assert abs(oracle.gelu_reference(1.0) - 0.5 * (1 + math.erf(1 / math.sqrt(2)))) > 1e-4


def test_gelu_f16_against_float64_formula(oracle):
    x = np.arange(65536, dtype=np.uint16)
    xf = x.view(np.float16).astype(np.float64)
    with np.errstate(all="ignore"):
        want = (0.5 * xf * (1 + np.tanh(0.7978846 * (xf + 0.044715 * xf ** 3)))).astype(np.float16)
    got = oracle.gelu_f16(x).view(np.float16)
    # |x| <= 4: no cancellation in 1 + tanh(u) at f32, so at most one fp16 ulp.
    ok = np.isfinite(want) & (np.abs(xf) <= 4)
    ulps = np.abs(got[ok].view(np.int16).astype(np.int32) - want[ok].view(np.int16).astype(np.int32))
    assert ulps.max() <= 1
    # Beyond, the reference's f32 formula cancels (1 + tanh(u) -> 0); the
    # results are tiny, so bound the absolute error.
    tail = np.isfinite(want) & (np.abs(xf) > 4)
    assert np.max(np.abs(got[tail].astype(np.float64) - want[tail].astype(np.float64))) <= 1e-6


def test_reduce_sum_f16_matches_numpy_float16_sequential_adds(oracle):
    """device/reduce_add_f16.S:54-70 adds partials in order in fp16."""
    rng = np.random.default_rng(15)
    count, partials = 4096, 5
    init = rng.standard_normal(count).astype(np.float16)
    remote = (rng.standard_normal((partials, count)) * 50).astype(np.float16)
    acc = init.copy()
    for p in range(partials):
        acc = (acc + remote[p]).astype(np.float16)
    got = oracle.reduce_sum_f16(init.view(np.uint16), remote.view(np.uint16), partials, count)
    assert np.array_equal(got, acc.view(np.uint16))


def test_reduce_rows(oracle):
    rng = np.random.default_rng(16)
    x = rng.standard_normal((64, 1000)).astype(np.float16)
    got = oracle.reduce_rows_f16(x.view(np.uint16), 64, 1000)
    assert np.allclose(got, x.astype(np.float64).sum(axis=1), rtol=1e-7, atol=1e-6)
    bm = oracle.rearrange_row_major_f16(x.view(np.uint16), 2, 1, 64, 64, 1000, 1000, 64, 8)
    assert np.array_equal(oracle.reduce_rows_block_major_f16(bm, 64, 8, 64, 1000), got)


def test_add_broadcasting_matches_numpy(oracle):
    rng = np.random.default_rng(17)
    for ls, rs in [((3, 1, 5), (4, 1)), ((2, 3), (3,)), ((1,), (2, 2, 2)), ((4, 5), (4, 5))]:
        a = rng.random(ls, dtype=np.float32)
        b = rng.random(rs, dtype=np.float32)
        assert np.array_equal(oracle.add_f32(a, b), a + b)


def test_split_heads_matches_reshape(oracle):
    x = np.arange(2 * 3 * 12, dtype=np.float32).reshape(2, 3, 12)
    want = x.reshape(2, 3, 4, 3).transpose(0, 2, 1, 3).reshape(8, 3, 3)
    assert np.array_equal(oracle.split_heads(x, 4), want)


def test_splitmix64_published_vector(oracle):
    """First outputs of SplitMix64 seeded with 1234567 (Vigna's reference
    implementation): state advances by the golden gamma before mixing."""
    gamma = 0x9E3779B97F4A7C15
    outs = [oracle.splitmix64((1234567 + i * gamma) % 2**64) for i in range(3)]
    assert outs == [6457827717110365317, 3203168211198807973, 9817491932198370423]


# ---------------------------------------------------------------------------
# Committed fixtures
# ---------------------------------------------------------------------------
def test_golden_fixtures(oracle):
    path = os.path.join(GOLDEN, "kat_vectors.npz")
    data = np.load(path, allow_pickle=False)
    # fp16 conversion table (numpy IEEE float16 at generation time)
    assert np.array_equal(oracle.f32_to_f16(data["f32_values"]), data["f16_bits"])
    # block-major 64x16 map of a 64x32 shard from the assembly's byte formula
    assert np.array_equal(
        oracle.rearrange_row_major_f16(data["bm_src"], 2, 1, 64, 64, 32, 32, 64, 16),
        data["bm_dst"])
    # one-hot GEMM KAT
    M, K, N = data["gemm_shape"]
    assert np.array_equal(oracle.gemm_f16(data["gemm_left"], data["gemm_right"], M, N, K),
                          data["gemm_out"].reshape(-1))
    # tanh-GELU at fixed points (float64 closed form at generation time)
    got = np.array([oracle.gelu_reference(float(x)) for x in data["gelu_x"]])
    assert np.allclose(got, data["gelu_y"], rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# Tiled host bindings: the oracle's packer against the byte construction of
# the reference's own hardware tests (crates/ipu-tests/src/main.rs), which
# fill each tile's slice element by element from the layout's coordinates.
# ---------------------------------------------------------------------------
def _amp_left(tiles, inner=64):
    """Layout::amp_left(inner, tiles) (layout.rs:376-389)."""
    return [dict(axis=("end", 2), partitions=tiles, block_size=1),
            dict(axis=("end", 1), partitions=1, block_size=inner, zero_padding=True)]


def _block_major_matrix(row_block, tiles):
    """Layout::block_major_matrix -> block_major_matrix_storage(row_block, 64,
    tiles, 1, 1) (layout.rs:391-400, 552-590)."""
    return [dict(axis=("end", 1), partitions=tiles, block_size=64, zero_padding=True,
                 tile_stride=1),
            dict(axis=("end", 2), partitions=1, block_size=row_block, zero_padding=True)]


def _attention_output(heads, parts):
    """Layout::attention_output (layout.rs:305-316, 367-375)."""
    return [dict(axis=("end", 2), partitions=parts, block_size=1, tile_stride=heads),
            dict(axis=("end", 3), partitions=heads, block_size=1, tile_stride=1),
            dict(axis=("end", 1), partitions=1, block_size=16, zero_padding=True)]


@pytest.mark.parametrize("batch,tiles", [(1, 4), (3, 4), (3, 7)])
def test_pack_gemm_smoke_left_matches_run_gemm(oracle, batch, tiles):
    """main.rs:1079-1089: tile t's slice holds batch x 64 elements whose
    (batch_index, inner) = amp_matrix_coordinates(Left, F16, batch, 64,
    linear) is logical element [batch_index, t, inner]; slices follow in tile
    order (package.rs:2112-2128)."""
    x = (np.arange(batch * tiles * 64, dtype=np.uint32) % 65000 + 1).astype(np.uint16)
    got = oracle.pack_tiled(x, [batch, tiles, 64], 1, oracle.AMP_LEFT, tiles, 1, _amp_left(tiles))
    x3 = x.reshape(batch, tiles, 64)
    slice_elements = batch * 64
    assert got.size == tiles * slice_elements
    for t in range(tiles):
        for linear in range(slice_elements):
            b, inner = oracle.amp_matrix_coordinates(oracle.AMP_LEFT, oracle.F16, batch, 64, linear)
            assert got[t * slice_elements + linear] == x3[b, t, inner]


@pytest.mark.parametrize("tiles", [1, 3])
def test_pack_gemm_smoke_right_matches_run_gemm(oracle, tiles):
    """main.rs:1090-1105: tile t's slice is the 64 x 64 column block t in
    block-major {64, 16}: (inner, column) = block_major_matrix_coordinates(
    Matrix{64, 16}, F16, 64, 64, linear) is logical [0, inner, 64 t + column]."""
    x = (np.arange(64 * tiles * 64, dtype=np.uint32) % 65000 + 1).astype(np.uint16)
    got = oracle.pack_tiled(x, [1, 64, tiles * 64], 2, 0, tiles, 1, _block_major_matrix(64, tiles),
                            64, 16)
    x3 = x.reshape(1, 64, tiles * 64)
    assert got.size == tiles * 4096
    for t in range(tiles):
        for linear in range(4096):
            inner, col = oracle.block_major_matrix_coordinates(0, 64, 16, oracle.F16, 64, 64,
                                                               linear)
            assert got[t * 4096 + linear] == x3[0, inner, t * 64 + col]


def test_pack_mlp_smoke_weights_leave_empty_shards(oracle):
    """main.rs:1146-1166: a [64, 64] weight in block_major_matrix(64, tiles)
    has one 64-column block, so tile 0 holds it all and the other tiles'
    slices are empty."""
    tiles = 4
    x = (np.arange(4096, dtype=np.uint32) + 1).astype(np.uint16)
    got = oracle.pack_tiled(x, [64, 64], 2, 0, tiles, 1, _block_major_matrix(64, tiles), 64, 16)
    assert got.size == 4096
    for linear in range(4096):
        inner, col = oracle.block_major_matrix_coordinates(0, 64, 16, oracle.F16, 64, 64, linear)
        assert got[linear] == x[inner * 64 + col]


def _balanced_range(extent, partitions, partition):
    """main.rs:1507-1512."""
    base, rem = divmod(extent, partitions)
    return partition * base + min(partition, rem), base + (1 if partition < rem else 0)


@pytest.mark.parametrize("heads,rows,parts", [(4, 17, 4), (4, 17, 5), (2, 19, 1)])
def test_pack_attention_smoke_query_matches_run_attention_smoke(oracle, heads, rows, parts):
    """main.rs:1334-1362: tile = head + heads * partition; a slice holds the
    partition's balanced row range (balanced_range) of that head, row-major
    with the width padded from 72 to 80, padding 0."""
    width, padded = 72, 80
    x = (np.arange(heads * rows * width, dtype=np.uint32) % 65000 + 1).astype(np.uint16)
    got = oracle.pack_tiled(x, [heads, rows, width], 0, 0, heads * parts, 1,
                            _attention_output(heads, parts))
    x3 = x.reshape(heads, rows, width)
    offset = 0
    for tile in range(heads * parts):
        head, partition = tile % heads, tile // heads
        row_start, count = _balanced_range(rows, parts, partition)
        for linear in range(count * padded):
            local_row, column = divmod(linear, padded)
            want = x3[head, row_start + local_row, column] if column < width else 0
            assert got[offset + linear] == want
        offset += count * padded
    assert got.size == offset


def test_pack_transposed_orders_place_every_element_once(oracle):
    """AMP TransposedRight / TransposedLeft / Output / TransposedOutput and
    transposed block-major shards: every logical element lands once and the
    padding is zero (bijection of storage.rs's maps over the shard)."""
    shape = [2, 32, 48]
    x = (np.arange(np.prod(shape), dtype=np.uint32) + 1).astype(np.uint16)
    axes = [dict(axis=("end", 3), partitions=2, block_size=1)]
    for kind, variant, rb, cb in [(1, oracle.AMP_TRANSPOSED_RIGHT, 0, 0),
                                  (1, oracle.AMP_TRANSPOSED_LEFT, 0, 0),
                                  (1, oracle.AMP_OUTPUT, 0, 0),
                                  (1, oracle.AMP_TRANSPOSED_OUTPUT, 0, 0),
                                  (2, 1, 16, 16), (2, 0, 32, 16)]:
        got = oracle.pack_tiled(x, shape, kind, variant, 2, 1, axes, rb, cb)
        assert sorted(got.tolist()) == sorted(x.tolist()), (kind, variant)

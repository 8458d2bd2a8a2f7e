"""The no-allocation split-K entry point (ipus_gemm_f16_split_noalloc)
against the allocating form of the same computation: ipu_stack_gemm_f16_split
into a partials buffer from ipus_buffer_alloc, then
ipu_stack_reduce_splits_f16.  Both run the same kernels, so the results must
be equal bit for bit; two calls in a row, the second smaller, show that the
shared scratch array carries nothing from one call into the next."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _allocating(ctx, a, b, M, N, K, tl, tr, batches, lbs, rbs, splits, gelu):
    parts = ctx.alloc(splits * batches * M * N * 4)
    out = ctx.alloc(batches * M * N * 2)
    ctx.launch("ipu_stack_gemm_f16_split", parts, [a, b],
               [batches, M, N, K, tl, tr, lbs, rbs, splits])
    ctx.launch("ipu_stack_reduce_splits_f16", out, [parts], [splits, batches * M * N, int(gelu)])
    got = out.download(np.uint16)
    parts.free()
    out.free()
    return got


@pytest.mark.parametrize("first,second", [
    # (M, N, K, tl, tr, batches, splits, gelu): the reference's SigLIP MLP
    # second GEMM at build_package's 4 splits, then a smaller batched one.
    ((729, 1152, 4304, 0, 0, 1, 4, 0), (264, 136, 3000, 0, 1, 2, 5, 1)),
])
def test_no_alloc_split_k_matches_allocating_form(ipus, ctx, first, second):
    base = ctx.live_buffers()
    outs = []
    for M, N, K, tl, tr, batches, splits, gelu in (first, second):
        a = ipus.synth_f16(batches * M * K, 61, 1, ipus.NORMAL, 1.0)
        b = ipus.synth_f16(batches * K * N, 61, 2, ipus.NORMAL, 0.05)
        da, db = ctx.upload(a), ctx.upload(b)
        lbs, rbs = M * K, K * N
        want = _allocating(ctx, da, db, M, N, K, tl, tr, batches, lbs, rbs, splits, gelu)
        out = ctx.upload(np.full(batches * M * N, 0x7E00, dtype=np.uint16))
        live = ctx.live_buffers()
        ctx.gemm_f16_split_noalloc(out, da, db, batches, M, N, K, tl, tr, lbs, rbs, splits, gelu)
        ctx.sync()
        assert ctx.live_buffers() == live      # nothing allocated through the library
        got = out.download(np.uint16)
        assert np.array_equal(got, want), (M, N, K)
        outs.append(got)
        for x in (da, db, out):
            x.free()
    assert ctx.live_buffers() == base


def test_no_alloc_split_k_rejects_partials_beyond_the_scratch(ipus, ctx):
    out = ctx.alloc(64)
    # 2048 x 2048 x 2 splits of fp32 partials = 32 MiB > 16 MiB.
    with pytest.raises(ipus.IpusError) as err:
        ctx.gemm_f16_split_noalloc(out, out, out, 1, 2048, 2048, 4096, splits=2)
    assert err.value.status == ipus.ERROR_UNSUPPORTED_COUNT and "scratch" in err.value.message
    out.free()


def test_no_alloc_split_k_rejects_a_size_product_past_64_bits(ipus, ctx):
    out = ctx.alloc(64)
    # 2^31 x 2^31 fp32 partials are 2^64 bytes: the size product wraps to 0
    # in 64 bits and must still be refused before any launch.
    with pytest.raises(ipus.IpusError) as err:
        ctx.gemm_f16_split_noalloc(out, out, out, 1, 1 << 31, 1 << 31, 64, splits=1)
    assert err.value.status == ipus.ERROR_UNSUPPORTED_COUNT and "scratch" in err.value.message
    out.free()

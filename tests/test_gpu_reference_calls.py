"""Reference-shaped ComputeSteps launched through ipus_launch on the GPU.

The symbols and scalars are built as the reference builds them
(tests/test_reference_calls.py restates kernel.rs:1149-1193 and the
per-shape symbol names); each launch is checked against the oracle:
bit-exact for the layout conversions and FillZero, the north-star
tolerance for attention."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import fp16_close
from test_reference_calls import attention_call, fill_zero_call, rearrange_call, unpack_call

pytestmark = pytest.mark.gpu


def launch(ctx, symbol, out_nbytes, inputs, scalars, dtype=np.uint16, fill=0xA5):
    bufs = [ctx.upload(x) for x in inputs]
    out = ctx.upload(np.full(out_nbytes, fill, dtype=np.uint8))
    ctx.launch(symbol, out, bufs, scalars)
    got = out.download(dtype)
    for b in bufs:
        b.free()
    out.free()
    return got


@pytest.mark.parametrize("lr,pr,lc,pc,order", [
    (64, 64, 4096, 4096, 2), (40, 64, 100, 112, 2), (64, 64, 256, 256, 2),
    (729, 736, 1152, 1152, 0), (19, 19, 72, 80, 0), (64, 64, 16, 16, 1), (50, 64, 32, 32, 1),
    (256, 256, 512, 512, 1)])
def test_reference_rearrange_symbol_bit_exact(ipus, oracle, ctx, lr, pr, lc, pc, order):
    symbol, _, scalars = rearrange_call(lr, pr, lc, pc, order)
    print(symbol, scalars, flush=True)
    x = ipus.synth_f16(lr * lc, 71, order, 1)
    got = launch(ctx, symbol, pr * pc * 2, [x], scalars)
    # block-major {64, 16} for target 2, the block shape the suffix implies
    want = oracle.rearrange_row_major_f16(x, order, 1, lr, pr, lc, pc, 64, 16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("matrices,lr,pr,lc,pc,source", [
    (1, 729, 736, 1152, 1152, 0), (4, 30, 32, 40, 48, 1), (2, 64, 64, 64, 64, 0),
    (1, 256, 256, 512, 512, 1)])
def test_reference_unpack_symbol_bit_exact(ipus, oracle, ctx, matrices, lr, pr, lc, pc, source):
    symbol, _, scalars = unpack_call(matrices, lr, pr, lc, pc, source)
    print(symbol, scalars, flush=True)
    x = ipus.synth_f16(matrices * pr * pc, 72, source, 1)
    got = launch(ctx, symbol, x.nbytes, [x], scalars)
    want = oracle.unpack_to_row_major_f16(x, source, matrices, lr, pr, lc, pc)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("matrices,q,k,d,v,scale", [
    (4, 17, 19, 72, 72, None), (2, 256, 300, 128, 128, None), (3, 130, 64, 64, 64, 0.05),
    (1, 33, 45, 160, 160, None)])
def test_reference_attention_symbol(ipus, oracle, ctx, matrices, q, k, d, v, scale):
    symbol, _, scalars = attention_call(matrices, q, k, d, v, scale)
    print(symbol, flush=True)
    qh = ipus.synth_f16(matrices * q * d, 73, 1, 1)
    kh = ipus.synth_f16(matrices * k * d, 73, 2, 1)
    vh = ipus.synth_f16(matrices * k * v, 73, 3, 1)
    got = launch(ctx, symbol, matrices * q * v * 4, [qh, kh, vh], scalars, np.float32)
    want = oracle.attention(oracle.f16_to_f32(qh), oracle.f16_to_f32(kh), oracle.f16_to_f32(vh),
                            matrices, q, k, d, v, False, scale)
    assert fp16_close(got.reshape(matrices * q, v), want)


@pytest.mark.parametrize("nbytes", [48, 4104, 1 << 20])
def test_reference_fill_zero_symbol(ipus, ctx, nbytes):
    symbol, _, scalars = fill_zero_call(nbytes)
    got = launch(ctx, symbol, nbytes + 64, [], scalars, np.uint8)
    assert not got[:nbytes].any()
    assert (got[nbytes:] == 0xA5).all()

"""Writes tests/golden/kat_vectors.npz: known-answer vectors built WITHOUT the
oracle, from the reference's own test designs and independent constructions.

  f32_values/f16_bits  numpy's IEEE binary16 round-to-nearest-even (the `half`
                       crate semantics used by main.rs:2040-2046)
  bm_src/bm_dst        64x32 shard placed by the byte-address formula of
                       device/rearrange_block_major_f16.S:69-104
  gemm_*               one-hot x 5-level KAT of main.rs:1079-1105, 2133-2136
  gelu_x/gelu_y        float64 tanh-GELU of main.rs:1985-1987

The reference is Rust + Graphcore SDK and cannot run here, so no vector comes
from executing it.  Run: python tests/golden/make_golden.py
"""
import math
import os

import numpy as np

rng = np.random.default_rng(0x601DE2)
f32 = np.concatenate([
    rng.standard_normal(512).astype(np.float32) * np.float32(1000),
    (rng.random(256) * 1e-4).astype(np.float32),
    np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 6.1035156e-05, 5.9604645e-08, np.inf, -np.inf],
             dtype=np.float32)])
f16 = f32.astype(np.float16).view(np.uint16)

src = (np.arange(64 * 32, dtype=np.uint32) * 2654435761 % 65521).astype(np.uint16)
dst = np.zeros(64 * 32, dtype=np.uint16)
for r in range(64):
    for c in range(32):
        byte = (c // 16) * 2048 + (r // 16) * 512 + (r % 16) * 2 + (c % 16) * 32
        dst[byte // 2] = src[r * 32 + c]

levels = np.array([0xBC00, 0xB800, 0x0000, 0x3800, 0x3C00], dtype=np.uint16)
M, K, N = 32, 64, 48
left = np.zeros((M, K), dtype=np.uint16)
sel = (np.arange(M) * 7) % 64
left[np.arange(M), sel] = 0x3C00
right = levels[(np.arange(K)[:, None] * 3 + np.arange(N)[None, :]) % 5]
out = right[sel]

gx = np.linspace(-6, 6, 49)
gy = np.array([0.5 * x * (1 + math.tanh(0.7978846 * (x + 0.044715 * x ** 3))) for x in gx])

np.savez(os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat_vectors.npz"),
         f32_values=f32, f16_bits=f16, bm_src=src, bm_dst=dst,
         gemm_shape=np.array([M, K, N]), gemm_left=left, gemm_right=right, gemm_out=out,
         gelu_x=gx, gelu_y=gy)
print("wrote kat_vectors.npz")

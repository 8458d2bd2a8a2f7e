// Device-side helpers shared by the gfx950 kernels of libipus.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ipus {

typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Packs the low (sel_hi = false) or high 16-bit halves of two words:
// result = {a.half, b.half} with a in the low half.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

// Transposes an 8x8 block of 16-bit elements held as 8 rows of 16 bytes.
// in[j] holds row j (elements 0..7 of that row, element e in half e of word
// e/2); out[i] receives column i as a row: out[i] element j = in[j] element i.
__device__ __forceinline__ void transpose8x8_u16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int w = i >> 1;
    const bool hi = (i & 1) != 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t a = in[2 * t][w];
      const uint32_t b = in[2 * t + 1][w];
      out[i][t] = hi ? pack_hi(a, b) : pack_lo(a, b);
    }
  }
}

// Transposes a 4x4 block of 32-bit elements (4 rows of 16 bytes).
__device__ __forceinline__ void transpose4x4_u32(const u32x4 in[4], u32x4 out[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) out[i][j] = in[j][i];
}

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// Wave-wide sum via cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}

// tanh-approximation GELU of one fp16 value widened to fp32 (the value the
// reference's formula is applied to, crates/ipu-tests/src/main.rs:1985-1987):
//   0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)),  u = 0.7978846 (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_tanh(float x) {
  // x / (1 + exp(-2u)) with exp(-2u) = exp2(-2 log2(e) u): v_exp_f32 and
  // v_rcp_f32 (about 1 ulp of fp32 each, far below the fp16 result's
  // rounding); x -> -inf gives x * rcp(inf) = -0 as the exact form does.
  constexpr float kA = -2.0f * 0.7978846f * 1.4426950408889634f;
  const float t = x * x;
  const float v = x * fmaf(t, 0.044715f, 1.0f);  // x + 0.044715 x^3
  const float e = __builtin_amdgcn_exp2f(v * kA);
  // The product is rounded to fp32 here: left visible, the compiler fuses
  // it with a caller's conversion to fp16 (v_fma_mix, one rounding instead
  // of two) in some kernels and not in others, and the GEMM epilogue must
  // produce the GELU kernel's bits.
  float y = x * __builtin_amdgcn_rcpf(1.0f + e);
  asm("" : "+v"(y));
  return y;
}

}  // namespace ipus

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

}  // namespace ipus

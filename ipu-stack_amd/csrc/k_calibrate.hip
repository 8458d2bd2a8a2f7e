// Roofline calibration: the sustained v_mfma_f32_32x32x16_f16 (or
// v_mfma_f32_16x16x32_f16) rate and the shader clock under full MFMA load,
// for a given operand bit pattern.
//
// Each lane loads one A and one B fragment (8 fp16 each) from `operands` and
// runs `iterations` rounds of 8 independent MFMAs on them; nothing else
// touches memory until a final store that keeps the results live.  Lane 0 of
// block 0 records s_memtime (shader clock) and s_memrealtime (100 MHz) around
// its loop, so clock = d(memtime) / (d(realtime) / 100 MHz).  The MI355X
// clock under dense MFMA depends on operand entropy (power limit), which is
// why the calibration takes the operand pattern as input.
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

namespace ipus {
namespace {

__global__ __launch_bounds__(256) void mfma_calibrate_kernel(uint64_t* __restrict__ clocks,
                                                             float* __restrict__ sink,
                                                             const half8_t* __restrict__ operands,
                                                             uint32_t operand_count,
                                                             uint32_t iterations) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const half8_t a = operands[gid % operand_count];
  const half8_t b = operands[(gid + 7) % operand_count];
  float16_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) c[j][e] = 0.0f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[j][e];
  sink[gid] = s;
  if (gid == 0) {
    clocks[0] = t1 - t0;
    clocks[1] = r1 - r0;
  }
}

// The same for v_mfma_f32_16x16x32_f16, the form the GEMM and attention
// kernels issue, with eight fragment pairs per lane so that consecutive
// MFMAs see different operands, as in a K loop.
__global__ __launch_bounds__(256) void mfma16_calibrate_kernel(uint64_t* __restrict__ clocks,
                                                               float* __restrict__ sink,
                                                               const half8_t* __restrict__ operands,
                                                               uint32_t operand_count,
                                                               uint32_t iterations) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  half8_t a[8], b[8];
#pragma unroll
  for (uint32_t j = 0; j < 8; ++j) {
    a[j] = operands[(gid + 131 * j) % operand_count];
    b[j] = operands[(gid + 7 + 257 * j) % operand_count];
  }
  float4_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  // Accumulators tied to AGPRs by inline assembly, as in the GEMM kernel:
  // with the builtin, the compiler copies the accumulators between
  // registers around every MFMA of this form.
  for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c[j]) : "v"(a[j]), "v"(b[j]));
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  // 24 wait states before reading the accumulators (the compiler does not
  // pad inline assembly).
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += c[j][e];
  sink[gid] = s;
  if (gid == 0) {
    clocks[0] = t1 - t0;
    clocks[1] = r1 - r0;
  }
}

// Plain copy for the HBM traffic counters' calibration: ordinary (temporal)
// 16-byte loads and stores, one vector per thread, so its FETCH_SIZE /
// WRITE_SIZE read as a kernel whose loads take the ordinary cache path (the
// library's streaming copy uses non-temporal accesses, which the counters
// weigh differently).
__global__ __launch_bounds__(256) void copy_plain_kernel(u32x4* __restrict__ dst,
                                                         const u32x4* __restrict__ src,
                                                         uint64_t vectors) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < vectors) dst[i] = src[i];
}

}  // namespace

int launch_calibrate_copy(hipStream_t stream, void* dst, const void* src, uint32_t bytes) {
  if (bytes % 16 != 0 || (uintptr_t)dst % 16 != 0 || (uintptr_t)src % 16 != 0)
    return IPUS_ERROR_INVALID_ARGUMENT;
  const uint64_t vectors = bytes / 16;
  if (vectors == 0) return 0;
  hipLaunchKernelGGL(copy_plain_kernel, dim3((uint32_t)((vectors + 255) / 256)), dim3(256), 0,
                     stream, (u32x4*)dst, (const u32x4*)src, vectors);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e;
}

uint64_t calibrate_output_bytes(uint32_t blocks) { return 16 + (uint64_t)blocks * 256 * 4; }

int launch_calibrate_mfma_f16(hipStream_t stream, void* out, const void* operands,
                              uint32_t operand_count, uint32_t iterations, uint32_t blocks,
                              bool form16) {
  if (operand_count == 0 || blocks == 0) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(form16 ? mfma16_calibrate_kernel : mfma_calibrate_kernel, dim3(blocks),
                     dim3(256), 0, stream, (uint64_t*)out, (float*)((uint8_t*)out + 16),
                     (const half8_t*)operands, operand_count, iterations);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e;
}

}  // namespace ipus

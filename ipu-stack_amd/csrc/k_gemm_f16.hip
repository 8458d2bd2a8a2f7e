// fp16 GEMM on gfx950 MFMA with fp32 accumulation and fp16 output:
//   C[b] = A[b] . B[b]   (A [M,K] or its transpose, B [K,N] or its transpose)
// Replaces gemm_f16_amp (device/gemm_f16_amp.S:186-440), whose partials pass
// through fp16; the accumulation here is fp32 throughout, matching the CPU
// evaluator's fp32 sgemm followed by one fp16 rounding
// (crates/ipu-tests/src/diagnostic.rs:533-654, 841-847).
//
// Fast kernel (M % 256 == 0, N % 256 == 0, K % 64 == 0):
//   * block tile 256 x 256 x 64, 256 threads = 4 waves in a 2 x 2 grid, each
//     wave owns 128 x 128 of C as 4 x 4 tiles of v_mfma_f32_32x32x16_f16;
//   * both operands are staged in LDS K-contiguous ([row][64 k], 128 B rows)
//     with the 16-byte chunk index XOR-swizzled by ((r ^ r >> 3) & 7), which
//     keeps the MFMA fragment reads and both kinds of tile stores free of bank
//     conflicts;
//   * an operand whose rows are not K-contiguous in memory (row-major B, or a
//     transposed A) is loaded as 8 x 8 blocks and transposed in registers
//     before the LDS store;
//   * two LDS stages: the next tile's global loads are in flight while the
//     current tile is multiplied, one barrier per K step;
//   * the MFMA computes the tile of C^T (B fragment as the first operand) so
//     each lane ends up holding 4 consecutive columns of one row of C, stored
//     as one 8-byte write;
//   * block ids are remapped so that the blocks one XCD runs (round-robin
//     dispatch over 8 XCDs) form a compact group of C tiles sharing L2.
// General kernel: 64 x 64 tiles, bounds-checked scalar loads, any shape.
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

namespace ipus {
namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kTileBytes = kBM * kBK * 2;  // 32 KiB per operand tile

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk) {
  return row * 128u + ((chunk ^ ((row ^ (row >> 3)) & 7u)) << 4);
}

// Loads this thread's share of a 256-row x 64-k operand tile.
// KContig: element (r, k) at base[(row0 + r) * ld + k0 + k]
// else:    element (r, k) at base[(k0 + k) * ld + row0 + r]
template <bool KContig>
__device__ __forceinline__ void load_tile(const uint16_t* __restrict__ base, uint64_t ld,
                                          uint32_t row0, uint32_t k0, u32x4 v[8]) {
  const uint32_t t = threadIdx.x;
  if constexpr (KContig) {
    const uint16_t* p = base + (uint64_t)(row0 + t / 8) * ld + k0 + (t % 8) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = load16(p + (uint64_t)(32 * i) * ld);
  } else {
    const uint16_t* p = base + (uint64_t)(k0 + (t / 32) * 8) * ld + row0 + (t % 32) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = load16(p + (uint64_t)j * ld);
  }
}

template <bool KContig>
__device__ __forceinline__ void store_tile(uint8_t* lds, const u32x4 v[8]) {
  const uint32_t t = threadIdx.x;
  if constexpr (KContig) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = t / 8 + 32 * i;
      *reinterpret_cast<u32x4*>(lds + swz(r, t % 8)) = v[i];
    }
  } else {
    u32x4 w[8];
    transpose8x8_u16(v, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = (t % 32) * 8 + i;
      *reinterpret_cast<u32x4*>(lds + swz(r, t / 32)) = w[i];
    }
  }
}

__device__ __forceinline__ half8_t read_frag(const uint8_t* lds, uint32_t row, uint32_t chunk) {
  return __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(lds + swz(row, chunk)));
}

template <bool TransposeLeft, bool TransposeRight>
__global__ __launch_bounds__(kThreads, 1) void gemm_f16_256_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ left,
    const uint16_t* __restrict__ right, uint32_t M, uint32_t N, uint32_t K,
    uint64_t left_batch_stride, uint64_t right_batch_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const uint32_t nbm = M / kBM, nbn = N / kBN;
  const uint32_t tiles = nbm * nbn;
  uint32_t pid = blockIdx.x;
  if (tiles % 8 == 0) pid = (pid % 8) * (tiles / 8) + pid / 8;  // XCD-contiguous
  constexpr uint32_t kGroup = 8;
  const uint32_t group = pid / (kGroup * nbn);
  const uint32_t first_m = group * kGroup;
  const uint32_t group_rows = (nbm - first_m) < kGroup ? (nbm - first_m) : kGroup;
  const uint32_t in_group = pid % (kGroup * nbn);
  const uint32_t bm = first_m + in_group % group_rows;
  const uint32_t bn = in_group / group_rows;

  const uint64_t batch = blockIdx.y;
  const uint16_t* A = left + batch * left_batch_stride;
  const uint16_t* B = right + batch * right_batch_stride;
  uint16_t* C = out + batch * (uint64_t)M * N;
  // Leading dimensions of the stored operands.
  const uint64_t lda = TransposeLeft ? M : K;
  const uint64_t ldb = TransposeRight ? K : N;
  constexpr bool kAContig = !TransposeLeft;  // A rows (m) K-contiguous
  constexpr bool kBContig = TransposeRight;  // B^T rows (n) K-contiguous

  const uint32_t m0 = bm * kBM, n0 = bn * kBN;
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t wm = (wave / 2) * 128, wn = (wave % 2) * 128;

  float16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  u32x4 ra[8], rb[8];
  load_tile<kAContig>(A, lda, m0, 0, ra);
  load_tile<kBContig>(B, ldb, n0, 0, rb);
  store_tile<kAContig>((smem + 0 + (0) * 2 * kTileBytes), ra);
  store_tile<kBContig>((smem + kTileBytes + (0) * 2 * kTileBytes), rb);
  __syncthreads();

  const uint32_t ksteps = K / kBK;
  for (uint32_t kt = 0; kt < ksteps; ++kt) {
    const uint32_t cur = kt & 1;
    const bool more = kt + 1 < ksteps;
    if (more) {
      load_tile<kAContig>(A, lda, m0, (kt + 1) * kBK, ra);
      load_tile<kBContig>(B, ldb, n0, (kt + 1) * kBK, rb);
    }
    const uint8_t* la = (smem + 0 + (cur) * 2 * kTileBytes);
    const uint8_t* lb = (smem + kTileBytes + (cur) * 2 * kTileBytes);
#pragma unroll
    for (uint32_t ks = 0; ks < kBK / 16; ++ks) {
      const uint32_t chunk = ks * 2 + lane / 32;
      half8_t fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = read_frag(la, wm + i * 32 + lane % 32, chunk);
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = read_frag(lb, wn + j * 32 + lane % 32, chunk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    if (more) {
      store_tile<kAContig>((smem + 0 + (cur ^ 1) * 2 * kTileBytes), ra);
      store_tile<kBContig>((smem + kTileBytes + (cur ^ 1) * 2 * kTileBytes), rb);
    }
    __syncthreads();
  }

  // acc[i][j][r] = C[m0 + wm + 32 i + lane % 32][n0 + wn + 32 j + 8 (r / 4) + 4 (lane / 32) + r % 4]
  const uint32_t row = m0 + wm + lane % 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t* crow = C + (uint64_t)(row + 32 * i) * N + n0 + wn + 4 * (lane / 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4_t h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (half_t)acc[i][j][4 * g + e];
        *reinterpret_cast<half4_t*>(crow + 32 * j + 8 * g) = h;
      }
    }
  }
}

// General fp16 GEMM: 64 x 64 tile, 4 waves of one 32 x 32 MFMA tile each,
// K step 16, bounds-checked scalar loads.  Any shape, transposes, batches.
__global__ __launch_bounds__(256) void gemm_f16_general_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ left,
    const uint16_t* __restrict__ right, uint32_t M, uint32_t N, uint32_t K, bool tl, bool tr,
    uint64_t left_batch_stride, uint64_t right_batch_stride, uint32_t tiles_n) {
  __shared__ __attribute__((aligned(16))) half_t As[64][24];
  __shared__ __attribute__((aligned(16))) half_t Bs[64][24];
  const uint64_t batch = blockIdx.y;
  const uint16_t* A = left + batch * left_batch_stride;
  const uint16_t* B = right + batch * right_batch_stride;
  uint16_t* C = out + batch * (uint64_t)M * N;
  const uint32_t m0 = (blockIdx.x / tiles_n) * 64, n0 = (blockIdx.x % tiles_n) * 64;
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t wm = (wave / 2) * 32, wn = (wave % 2) * 32;
  const uint64_t lda = tl ? M : K, ldb = tr ? K : N;
  float16_t acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
  for (uint32_t k0 = 0; k0 < K; k0 += 16) {
    for (uint32_t idx = threadIdx.x; idx < 64 * 16; idx += 256) {
      const uint32_t r = idx / 16, k = idx % 16;
      const uint32_t m = m0 + r, n = n0 + r, kk = k0 + k;
      uint16_t a = 0, b = 0;
      if (m < M && kk < K) a = tl ? A[(uint64_t)kk * lda + m] : A[(uint64_t)m * lda + kk];
      if (n < N && kk < K) b = tr ? B[(uint64_t)n * ldb + kk] : B[(uint64_t)kk * ldb + n];
      As[r][k] = __builtin_bit_cast(half_t, a);
      Bs[r][k] = __builtin_bit_cast(half_t, b);
    }
    __syncthreads();
    const half8_t fa = *reinterpret_cast<const half8_t*>(&As[wm + lane % 32][(lane / 32) * 8]);
    const half8_t fb = *reinterpret_cast<const half8_t*>(&Bs[wn + lane % 32][(lane / 32) * 8]);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb, fa, acc, 0, 0, 0);
    __syncthreads();
  }
  const uint32_t m = m0 + wm + lane % 32;
  if (m >= M) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t n = n0 + wn + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
    if (n < N) C[(uint64_t)m * N + n] = __builtin_bit_cast(uint16_t, (half_t)acc[r]);
  }
}

template <bool TL, bool TR>
int launch_fast(hipStream_t stream, const GemmArgs& a) {
  const uint32_t tiles = (a.rows / kBM) * (a.columns / kBN);
  constexpr size_t lds = 4 * kTileBytes;  // two stages of A and B
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute((const void*)gemm_f16_256_kernel<TL, TR>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_status(e);
    configured = true;
  }
  hipLaunchKernelGGL((gemm_f16_256_kernel<TL, TR>), dim3(tiles, a.batches), dim3(kThreads), lds,
                     stream, (uint16_t*)a.out, (const uint16_t*)a.left, (const uint16_t*)a.right,
                     a.rows, a.columns, a.inner, a.left_batch_stride, a.right_batch_stride);
  return hip_status(hipGetLastError());
}

}  // namespace

int launch_gemm_f16(hipStream_t stream, const GemmArgs& a) {
  if (a.batches == 0 || a.rows == 0 || a.columns == 0) return 0;
  if (a.batches > 65535) return IPUS_ERROR_INVALID_ARGUMENT;
  const bool aligned = ((uintptr_t)a.left % 16 == 0) && ((uintptr_t)a.right % 16 == 0) &&
                       ((uintptr_t)a.out % 16 == 0) && a.left_batch_stride % 8 == 0 &&
                       a.right_batch_stride % 8 == 0;
  if (aligned && a.rows % kBM == 0 && a.columns % kBN == 0 && a.inner % kBK == 0 && a.inner > 0) {
    if (!a.transpose_left && !a.transpose_right) return launch_fast<false, false>(stream, a);
    if (!a.transpose_left && a.transpose_right) return launch_fast<false, true>(stream, a);
    if (a.transpose_left && !a.transpose_right) return launch_fast<true, false>(stream, a);
    return launch_fast<true, true>(stream, a);
  }
  const uint32_t tiles_m = (a.rows + 63) / 64, tiles_n = (a.columns + 63) / 64;
  hipLaunchKernelGGL(gemm_f16_general_kernel, dim3(tiles_m * tiles_n, a.batches), dim3(256), 0,
                     stream, (uint16_t*)a.out, (const uint16_t*)a.left, (const uint16_t*)a.right,
                     a.rows, a.columns, a.inner, a.transpose_left, a.transpose_right,
                     a.left_batch_stride, a.right_batch_stride, tiles_n);
  return hip_status(hipGetLastError());
}

}  // namespace ipus

// fp32 GEMM on gfx950 MFMA (v_mfma_f32_32x32x2_f32), fp32 accumulation and
// output: replaces gemm_f32_64_amp (device/gemm_f32_64_amp.S:125-385), whose
// init mode clears the output and accumulates in fp32 (gemm_f32_64_amp.S:40-56).
//
// One kernel for every shape (16-byte aligned operands whose contiguous
// axes, and N, are multiples of 4 use 16-byte loads; the kEdge mode, used
// off the 128 x 128 x 32 grid, zero-fills loads past M, N or K and stores
// only rows < M and 4-column chunks < N; kScalar covers other shapes and
// alignments with bounds-checked element loads and stores):
//   * block tile 128 x 128 x 32, 4 waves in a 2 x 2 grid, each wave 64 x 64
//     as 2 x 2 MFMA tiles;
//   * each operand is staged in LDS in the layout it has in memory, so no
//     tile is transposed on the way: an operand whose x axis (m or n) is
//     contiguous k-major ([k][x], 16-byte chunks XOR-swizzled by (k >> 2) &
//     7), one whose k axis is contiguous x-major ([x][k], rows of 32 k,
//     chunks XOR-swizzled by (x >> 1) & 7);
//   * the k pair of MFMA substep p is (p, 16 + p) for lanes 0-31 and 32-63, a
//     permutation of the step's 32 k that both operands share, so a lane reads
//     four substeps' values of an x-major tile as one 16-byte chunk (k-major
//     tiles: one element per substep);
//   * one LDS stage (32 KiB, so three workgroups share a CU): the next K
//     step's tiles load into registers during the MFMAs and are stored
//     between two barriers (4096^3: 121 -> 126 TFLOP/s against two stages
//     and two workgroups per CU);
//   * the MFMA computes C^T tiles so each lane holds 4 consecutive columns
//     of C (one 16-byte store).
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"

namespace ipus {
namespace {

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kThreads = 256;
constexpr int kTileBytes = kBK * kBM * 4;  // 16 KiB per operand tile

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

// Byte offset of element (k, x) in a [32 k][128 x] fp32 tile (k-major,
// the layout of an operand whose x axis is contiguous in memory).
__device__ __forceinline__ uint32_t swz32(uint32_t k, uint32_t x) {
  return k * 512u + ((((x >> 2) ^ ((k >> 2) & 7u)) << 4) | ((x & 3u) << 2));
}
// Byte offset of 16-byte chunk c (k = 4 c .. 4 c + 3) of row x in a
// [128 x][32 k] fp32 tile (x-major, the layout of an operand whose k axis is
// contiguous in memory).
__device__ __forceinline__ uint32_t xk_off(uint32_t x, uint32_t c) {
  return x * 128u + ((c ^ ((x >> 1) & 7u)) << 4);
}

// Tile modes: kGrid (every tile whole), kEdge (chunks of 4 floats past the
// extents read as 0 and are not stored; the contiguous axes and N are
// multiples of 4, so a chunk is wholly inside or outside), kScalar (any
// shape and alignment: element loads and stores, each bounds-checked).
enum TileMode : int { kGrid = 0, kEdge = 1, kScalar = 2 };

// Loads a 128 (x) by 32 (k) operand tile.
// XContig: element (x, k) at base[(k0 + k) * ld + x0 + x]  (stored [K][X])
// else:    element (x, k) at base[(x0 + x) * ld + k0 + k]  (stored [X][K])
template <bool XContig, int Mode>
__device__ __forceinline__ void load_tile32(const float* __restrict__ base, uint64_t ld,
                                            uint32_t x0, uint32_t k0, u32x4 v[4], uint32_t X,
                                            uint32_t K) {
  const uint32_t t = threadIdx.x;
  const u32x4 zero = {0, 0, 0, 0};
  if constexpr (XContig) {
    const uint32_t k = k0 + t / 32, x = x0 + (t % 32) * 4;
    const float* p = base + (uint64_t)k * ld + x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (Mode == kScalar) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[i][e] = k + 8 * i < K && x + e < X ? __float_as_uint(p[(uint64_t)(8 * i) * ld + e]) : 0u;
      } else {
        v[i] = Mode == kGrid || (k + 8 * i < K && x < X) ? load16(p + (uint64_t)(8 * i) * ld) : zero;
      }
    }
  } else {
    const uint32_t x = x0 + (t / 8) * 4, k = k0 + (t % 8) * 4;
    const float* p = base + (uint64_t)x * ld + k;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (Mode == kScalar) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[j][e] = x + j < X && k + e < K ? __float_as_uint(p[(uint64_t)j * ld + e]) : 0u;
      } else {
        v[j] = Mode == kGrid || (x + j < X && k < K) ? load16(p + (uint64_t)j * ld) : zero;
      }
    }
  }
}

template <bool XContig>
__device__ __forceinline__ void store_tile32(uint8_t* lds, const u32x4 v[4]) {
  const uint32_t t = threadIdx.x;
  if constexpr (XContig) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(lds + swz32(t / 32 + 8 * i, (t % 32) * 4)) = v[i];
  } else {
    // v[j] = x row (t/8)*4 + j, k chunk t%8: stored as loaded.
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4*>(lds + xk_off((t / 8) * 4 + j, t % 8)) = v[j];
  }
}

__device__ __forceinline__ float read32(const uint8_t* lds, uint32_t k, uint32_t x) {
  return *reinterpret_cast<const float*>(lds + swz32(k, x));
}

template <bool TransposeLeft, bool TransposeRight, int Mode>
__global__ __launch_bounds__(kThreads, 3) void gemm_f32_128_kernel(
    float* __restrict__ out, const float* __restrict__ left, const float* __restrict__ right,
    uint32_t M, uint32_t N, uint32_t K, uint64_t left_batch_stride, uint64_t right_batch_stride) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kTileBytes];

  const uint32_t nbm = (M + kBM - 1) / kBM, nbn = (N + kBN - 1) / kBN;
  const uint32_t tiles = nbm * nbn;
  uint32_t pid = blockIdx.x;
  if (tiles % 8 == 0) pid = (pid % 8) * (tiles / 8) + pid / 8;
  constexpr uint32_t kGroup = 8;
  const uint32_t group = pid / (kGroup * nbn);
  const uint32_t first_m = group * kGroup;
  const uint32_t group_rows = (nbm - first_m) < kGroup ? (nbm - first_m) : kGroup;
  const uint32_t in_group = pid % (kGroup * nbn);
  const uint32_t bm = first_m + in_group % group_rows;
  const uint32_t bn = in_group / group_rows;

  const uint64_t batch = blockIdx.y;
  const float* A = left + batch * left_batch_stride;
  const float* B = right + batch * right_batch_stride;
  float* C = out + batch * (uint64_t)M * N;
  const uint64_t lda = TransposeLeft ? M : K;
  const uint64_t ldb = TransposeRight ? K : N;
  constexpr bool kAX = TransposeLeft;    // A stored [K][M]: m contiguous
  constexpr bool kBX = !TransposeRight;  // B stored [K][N]: n contiguous

  const uint32_t m0 = bm * kBM, n0 = bn * kBN;
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t wm = (wave / 2) * 64, wn = (wave % 2) * 64;

  float16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  u32x4 ra[4], rb[4];
  load_tile32<kAX, Mode>(A, lda, m0, 0, ra, M, K);
  load_tile32<kBX, Mode>(B, ldb, n0, 0, rb, N, K);
  store_tile32<kAX>(smem, ra);
  store_tile32<kBX>(smem + kTileBytes, rb);
  __syncthreads();

  const uint32_t ksteps = (K + kBK - 1) / kBK;
  for (uint32_t kt = 0; kt < ksteps; ++kt) {
    const bool more = kt + 1 < ksteps;
    if (more) {
      load_tile32<kAX, Mode>(A, lda, m0, (kt + 1) * kBK, ra, M, K);
      load_tile32<kBX, Mode>(B, ldb, n0, (kt + 1) * kBK, rb, N, K);
    }
    const uint8_t* la = smem;
    const uint8_t* lb = smem + kTileBytes;
    // The k pair of substep p is (p, 16 + p) for lanes 0-31 and 32-63 (a
    // permutation of the step's 32 k that A and B share): in an x-major
    // tile a lane's values for 4 consecutive substeps are one 16-byte chunk
    // of its row; a k-major tile is read one element per substep.
    const uint32_t g = lane / 32;
    auto frag4 = [&]<bool XContig>(const uint8_t* l, uint32_t x, uint32_t q) __attribute__((always_inline)) {
      if constexpr (XContig) {
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = __float_as_uint(read32(l, 16 * g + 4 * q + w, x));
        return v;
      } else {
        return *reinterpret_cast<const u32x4*>(l + xk_off(x, 4 * g + q));
      }
    };
#pragma unroll
    for (uint32_t q = 0; q < kBK / 8; ++q) {
      u32x4 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = frag4.template operator()<kAX>(la, wm + 32 * i + lane % 32, q);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = frag4.template operator()<kBX>(lb, wn + 32 * j + lane % 32, q);
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(fb[j][w]),
                                                            __uint_as_float(fa[i][w]), acc[i][j], 0, 0, 0);
    }
    if (more) {
      __syncthreads();  // every wave is done reading this tile
      store_tile32<kAX>(smem, ra);
      store_tile32<kBX>(smem + kTileBytes, rb);
    }
    __syncthreads();
  }

  const uint32_t row = m0 + wm + lane % 32;
  const uint32_t col = n0 + wn + 4 * (lane / 32);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (Mode != kGrid && row + 32 * i >= M) continue;
    float* crow = C + (uint64_t)(row + 32 * i) * N + col;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t c = col + 32 * j + 8 * g;
        if (Mode != kGrid && c >= N) continue;
        if constexpr (Mode == kScalar) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (c + e < N) crow[32 * j + 8 * g + e] = acc[i][j][4 * g + e];
        } else {
          float4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e];
          *reinterpret_cast<float4_t*>(crow + 32 * j + 8 * g) = v;
        }
      }
  }
}

template <bool TL, bool TR>
int launch_fast(hipStream_t stream, const GemmArgs& a, bool chunked) {
  const uint32_t tiles = ((a.rows + kBM - 1) / kBM) * ((a.columns + kBN - 1) / kBN);
  const bool grid = a.rows % kBM == 0 && a.columns % kBN == 0 && a.inner % kBK == 0;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(tiles, a.batches), dim3(kThreads), 0, stream, (float*)a.out,
                       (const float*)a.left, (const float*)a.right, a.rows, a.columns, a.inner,
                       a.left_batch_stride, a.right_batch_stride);
  };
  if (!chunked) go(gemm_f32_128_kernel<TL, TR, kScalar>);
  else if (grid) go(gemm_f32_128_kernel<TL, TR, kGrid>);
  else go(gemm_f32_128_kernel<TL, TR, kEdge>);
  return hip_status(hipGetLastError());
}

}  // namespace

int launch_gemm_f32(hipStream_t stream, const GemmArgs& a) {
  if (a.batches == 0 || a.rows == 0 || a.columns == 0) return 0;
  if (a.batches > 65535) return IPUS_ERROR_INVALID_ARGUMENT;
  const bool aligned = ((uintptr_t)a.left % 16 == 0) && ((uintptr_t)a.right % 16 == 0) &&
                       ((uintptr_t)a.out % 16 == 0) && a.left_batch_stride % 4 == 0 &&
                       a.right_batch_stride % 4 == 0;
  // 4-float chunks run along the contiguous axis of each operand and of C:
  // N always, K for row-major A or transposed B, M for transposed A.
  const bool chunked = a.columns % 4 == 0 && (a.transpose_left ? a.rows % 4 == 0 : a.inner % 4 == 0) &&
                       (!a.transpose_right || a.inner % 4 == 0);
  // Other shapes and alignments, and K = 0 (every load masked, zeros
  // stored): the same kernel with element loads and stores.
  const bool vec = aligned && chunked && a.inner > 0;
  if (!a.transpose_left && !a.transpose_right) return launch_fast<false, false>(stream, a, vec);
  if (!a.transpose_left && a.transpose_right) return launch_fast<false, true>(stream, a, vec);
  if (a.transpose_left && !a.transpose_right) return launch_fast<true, false>(stream, a, vec);
  return launch_fast<true, true>(stream, a, vec);
}

}  // namespace ipus

// fp16 GEMM on gfx950 MFMA with fp32 accumulation and fp16 output:
//   C[b] = A[b] . B[b]   (A [M,K] or its transpose, B [K,N] or its transpose)
// Replaces gemm_f16_amp (device/gemm_f16_amp.S:186-440), whose partials pass
// through fp16; the accumulation here is fp32 throughout, matching the CPU
// evaluator's fp32 sgemm followed by one fp16 rounding
// (crates/ipu-tests/src/diagnostic.rs:533-654, 841-847).
//
// Fast kernel (16-byte aligned operands; N and K multiples of 8, and M too
// when A is transposed; any M, N, K otherwise):
//   * block tile 256 x 256 x 64, 256 threads = 4 waves in a 2 x 2 grid, each
//     wave owns 128 x 128 of C as 8 x 8 tiles of v_mfma_f32_16x16x32_f16
//     (64 accumulators of 4 fp32, in AGPRs); a K step is two 32-k substeps.
//     On this board the MFMA pipes run under a power limit, and with operands
//     that change every instruction the 16 x 16 x 32 form sustains a ~10%
//     higher clock than 32 x 32 x 16 at the same rate per clock;
//   * the MFMAs are inline assembly with the accumulators tied to AGPRs ("+a"):
//     the compiler's own register assignment for this MFMA copies accumulators
//     between instructions.  Their results are read only after the K loop,
//     past explicit wait states (the compiler pads its own reads of MFMA
//     results, not those of inline assembly);
//   * operand tiles go global -> LDS with buffer_load ... lds (16 bytes per
//     lane, no staging registers; out-of-range reads return 0 instead of
//     faulting).  The DMA writes lane i at base + 16 i, so the LDS swizzle is
//     produced by choosing which global chunk each lane fetches;
//   * an operand whose rows are K-contiguous in memory is stored as
//     [256 rows][64 k] and read with ds_read_b128 (16 rows of one 16-byte
//     chunk per 16 lanes);
//   * an operand whose rows are M/N-contiguous (row-major B, transposed A) is
//     stored as [64 k][256 mn] (512-byte rows) and read with
//     ds_read_b64_tr_b16: in each 16-lane group, source lane s points at row
//     k + s/4, column n + 4 (s % 4), and every lane receives 4 consecutive k
//     of its own column; two such reads give a lane the 8 k of its fragment;
//   * both swizzles are free of bank conflicts for the reads above
//     (SQ_LDS_BANK_CONFLICT checked per layout);
//   * two LDS stages, each a distinct LDS object.  The fragments of a substep
//     are read during the first half of the previous substep into the other
//     of two register buffers, so every read of a stage is issued within its
//     step's first substep and the one raw s_barrier per K step sits between
//     the two; the second substep issues the DMA for step + 2 into the stage
//     just released.  MFMAs, reads and DMA instructions are placed in a fixed
//     order (scheduling fences between slots);
//   * the MFMA computes tiles of C^T (B fragment as the first operand) so
//     each lane holds 4 consecutive columns of one row of C; the epilogue
//     stages each wave's 128 x 128 result in LDS and writes 256-byte row
//     runs with streaming stores (cached stores for a GELU result, which the
//     next GEMM of an MLP reads);
//   * block ids are remapped so that the blocks one XCD runs (round-robin
//     dispatch over 8 XCDs) form a compact group of C tiles sharing L2;
//   * partial tiles: rows of a K-contiguous operand past M or N lie past
//     the buffer's range and read as 0; MN-contiguous chunks past M or N,
//     and (in the KTail instantiation, K % 64 != 0) K-contiguous chunks and
//     MN-contiguous rows past K on the last step, get an offset past the
//     range; the epilogue stores only rows < M and 8-column chunks < N.
// Small-tile kernel (64 x 64 or 32 x 32 tiles): shapes with few 256 x 256
// tiles, and any shape or alignment the fast kernel does not take.
#include "../../include/ipus.h"

#include <mutex>

#include "device_common.h"
#include "kernels.h"

#define LDS_AS __attribute__((address_space(3)))

namespace ipus {
namespace {

constexpr int kBM = 256, kBN = 256;
constexpr int kThreads = 256;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, dword 3 of the descriptor

typedef short short4_t __attribute__((vector_size(8)));

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

// K-contiguous tile [256 rows][BK k]: byte offset of (row, 16-byte chunk).
// A fragment read covers 16 consecutive rows and, per 16-lane group, one
// chunk (4 chunks per instruction); XOR-ing the chunk with the row's low 3
// bits reads without bank conflicts (SQ_LDS_BANK_CONFLICT = 0 in a probe of
// this pattern; the XOR with (row ^ row >> 3) & 7 that suits 32-row reads
// costs 4 conflict cycles per read here).
template <int BK>
__device__ __forceinline__ uint32_t kc_off(uint32_t row, uint32_t chunk) {
  static_assert(BK == 64, "128-byte rows, 8 chunks");
  return row * 128u + ((chunk ^ (row & 7u)) << 4);
}
// MN-contiguous tile [BK k][256 mn]: byte offset of (k, 16-byte chunk along
// mn).  A transposed fragment read covers rows 32 s + 8 g + 4 h + {0..3}
// (g = lane / 16, 16 rows per instruction) and 32 bytes of each; the XOR
// 2 x(k), x(k) = (k & 3) | ((k >> 3) & 1) << 2, spreads those 16 rows over
// the 16 bank groups of 16 bytes twice (two 256-byte cycles, the minimum).
__device__ __forceinline__ uint32_t mc_off(uint32_t k, uint32_t chunk) {
  const uint32_t x = (k & 3u) | (((k >> 3) & 1u) << 2);
  return k * 512u + ((chunk ^ (x << 1)) << 4);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, uint32_t voffset,
                                      uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LDS_AS void*)lds, 16, voffset, soffset, 0, 0);
}

template <int BK>
struct Tile {
  static constexpr int kBytes = kBM * BK * 2;         // one operand tile
  static constexpr int kDmaPerWave = kBytes / 1024 / 4;  // 1 KiB per DMA instruction
};

// Per-lane byte offsets (relative to the block's rsrc base, before the K
// offset) of the DMA instructions this wave issues for one operand tile.  The
// DMA writes lane i at base + 16 i, so each lane fetches the global chunk
// that the swizzle places at its LDS slot.
// Offset of a chunk outside the operand (past M or N along an MN-contiguous
// row, or past K on the last K step of a K-contiguous row): beyond every
// buffer range (< 2^31) plus any K offset (< 2^31) without wrapping, so the
// load returns 0.
constexpr uint32_t kPadOffset = 0x80000000u;

template <int BK, bool KContig>
__device__ __forceinline__ void tile_offsets(uint32_t wave, uint32_t lane, uint32_t ld,
                                             uint32_t mn_limit, uint32_t* voff) {
  constexpr int kChunks = BK / 8;  // 16-byte chunks per K-contiguous row
#pragma unroll
  for (uint32_t j = 0; j < (uint32_t)Tile<BK>::kDmaPerWave; ++j) {
    const uint32_t inst = wave * Tile<BK>::kDmaPerWave + j;
    if constexpr (KContig) {
      const uint32_t row = inst * (1024 / (BK * 2)) + lane / kChunks;
      const uint32_t phys = lane % kChunks;
      // invert the XOR of kc_off for this row
      const uint32_t chunk = (kc_off<BK>(row, phys) - row * (BK * 2)) >> 4;
      voff[j] = (row * ld + chunk * 8) * 2;
    } else {
      const uint32_t k = inst * 2 + lane / 32;  // 2 rows of 512 bytes
      const uint32_t phys = lane % 32;
      const uint32_t chunk = (mc_off(k, phys) - k * 512u) >> 4;
      // mn_limit: columns of this tile inside the operand (rows past K, on
      // the last step only, are masked by issue_one).
      voff[j] = chunk * 8 < mn_limit ? (k * ld + chunk * 8) * 2 : kPadOffset;
    }
  }
}

// DMA instruction j of this wave for one operand tile.  On the last K step
// when K % BK != 0 (k_limit = the step's valid k count, else 0), the chunks
// of a K-contiguous row whose k range starts at or past k_limit, or the rows
// of an MN-contiguous tile at or past k_limit, get an offset past the range
// and read 0: the step's K offset travels in the scalar offset, which the
// descriptor's range check does not cover, so rows past K cannot be left to
// the range of the vector offset alone (they would read the memory after the
// operand).
template <int BK, bool KContig>
__device__ __forceinline__ void issue_one(__amdgpu_buffer_rsrc_t rsrc, uint8_t* tile, uint32_t wave,
                                          uint32_t lane, uint32_t voff, uint32_t j, uint32_t soffset,
                                          uint32_t k_limit) {
  constexpr int kChunks = BK / 8;
  const uint32_t inst = wave * Tile<BK>::kDmaPerWave + j;
  if (k_limit != 0) {
    if constexpr (KContig) {
      const uint32_t row = inst * (1024 / (BK * 2)) + lane / kChunks;
      const uint32_t chunk = (kc_off<BK>(row, lane % kChunks) - row * (BK * 2)) >> 4;
      voff = chunk * 8 < k_limit ? voff : kPadOffset;
    } else {
      voff = inst * 2 + lane / 32 < k_limit ? voff : kPadOffset;  // as tile_offsets
    }
  }
  dma16(rsrc, tile + inst * 1024, voff, soffset);
}

// Epilogues: the plain fp16 product; GELU of it; or the sum of it and an
// addend element (C += A . B, the reference's accumulate mode).
enum Epilogue : int { kEpiPlain = 0, kEpiGelu = 1, kEpiAdd = 2 };

// fp16 result of one accumulator; with GELU, GELU of that fp16 value (the
// same number the separate GELU kernel would produce from the stored GEMM
// output).  The add epilogue applies add_f16 to this value afterwards.
template <int Epi>
__device__ __forceinline__ half_t epilogue(float acc) {
  const half_t h = (half_t)acc;
  if constexpr (Epi == kEpiGelu) return (half_t)gelu_tanh((float)h);
  return h;
}

// The fp16 Add kernel's arithmetic (k_memory.hip add_kernel): both operands
// widened to fp32, summed, rounded once to fp16, so a fused accumulate is
// bit-identical to a GEMM followed by an Add.
__device__ __forceinline__ half_t add_f16(half_t product, half_t addend) {
  return (half_t)((float)addend + (float)product);
}
__device__ __forceinline__ u32x4 add_f16x8(u32x4 product, u32x4 addend) {
  const half8_t p = __builtin_bit_cast(half8_t, product), a = __builtin_bit_cast(half8_t, addend);
  half8_t r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = add_f16(p[e], a[e]);
  return __builtin_bit_cast(u32x4, r);
}

// Split: workgroup z covers K range [z k_chunk, (z + 1) k_chunk) (k_chunk a
// multiple of 64) and writes its fp32 partial tile to out viewed as
// float[splits][batches][M][N] (ipu_stack_gemm_f16_split); otherwise
// k_chunk == K and out is the fp16 C.
// acc += a . b on one 16 x 16 x 32 tile (a: the first operand's 16 rows, b:
// the second's 16 columns), the accumulator tied to AGPRs.
__device__ __forceinline__ void mfma16(float4_t& acc, half8_t a, half8_t b) {
  asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// out may be the addend itself (in place: every element is read and then
// written by the same lane), but not an operand.
template <bool TransposeLeft, bool TransposeRight, int Epi, bool KTail, bool Split>
__global__ __launch_bounds__(kThreads, 1) void gemm_f16_256_kernel(
    uint16_t* out, const uint16_t* __restrict__ left, const uint16_t* __restrict__ right,
    uint32_t M, uint32_t N, uint32_t K, uint64_t left_batch_stride, uint64_t right_batch_stride,
    uint32_t k_chunk, const uint16_t* addend, uint64_t addend_batch_stride,
    uint32_t addend_row_stride) {
  constexpr int BK = 64;
  constexpr int kTileBytes = Tile<BK>::kBytes;
  constexpr int kDma = Tile<BK>::kDmaPerWave;
  // The two stages are distinct LDS objects: the compiler can then see that
  // a DMA into one never aliases the fragment reads of the other.
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b1[kTileBytes];
  constexpr bool kAK = !TransposeLeft;  // A rows (m) K-contiguous
  constexpr bool kBK_ = TransposeRight; // B^T rows (n) K-contiguous

  const uint32_t nbm = (M + kBM - 1) / kBM, nbn = (N + kBN - 1) / kBN;
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
  const uint32_t m0 = bm * kBM, n0 = bn * kBN;

  const uint64_t batch = blockIdx.y;
  const uint16_t* A = left + batch * left_batch_stride;
  const uint16_t* B = right + batch * right_batch_stride;
  uint16_t* C = out + batch * (uint64_t)M * N;

  // This workgroup's K range (the whole of K unless Split).
  const uint32_t k_begin = Split ? blockIdx.z * k_chunk : 0;
  const uint32_t k_len = Split ? (K - k_begin < k_chunk ? K - k_begin : k_chunk) : K;

  // Buffer descriptors based at this block's first row / column and first
  // k; their ranges run to the operand's end.
  const uint16_t* a_base = kAK ? A + (uint64_t)m0 * K + k_begin : A + m0 + (uint64_t)k_begin * M;
  const uint16_t* b_base = kBK_ ? B + (uint64_t)n0 * K + k_begin : B + n0 + (uint64_t)k_begin * N;
  const uint64_t a_bytes = (uint64_t)M * K * 2 - (uint64_t)(a_base - A) * 2;
  const uint64_t b_bytes = (uint64_t)N * K * 2 - (uint64_t)(b_base - B) * 2;
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a_base, 0, (int)(a_bytes > 0x7fffffffull ? 0x7fffffff : a_bytes), kBufferFlags);
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)b_base, 0, (int)(b_bytes > 0x7fffffffull ? 0x7fffffff : b_bytes), kBufferFlags);

  // wave is uniform: readfirstlane puts it in an SGPR, so the LDS
  // addresses of the DMA (M0) are scalar arithmetic.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t lane = threadIdx.x % kWave;
  uint32_t a_voff[kDma], b_voff[kDma];
  tile_offsets<BK, kAK>(wave, lane, kAK ? K : M, M - m0, a_voff);
  tile_offsets<BK, kBK_>(wave, lane, kBK_ ? K : N, N - n0, b_voff);
  // K advance per step in bytes.
  const uint32_t a_kstep = kAK ? BK * 2 : BK * M * 2;
  const uint32_t b_kstep = kBK_ ? BK * 2 : BK * N * 2;

  const uint32_t wm = (wave / 2) * 128, wn = (wave % 2) * 128;

  float4_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t ksteps = (k_len + BK - 1) / BK;
  // K-contiguous operands mask the chunks past K on the last step (MN-
  // contiguous rows past K are past the buffer's range).
  const uint32_t k_tail = k_len % BK;  // nonzero only on the last split
  auto clamp = [&](uint32_t k) { return k < ksteps ? k : ksteps - 1; };
  // KTail (K % BK != 0) is a separate instantiation, so the tail test never
  // enters the K loop of the common case.
  auto limit = [&](uint32_t k) { return KTail && k == ksteps - 1 ? k_tail : 0u; };
  auto dma_a = [&](uint8_t* ta, uint32_t k, uint32_t j) __attribute__((always_inline)) {
    issue_one<BK, kAK>(a_rsrc, ta, wave, lane, a_voff[j], j, k * a_kstep, limit(k));
  };
  auto dma_b = [&](uint8_t* tb, uint32_t k, uint32_t j) __attribute__((always_inline)) {
    issue_one<BK, kBK_>(b_rsrc, tb, wave, lane, b_voff[j], j, k * b_kstep, limit(k));
  };
  auto fetch = [&](uint8_t* ta, uint8_t* tb, uint32_t k) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t j = 0; j < (uint32_t)kDma; ++j) dma_a(ta, k, j);
#pragma unroll
    for (uint32_t j = 0; j < (uint32_t)kDma; ++j) dma_b(tb, k, j);
  };
  // Prologue: K steps 0 and 1 (clamped: K = 64 re-fetches step 0 into a
  // stage that is never read).
  fetch(lds_a0, lds_b0, 0);
  fetch(lds_a1, lds_b1, clamp(1));

  // Fragment addresses from per-lane bases (equal to kc_off / mc_off),
  // r = lane % 16, g = lane / 16.  K-contiguous tile t (rows w0 + 16 t + r),
  // substep s (chunk 4 s + g):
  //   (kbase ^ (64 s)) + 2048 t;
  // MN-contiguous tile t (columns w0 + 16 t + ..), substep s, half h (rows
  // 32 s + 8 g + 4 h + r / 4):
  //   (mbase ^ (t << 5)) + 16384 s + 2048 h.
  const uint32_t r16 = lane % 16, g4 = lane / 16;
  auto k_base = [&](uint32_t w0) {
    return (w0 + r16) * 128 + ((g4 ^ (r16 & 7)) << 4);
  };
  auto m_base = [&](uint32_t w0) {
    const uint32_t r4 = r16 / 4, c1 = (r16 % 4) / 2, xr = r4 | ((g4 & 1) << 2);
    return (8 * g4 + r4) * 512 + 2 * w0 + 16 * c1 + 8 * (r16 % 2) + (xr << 5);
  };
  const uint32_t a_base_l = kAK ? k_base(wm) : m_base(wm);
  const uint32_t b_base_l = kBK_ ? k_base(wn) : m_base(wn);
  auto frag = [&]<bool KContig>(const uint8_t* tile, uint32_t base, int t, int s) __attribute__((always_inline)) {
    if constexpr (KContig) {
      return __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4*>(tile + ((base ^ (64 * s)) + 2048 * t)));
    } else {
      const uint32_t a = (base ^ (t << 5)) + 16384 * s;
      const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(tile + a));
      const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(tile + a + 2048));
      return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  half8_t fa[2][8], fb[2][8];
  // Fragment item r of a substep: r < 8 is B tile r, r >= 8 is A tile r - 8
  // (the order in which that substep's MFMAs first use them).
  auto read_item = [&](const uint8_t* ta, const uint8_t* tb, int s, int buf, int r) __attribute__((always_inline)) {
    if (r < 8) fb[buf][r] = frag.template operator()<kBK_>(tb, b_base_l, r, s);
    else fa[buf][r - 8] = frag.template operator()<kAK>(ta, a_base_l, r - 8, s);
  };
  // One substep: the 64 MFMAs of register buffer buf; after every second
  // MFMA of the first 32, one fragment of the next substep (into buffer
  // 1 - buf); with dma_k >= 0, the step's 2 x kDma DMA instructions after
  // every fourth MFMA.  Fences keep this order.
  auto substep = [&](int buf, const uint8_t* ra, const uint8_t* rb, int rs, uint8_t* da, uint8_t* db,
                     int64_t dma_k) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 64; ++m) {
      const int i = m / 8, j = m % 8;
      mfma16(acc[i][j], fb[buf][j], fa[buf][i]);
      if (m < 32 && m % 2 == 1) read_item(ra, rb, rs, 1 - buf, m / 2);
      if (dma_k >= 0 && m % 4 == 1) {
        const int d = m / 4;
        if (d < kDma) dma_a(da, (uint32_t)dma_k, d);
        else dma_b(db, (uint32_t)dma_k, d - kDma);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int r = 0; r < 16; ++r) read_item(lds_a0, lds_b0, 0, 0, r);
  auto step = [&](uint8_t* ta, uint8_t* tb, const uint8_t* na, const uint8_t* nb, uint32_t kt)
      __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    substep(0, ta, tb, 1, nullptr, nullptr, -1);
    // This wave's reads of (ta, tb) have returned and its DMA of step kt + 1
    // has landed; after the barrier, every wave's have.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    substep(1, na, nb, 0, ta, tb, (int64_t)clamp(kt + 2));
  };

  uint32_t kt = 0;
  for (; kt + 1 < ksteps; kt += 2) {
    step(lds_a0, lds_b0, lds_a1, lds_b1, kt);
    step(lds_a1, lds_b1, lds_a0, lds_b0, kt + 1);
  }
  if (kt < ksteps) step(lds_a0, lds_b0, lds_a1, lds_b1, kt);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // drain the redundant prefetches
  // 24 wait states before any read of the accumulators (see mfma16).
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  // acc[i][j][e] = C[m0 + wm + 16 i + lane % 16][n0 + wn + 16 j + 4 (lane / 16) + e]
  if constexpr (Split) {
    // fp32 partial tile, 16-byte stores of 4 consecutive columns.
    float* P = reinterpret_cast<float*>(out) +
               ((uint64_t)blockIdx.z * gridDim.y + batch) * (uint64_t)M * N;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t row = m0 + wm + 16 * i + r16;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t col = n0 + wn + 16 * j + 4 * g4;
        if (col >= N) continue;
        __builtin_nontemporal_store(acc[i][j], reinterpret_cast<float4_t*>(P + (uint64_t)row * N + col));
      }
    }
    return;
  }

  // The wave's 128 x 128 fp16 result goes through its own quarter of the
  // (now idle) LDS stages, so that it reaches memory as 256-byte row runs
  // written by 16 lanes with streaming stores instead of 8-byte pieces of
  // 16 rows per instruction.  Layout: row r (256 bytes), 16-byte chunk c at
  // chunk c ^ (r & 15).
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave is done with the stages
  uint8_t* cst = wave == 0 ? lds_a0 : wave == 1 ? lds_b0 : wave == 2 ? lds_a1 : lds_b1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t r = 16 * i + r16;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half4_t h;
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = epilogue<Epi>(acc[i][j][e]);
      const uint32_t c = 2 * j + g4 / 2;
      *reinterpret_cast<half4_t*>(cst + r * 256 + ((c ^ (r & 15)) << 4) + (g4 % 2) * 8) = h;
    }
  }
  uint16_t* cw = C + (uint64_t)(m0 + wm) * N + n0 + wn;
  if constexpr (Epi == kEpiAdd) {
    // The addend's chunks are loaded 8 at a time ahead of their stores
    // (out may be the addend, so a load cannot move past an earlier store).
    const uint16_t* aw = addend + batch * addend_batch_stride +
                         (uint64_t)(m0 + wm) * addend_row_stride + n0 + wn;
#pragma unroll
    for (int k0 = 0; k0 < 32; k0 += 8) {
      u32x4 d[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t v = (k0 + k) * kWave + lane, r = v / 16, c = v % 16;
        d[k] = m0 + wm + r < M && n0 + wn + c * 8 < N
                   ? *reinterpret_cast<const u32x4*>(aw + (uint64_t)r * addend_row_stride + c * 8)
                   : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t v = (k0 + k) * kWave + lane, r = v / 16, c = v % 16;
        const u32x4 x = *reinterpret_cast<const u32x4*>(cst + r * 256 + ((c ^ (r & 15)) << 4));
        if (m0 + wm + r < M && n0 + wn + c * 8 < N)
          __builtin_nontemporal_store(add_f16x8(x, d[k]),
                                      reinterpret_cast<u32x4*>(cw + (uint64_t)r * N + c * 8));
      }
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint32_t v = k * kWave + lane, r = v / 16, c = v % 16;
    const u32x4 x = *reinterpret_cast<const u32x4*>(cst + r * 256 + ((c ^ (r & 15)) << 4));
    // Rows past M and 8-column chunks past N (N % 8 == 0) are not stored.
    // A GELU result is the next GEMM's operand (the MLP's hidden layer), so
    // it is stored through the caches for that GEMM to find in L2 and the
    // MALL: the MLP graph 1,338 -> 1,357 TFLOP/s; cached stores of the plain
    // product cost the 8192^3 GEMMs 1.5%.
    if (m0 + wm + r < M && n0 + wn + c * 8 < N) {
      u32x4* p = reinterpret_cast<u32x4*>(cw + (uint64_t)r * N + c * 8);
      if constexpr (Epi == kEpiGelu) *p = x;
      else __builtin_nontemporal_store(x, p);
    }
  }
}

// Small fp16 GEMM: 64 x 64 or 32 x 32 output tiles, for shapes with fewer
// 256 x 256 tiles than kSmallBelowTiles, which would keep few of the 256
// CUs busy (configs[0]'s 256^3 is a single such tile).  256 threads = 4
// waves in a 2 x 2 grid, each (Tile / 2)^2 of C as tiles of
// v_mfma_f32_16x16x32_f16 (C^T as in the 256 x 256 kernel, so a lane holds
// 4 consecutive columns).  K runs in chunks of 256: a chunk's
// operand tiles (4 steps of 64) are loaded to registers, 16 loads of 16
// bytes per thread in flight at once, stored to four LDS stages, and
// computed while the next chunk's loads are in flight; a K of at most 256
// takes one memory round trip.  K-contiguous tiles are stored [64 rows][64 k]
// with the 256 x 256 kernel's XOR swizzle and read with ds_read_b128;
// MN-contiguous tiles [64 k][64 mn] are read with ds_read_b64_tr_b16.
// Chunks past M, N or K are not loaded and stay 0.  Vec = 8: N and K, and
// M when A is transposed, are multiples of 8 and the operands 16-byte
// aligned, as for the 256 x 256 kernel.  Vec = 4 or 1 (any other shape or
// alignment, where the 256 x 256 kernel cannot run): each 16-byte LDS chunk
// is gathered from 8-byte or 2-byte loads, elements past M, N or K are 0,
// and the epilogue stores element by element.
constexpr uint32_t kSmallChunk = 256;
constexpr uint32_t kSmallSteps = kSmallChunk / 64;
constexpr uint64_t kSmallBelowTiles = 32;

template <uint32_t Tile, bool TransposeLeft, bool TransposeRight, int Epi, int Vec = 8>
__global__ __launch_bounds__(256) void gemm_f16_small_kernel(
    uint16_t* out, const uint16_t* __restrict__ left, const uint16_t* __restrict__ right,
    uint32_t M, uint32_t N, uint32_t K, uint64_t left_batch_stride, uint64_t right_batch_stride,
    uint32_t tiles_n, const uint16_t* addend, uint64_t addend_batch_stride,
    uint32_t addend_row_stride) {
  constexpr uint32_t kWT = Tile / 32;                 // 16 x 16 tiles per wave and dimension
  constexpr uint32_t kStepBytes = Tile * 64 * 2;      // one operand, one 64-k step
  constexpr uint32_t kMnRow = Tile * 2;               // bytes of an MN-contiguous k row
  constexpr uint32_t kMnChunks = Tile / 8;            // 16-byte chunks of such a row
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][kSmallSteps][kStepBytes];
  constexpr bool kAK = !TransposeLeft;   // A rows (m) K-contiguous
  constexpr bool kBK_ = TransposeRight;  // B^T rows (n) K-contiguous
  const uint64_t batch = blockIdx.y;
  const uint16_t* A = left + batch * left_batch_stride;
  const uint16_t* B = right + batch * right_batch_stride;
  uint16_t* C = out + batch * (uint64_t)M * N;
  const uint32_t m0 = blockIdx.x / tiles_n * Tile, n0 = blockIdx.x % tiles_n * Tile;
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t wm = (wave / 2) * (Tile / 2), wn = (wave % 2) * (Tile / 2);
  const uint32_t r16 = lane % 16, g4 = lane / 16;

  // Chunk q = threadIdx.x + 256 i of an operand's 4 steps: step q / (steps'
  // chunks), then (row, k chunk) for a K-contiguous tile (8 chunks a row) or
  // (k row, mn chunk) for an MN-contiguous one (Tile / 8 chunks a row).
  constexpr uint32_t kStepChunks = kStepBytes / 16;
  constexpr uint32_t kPer = kSmallSteps * kStepChunks / 256;
  u32x4 ra[kPer], rb[kPer];
  auto load_operand = [&]<bool KContig>(const uint16_t* X, uint32_t mn0, uint32_t mn_limit,
                                        uint32_t ld, uint32_t k0, u32x4* r) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = threadIdx.x + 256 * i, step = q / kStepChunks, w = q % kStepChunks;
      const uint32_t per_row = KContig ? 8 : kMnChunks;
      const uint32_t major = w / per_row, minor = w % per_row * 8;
      const uint32_t k = KContig ? k0 + step * 64 + minor : k0 + step * 64 + major;
      const uint32_t mn = KContig ? mn0 + major : mn0 + minor;
      const uint16_t* p = X + (KContig ? (uint64_t)mn * ld + k : (uint64_t)k * ld + mn);
      if constexpr (Vec == 8) {
        const bool ok = k < K && mn < mn_limit;
        r[i] = ok ? load16(p) : u32x4{0, 0, 0, 0};
      } else {
        // The chunk's 8 elements run along the contiguous axis (k or mn);
        // groups of Vec are wholly in or out, as Vec divides that extent.
        const bool row_ok = KContig ? mn < mn_limit : k < K;
        const uint32_t c0 = KContig ? k : mn, c_limit = KContig ? K : mn_limit;
        uint16_t e[8];
#pragma unroll
        for (uint32_t g = 0; g < 8; g += Vec) {
          const bool ok = row_ok && c0 + g < c_limit;
          if constexpr (Vec == 4) {
            const u32x2 v = ok ? *reinterpret_cast<const u32x2*>(p + g) : u32x2{0, 0};
            e[g] = (uint16_t)v[0];
            e[g + 1] = (uint16_t)(v[0] >> 16);
            e[g + 2] = (uint16_t)v[1];
            e[g + 3] = (uint16_t)(v[1] >> 16);
          } else {
            e[g] = ok ? p[g] : (uint16_t)0;
          }
        }
        r[i] = u32x4{e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                     e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16};
      }
    }
  };
  auto store_operand = [&]<bool KContig>(uint8_t (*stage)[kStepBytes], const u32x4* r) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
      const uint32_t q = threadIdx.x + 256 * i, step = q / kStepChunks, w = q % kStepChunks;
      const uint32_t per_row = KContig ? 8 : kMnChunks;
      const uint32_t major = w / per_row, chunk = w % per_row;
      const uint32_t off = KContig ? kc_off<64>(major, chunk) : major * kMnRow + chunk * 16;
      *reinterpret_cast<u32x4*>(stage[step] + off) = r[i];
    }
  };
  auto load_chunk = [&](uint32_t k0) __attribute__((always_inline)) {
    load_operand.template operator()<kAK>(A, m0, M, kAK ? K : M, k0, ra);
    load_operand.template operator()<kBK_>(B, n0, N, kBK_ ? K : N, k0, rb);
  };
  auto store_chunk = [&]() __attribute__((always_inline)) {
    store_operand.template operator()<kAK>(lds[0], ra);
    store_operand.template operator()<kBK_>(lds[1], rb);
  };
  // Fragment of 16 rows (m or n) w0 + 16 t + .., k 32 ss + 8 (lane / 16) ..+7.
  auto frag = [&]<bool KContig>(const uint8_t* tile, uint32_t w0, uint32_t t, uint32_t ss) __attribute__((always_inline)) {
    if constexpr (KContig) {
      const uint32_t row = w0 + 16 * t + r16;
      return __builtin_bit_cast(
          half8_t, *reinterpret_cast<const u32x4*>(tile + kc_off<64>(row, 4 * ss + g4)));
    } else {
      // 16-lane group g reads k rows 32 ss + 8 g + {0..3} (then +4): lane s
      // addresses k row + s / 4, columns w0 + 16 t + 4 (s % 4) .. +3.
      const uint32_t k = 32 * ss + 8 * g4 + r16 / 4;
      const uint32_t a = k * kMnRow + (w0 + 16 * t + 4 * (r16 % 4)) * 2;
      const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(tile + a));
      const short4_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS short4_t*)(tile + a + 4 * kMnRow));
      return __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  float4_t acc[kWT][kWT];
#pragma unroll
  for (uint32_t i = 0; i < kWT; ++i)
#pragma unroll
    for (uint32_t j = 0; j < kWT; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t chunks = (K + kSmallChunk - 1) / kSmallChunk;
  load_chunk(0);
  store_chunk();
  __syncthreads();
  for (uint32_t c = 0; c < chunks; ++c) {
    if (c + 1 < chunks) load_chunk((c + 1) * kSmallChunk);
#pragma unroll
    for (uint32_t step = 0; step < kSmallSteps; ++step)
#pragma unroll
      for (uint32_t ss = 0; ss < 2; ++ss) {
        half8_t fa[kWT], fb[kWT];
#pragma unroll
        for (uint32_t t = 0; t < kWT; ++t) {
          fa[t] = frag.template operator()<kAK>(lds[0][step], wm, t, ss);
          fb[t] = frag.template operator()<kBK_>(lds[1][step], wn, t, ss);
        }
#pragma unroll
        for (uint32_t i = 0; i < kWT; ++i)
#pragma unroll
          for (uint32_t j = 0; j < kWT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[j], fa[i], acc[i][j], 0, 0, 0);
      }
    if (c + 1 < chunks) {
      __syncthreads();  // every wave is done reading the stages
      store_chunk();
      __syncthreads();
    }
  }
  // acc[i][j][e] = C[m0 + wm + 16 i + lane % 16][n0 + wn + 16 j + 4 (lane / 16) + e]
#pragma unroll
  for (uint32_t i = 0; i < kWT; ++i) {
    const uint32_t m = m0 + wm + 16 * i + r16;
    if (m >= M) continue;
#pragma unroll
    for (uint32_t j = 0; j < kWT; ++j) {
      const uint32_t n = n0 + wn + 16 * j + 4 * g4;
      if (n >= N) continue;
      half4_t h;
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = epilogue<Epi>(acc[i][j][e]);
      if constexpr (Vec == 8) {
        // N % 8 == 0: a lane's 4 columns are all in or all out.
        if constexpr (Epi == kEpiAdd) {
          const half4_t d = *reinterpret_cast<const half4_t*>(
              addend + batch * addend_batch_stride + (uint64_t)m * addend_row_stride + n);
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = add_f16(h[e], d[e]);
        }
        *reinterpret_cast<half4_t*>(C + (uint64_t)m * N + n) = h;
      } else {
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
          if (n + e >= N) break;
          half_t v = h[e];
          if constexpr (Epi == kEpiAdd)
            v = add_f16(v, __builtin_bit_cast(half_t, addend[batch * addend_batch_stride +
                                                             (uint64_t)m * addend_row_stride + n + e]));
          C[(uint64_t)m * N + n + e] = __builtin_bit_cast(uint16_t, v);
        }
      }
    }
  }
}

// 64 x 64 tiles, or 32 x 32 when there are fewer 64 x 64 tiles than a
// quarter of the CUs (256^3: 64 workgroups instead of 16).
template <int Epi, int Vec = 8>
int launch_small(hipStream_t stream, const GemmArgs& a) {
  const uint64_t tiles64 = (uint64_t)((a.rows + 63) / 64) * ((a.columns + 63) / 64);
  const uint32_t tile = tiles64 * a.batches < 64 ? 32 : 64;
  const uint32_t tiles_m = (a.rows + tile - 1) / tile;
  const uint32_t tiles_n = (a.columns + tile - 1) / tile;
  if ((uint64_t)tiles_m * tiles_n > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  const dim3 grid(tiles_m * tiles_n, a.batches);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, (uint16_t*)a.out,
                       (const uint16_t*)a.left, (const uint16_t*)a.right, a.rows, a.columns,
                       a.inner, a.left_batch_stride, a.right_batch_stride, tiles_n,
                       (const uint16_t*)a.addend, a.addend_batch_stride, a.addend_row_stride);
  };
  const bool tl = a.transpose_left, tr = a.transpose_right;
  if (tile == 32) {
    if (!tl && !tr) go(gemm_f16_small_kernel<32, false, false, Epi, Vec>);
    else if (!tl) go(gemm_f16_small_kernel<32, false, true, Epi, Vec>);
    else if (!tr) go(gemm_f16_small_kernel<32, true, false, Epi, Vec>);
    else go(gemm_f16_small_kernel<32, true, true, Epi, Vec>);
  } else {
    if (!tl && !tr) go(gemm_f16_small_kernel<64, false, false, Epi, Vec>);
    else if (!tl) go(gemm_f16_small_kernel<64, false, true, Epi, Vec>);
    else if (!tr) go(gemm_f16_small_kernel<64, true, false, Epi, Vec>);
    else go(gemm_f16_small_kernel<64, true, true, Epi, Vec>);
  }
  return hip_status(hipGetLastError());
}

// Elements per global load (8, 4 or 1) that every operand row, batch and
// base address allows, and 8 only where the addend and output allow the
// 16-byte epilogue too.
uint32_t small_vec(const GemmArgs& a) {
  auto fits = [&](uint32_t v) {
    const uint32_t lda = a.transpose_left ? a.rows : a.inner;
    const uint32_t ldb = a.transpose_right ? a.inner : a.columns;
    bool ok = lda % v == 0 && ldb % v == 0 && (uintptr_t)a.left % (2 * v) == 0 &&
              (uintptr_t)a.right % (2 * v) == 0 && a.left_batch_stride % v == 0 &&
              a.right_batch_stride % v == 0;
    if (v == 8)
      ok = ok && a.inner % 8 == 0 && a.columns % 8 == 0 && (uintptr_t)a.out % 16 == 0 &&
           (!a.addend || ((uintptr_t)a.addend % 16 == 0 && a.addend_batch_stride % 8 == 0 &&
                          a.addend_row_stride % 8 == 0));
    return ok;
  };
  return fits(8) ? 8u : fits(4) ? 4u : 1u;
}

template <int Epi>
int launch_small_any(hipStream_t stream, const GemmArgs& a) {
  switch (small_vec(a)) {
    case 8: return launch_small<Epi, 8>(stream, a);
    case 4: return launch_small<Epi, 4>(stream, a);
    default: return launch_small<Epi, 1>(stream, a);
  }
}

template <bool TL, bool TR, int Epi, bool Split>
int launch_fast(hipStream_t stream, const GemmArgs& a, uint32_t splits, uint32_t k_chunk) {
  const uint32_t tiles = ((a.rows + kBM - 1) / kBM) * ((a.columns + kBN - 1) / kBN);
  const dim3 grid(tiles, a.batches, splits);
  if (a.inner % 64 == 0)
    hipLaunchKernelGGL((gemm_f16_256_kernel<TL, TR, Epi, false, Split>), grid, dim3(kThreads), 0,
                       stream, (uint16_t*)a.out, (const uint16_t*)a.left, (const uint16_t*)a.right,
                       a.rows, a.columns, a.inner, a.left_batch_stride, a.right_batch_stride,
                       k_chunk, (const uint16_t*)a.addend, a.addend_batch_stride,
                       a.addend_row_stride);
  else
    hipLaunchKernelGGL((gemm_f16_256_kernel<TL, TR, Epi, true, Split>), grid, dim3(kThreads), 0,
                       stream, (uint16_t*)a.out, (const uint16_t*)a.left, (const uint16_t*)a.right,
                       a.rows, a.columns, a.inner, a.left_batch_stride, a.right_batch_stride,
                       k_chunk, (const uint16_t*)a.addend, a.addend_batch_stride,
                       a.addend_row_stride);
  return hip_status(hipGetLastError());
}

template <int Epi, bool Split>
int dispatch_fast(hipStream_t stream, const GemmArgs& a, uint32_t splits, uint32_t k_chunk) {
  if (!a.transpose_left && !a.transpose_right)
    return launch_fast<false, false, Epi, Split>(stream, a, splits, k_chunk);
  if (!a.transpose_left && a.transpose_right)
    return launch_fast<false, true, Epi, Split>(stream, a, splits, k_chunk);
  if (a.transpose_left && !a.transpose_right)
    return launch_fast<true, false, Epi, Split>(stream, a, splits, k_chunk);
  return launch_fast<true, true, Epi, Split>(stream, a, splits, k_chunk);
}

int epilogue_of(const GemmArgs& a) {
  return a.addend ? kEpiAdd : a.gelu ? kEpiGelu : kEpiPlain;
}

// Conditions of the 256 x 256 kernel: 16-byte aligned operands, 32-bit
// per-block buffer offsets, 16-byte chunks (N and K, and M when A is
// transposed, multiples of 8).
bool fast_ok(const GemmArgs& a) {
  const bool aligned = ((uintptr_t)a.left % 16 == 0) && ((uintptr_t)a.right % 16 == 0) &&
                       ((uintptr_t)a.out % 16 == 0) && a.left_batch_stride % 8 == 0 &&
                       a.right_batch_stride % 8 == 0;
  const uint64_t a_span = a.transpose_left ? (uint64_t)a.inner * a.rows * 2 : 256ull * a.inner * 2;
  const uint64_t b_span = a.transpose_right ? 256ull * a.inner * 2 : (uint64_t)a.inner * a.columns * 2;
  const bool fits = a_span < (1ull << 31) && b_span < (1ull << 31);
  const bool chunked = a.inner % 8 == 0 && a.columns % 8 == 0 && (!a.transpose_left || a.rows % 8 == 0);
  // The add epilogue loads the addend as 16-byte chunks of 8 columns.
  const bool addend_ok = !a.addend || ((uintptr_t)a.addend % 16 == 0 &&
                                       a.addend_batch_stride % 8 == 0 && a.addend_row_stride % 8 == 0);
  return aligned && fits && chunked && addend_ok && a.inner > 0;
}

// fp32 partials [splits][count] -> fp16 (optionally GELU of the fp16 value):
// 8 elements per thread, splits summed in order.
// With an addend (out may be the addend): out = add_f16(sum, addend) for the
// addend element of (batch, row, column), count = batches * rows * columns.
__global__ __launch_bounds__(256) void reduce_splits_f16_kernel(
    uint16_t* out, const float* __restrict__ parts, uint32_t splits, uint64_t count, bool gelu,
    const uint16_t* addend, uint32_t rows, uint32_t columns, uint64_t addend_batch_stride,
    uint32_t addend_row_stride) {
  const uint64_t i = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= count) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (uint32_t s = 0; s < splits; ++s) {
    const float* p = parts + (uint64_t)s * count + i;
    const float4_t lo = __builtin_nontemporal_load(reinterpret_cast<const float4_t*>(p));
    const float4_t hi = __builtin_nontemporal_load(reinterpret_cast<const float4_t*>(p + 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] += lo[e];
      acc[4 + e] += hi[e];
    }
  }
  half8_t h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = gelu ? epilogue<kEpiGelu>(acc[e]) : epilogue<kEpiPlain>(acc[e]);
  if (addend) {
    // columns % 8 == 0, so the 8 elements share one row.
    const uint64_t row = i / columns, col = i % columns;
    const uint64_t b = row / rows, m = row % rows;
    const half8_t d = *reinterpret_cast<const half8_t*>(addend + b * addend_batch_stride +
                                                        m * addend_row_stride + col);
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = add_f16(h[e], d[e]);
  }
  *reinterpret_cast<half8_t*>(out + i) = h;
}

}  // namespace

int gemm_f16_split_chunk(uint32_t inner, uint32_t splits) {
  if (splits == 0 || inner == 0) return 0;
  const uint32_t per = (inner + splits - 1) / splits;
  return (int)((per + 63) / 64 * 64);
}

int launch_gemm_f16_split(hipStream_t stream, const GemmArgs& a, uint32_t splits) {
  if (a.batches == 0 || a.rows == 0 || a.columns == 0) return 0;
  if (a.batches > 65535 || splits == 0 || splits > 64 || a.gelu || a.addend)
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (!fast_ok(a)) return IPUS_ERROR_UNAVAILABLE;
  const uint32_t k_chunk = (uint32_t)gemm_f16_split_chunk(a.inner, splits);
  // Every split must own at least one k: the plan picks splits so that
  // ceil(K / k_chunk) == splits.
  if ((a.inner + k_chunk - 1) / k_chunk != splits) return IPUS_ERROR_INVALID_ARGUMENT;
  return dispatch_fast<kEpiPlain, true>(stream, a, splits, k_chunk);
}

int launch_reduce_splits_f16(hipStream_t stream, void* dst, const void* parts, uint32_t splits,
                             uint64_t count, bool gelu, const SplitAddend* add) {
  if (count == 0) return 0;
  if (splits == 0 || count % 8 != 0 || (uintptr_t)dst % 16 != 0 || (uintptr_t)parts % 16 != 0)
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (add && (gelu || !add->addend || add->rows == 0 || add->columns == 0 ||
              add->columns % 8 != 0 || count % ((uint64_t)add->rows * add->columns) != 0 ||
              (uintptr_t)add->addend % 16 != 0 || add->batch_stride % 8 != 0 ||
              add->row_stride % 8 != 0))
    return IPUS_ERROR_INVALID_ARGUMENT;
  const uint64_t blocks = (count / 8 + 255) / 256;
  if (blocks > 0x7fffffffu) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(reduce_splits_f16_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     (uint16_t*)dst, (const float*)parts, splits, count, gelu,
                     add ? (const uint16_t*)add->addend : nullptr, add ? add->rows : 1u,
                     add ? add->columns : 8u, add ? add->batch_stride : 0ull,
                     add ? add->row_stride : 0u);
  return hip_status(hipGetLastError());
}

int launch_gemm_f16(hipStream_t stream, const GemmArgs& a) {
  if (a.batches == 0 || a.rows == 0 || a.columns == 0) return 0;
  if (a.batches > 65535 || (a.gelu && a.addend)) return IPUS_ERROR_INVALID_ARGUMENT;
  // Any M and N on the fast kernel: rows past the edge read as 0 and are not
  // stored.
  if (fast_ok(a)) {
    // Fewer 256 x 256 tiles than kSmallBelowTiles: the small-tile kernel
    // (measured: 256^3 10.7 -> 5.3 us a launch, 1024^3 22 -> 9.6, but
    // 2048^3 with 64 tiles 40 -> 47).
    const uint64_t tiles = (uint64_t)((a.rows + kBM - 1) / kBM) * ((a.columns + kBN - 1) / kBN);
    if (tiles * a.batches < kSmallBelowTiles) {
      switch (epilogue_of(a)) {
        case kEpiGelu: return launch_small<kEpiGelu>(stream, a);
        case kEpiAdd: return launch_small<kEpiAdd>(stream, a);
        default: return launch_small<kEpiPlain>(stream, a);
      }
    }
    switch (epilogue_of(a)) {
      case kEpiGelu: return dispatch_fast<kEpiGelu, false>(stream, a, 1, a.inner);
      case kEpiAdd: return dispatch_fast<kEpiAdd, false>(stream, a, 1, a.inner);
      default: return dispatch_fast<kEpiPlain, false>(stream, a, 1, a.inner);
    }
  }
  // Any other shape or alignment (or operands past the 256 x 256 kernel's
  // 31-bit buffer ranges): the small-tile kernel with the widest loads the
  // operands allow.
  switch (epilogue_of(a)) {
    case kEpiGelu: return launch_small_any<kEpiGelu>(stream, a);
    case kEpiAdd: return launch_small_any<kEpiAdd>(stream, a);
    default: return launch_small_any<kEpiPlain>(stream, a);
  }
}

// ---------------------------------------------------------------------------
// Split-K without allocation (ipus_gemm_f16_split_noalloc): the fp32
// partials go to `scratch`, a file-scope device array of
// IPUS_SPLIT_SCRATCH_BYTES that each device holds from module load until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol): split_scratch_init looks up
// each device's copy once, with that device current, and the launches take
// the looked-up pointer.  Every split writes its whole partial tile, so
// nothing in the array has to start at zero.  All calls on one device share
// its array: calls that overlap on one device (different streams) race.
// ---------------------------------------------------------------------------
namespace {
static __device__ __align__(256) float scratch[IPUS_SPLIT_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

int split_scratch_init(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return IPUS_ERROR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device]) return 0;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_status(e);
  if (!ptr) return IPUS_ERROR_INVALID_ARGUMENT;
  g_scratch_ptr[device] = ptr;
  return 0;
}

int launch_gemm_f16_split_noalloc(hipStream_t stream, int device, const GemmArgs& a,
                                  uint32_t splits) {
  if (a.batches == 0 || a.rows == 0 || a.columns == 0) return 0;
  void* parts = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (device >= 0 && device < kMaxScratchDevices) parts = g_scratch_ptr[device];
  }
  if (!parts) return IPUS_ERROR_NO_DEVICE;
  uint64_t count = 0, total = 0;
  if (splits == 0 || __builtin_mul_overflow((uint64_t)a.batches, (uint64_t)a.rows, &count) ||
      __builtin_mul_overflow(count, (uint64_t)a.columns, &count) ||
      __builtin_mul_overflow(count, (uint64_t)splits, &total) ||
      total > IPUS_SPLIT_SCRATCH_BYTES / sizeof(float))
    return IPUS_ERROR_UNSUPPORTED_COUNT;
  GemmArgs s = a;
  s.out = parts;
  s.gelu = false;
  if (int e = launch_gemm_f16_split(stream, s, splits)) return e;
  return launch_reduce_splits_f16(stream, a.out, parts, splits, count, a.gelu, nullptr);
}

}  // namespace ipus

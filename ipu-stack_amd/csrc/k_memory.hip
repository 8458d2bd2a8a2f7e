// Bandwidth-bound kernels for gfx950: transpose, rearranges into the
// reference's storage orders, unpack, row reduction, the reference's
// partial-sum reduction, GELU, casts, add and split_heads.
//
// Design: every hot kernel moves 16-byte vectors per lane and keeps each
// wave's global accesses in whole 128-byte lines.  Transposes of 16-bit data
// are done in registers on 8x8 blocks (no LDS, no bank conflicts): a lane
// reads 8 rows x 16 bytes and writes 8 rows x 16 bytes.  Inputs that are
// read once are loaded with non-temporal loads (measured on MI355X: row
// reductions 5.7 -> 6.0 and 6.0 -> 6.3 TB/s, GELU 5.6 -> 5.8, transpose
// +3%).
#include "../../include/ipus.h"
#include "device_common.h"
#include "kernels.h"
#include "layout_maps.h"

namespace ipus {

namespace {

constexpr int kThreads = 256;
// Rows of the tiles of the AMP-Left / AMP-TransposedRight conversions and
// the AMP-Output unpack: 256 rows x 64 columns per workgroup, 8 chunks of 16
// bytes per thread, all loaded before any is stored.
// Rows of the AMP-Output unpack's tiles (32 rows x 64 columns: one 16-byte
// chunk per thread; 64-row tiles with two chunks in flight per thread
// measured 5.35 TB/s against 5.40, 256-row tiles 2.8).
constexpr uint32_t kAmpTileRows = 32;

// LDS bytes a workgroup requests (on top of its static LDS) so that at most
// `workgroups` of it share a CU: the launch keeps no more than that many
// resident, whatever its registers would allow (160 KiB of LDS per CU).
constexpr uint32_t occupancy_lds(uint32_t workgroups, uint32_t static_bytes) {
  return 163840u / (workgroups + 1) + 1 - static_bytes;
}

inline int hip_status(hipError_t e) { return e == hipSuccess ? 0 : IPUS_ERROR_HIP_BASE - (int)e; }

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Tile (tr, tc) of a tiles_r x tiles_c grid (tiles_r * tiles_c == gridDim.x)
// for this workgroup.  Workgroups are dealt round-robin to the 8 XCDs, so the
// ids are first regrouped into one contiguous range of tiles per XCD; the
// column is then rotated by slope x the row (diagonal order) so that the
// tiles in flight write to spread-out destination rows.  Measured on 8192^2
// fp16: 4.3 -> 5.1 TB/s for the transpose together with streaming stores
// (slope 1); slope 7 or 9 is another 2% (5.43 -> 5.54 TB/s; plain
// dispatch order without the regroup: 3.8).
__device__ __forceinline__ void tile_of_block(uint32_t tiles_c, uint32_t slope, uint32_t* tr,
                                              uint32_t* tc) {
  const uint32_t n = gridDim.x;
  uint32_t b = blockIdx.x;
  if (n % 8 == 0) b = (b % 8) * (n / 8) + b / 8;
  *tr = b / tiles_c;
  *tc = (uint32_t)((b % tiles_c + (uint64_t)*tr * slope) % tiles_c);
}

// Non-temporal 16-byte load, for inputs that the kernel reads once.
__device__ __forceinline__ u32x4 load16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Streaming (non-temporal) 16-byte store, for outputs that the kernel
// writes in whole 128-byte lines per wave instruction: a streaming store
// of a partial line skips the L2 write merge (block-major stores, 32-byte
// runs per instruction, use ordinary stores).
__device__ __forceinline__ void store16_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Transpose: [matrices][rows][columns] -> [matrices][columns][rows].
// A wave owns a 64x64 tile; lane (rc = lane % 8, cc = lane / 8) owns the 8x8
// block at rows 8*rc, columns 8*cc.  For each of the 8 loads the wave reads 8
// rows x 128 contiguous bytes; for each store it writes 8 rows x 128 bytes.
// A workgroup of 8 waves stacks their tiles vertically (512 rows x 64
// columns), so together they write 1 KiB runs of each destination row, and
// one workgroup runs per CU (the launch requests LDS it does not use, see
// occupancy_lds): fewer tiles in flight at once keep the reads and writes
// of the whole chip on fewer DRAM rows.  Measured on 8192^2 fp16, TB/s:
// 256 x 64 tiles of 4 waves 5.40 with up to 6 workgroups per CU, 5.70 with
// 3; 512 x 64 with one 5.81-5.83 (with two 5.48; 1024 x 64, 768 x 64 and
// 512 x 128 with one: 5.36, 5.43, 5.39; 128 x 128 with 3-4: 5.21; a
// persistent grid loading the next tile before storing the current one:
// 4.9-5.5).
// ---------------------------------------------------------------------------
constexpr uint32_t kTransposeWaves = 8;
__global__ __launch_bounds__(64 * kTransposeWaves) void transpose_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows, uint32_t columns,
    uint32_t tiles_c) {
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  uint32_t tr, tc;
  tile_of_block(tiles_c, 7, &tr, &tc);
  const uint32_t block_r = tr * (64 * kTransposeWaves) + wave * 64;
  const uint32_t block_c = tc * 64;
  const uint64_t matrix = blockIdx.y;
  const uint32_t r0 = block_r + (lane % 8) * 8;
  const uint32_t c0 = block_c + (lane / 8) * 8;
  if (r0 >= rows || c0 >= columns) return;
  const uint16_t* s = src + matrix * rows * (uint64_t)columns;
  uint16_t* d = dst + matrix * rows * (uint64_t)columns;
  u32x4 in[8], out[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) in[j] = load16_nt(s + (uint64_t)(r0 + j) * columns + c0);
  transpose8x8_u16(in, out);
#pragma unroll
  for (int i = 0; i < 8; ++i) store16_nt(d + (uint64_t)(c0 + i) * rows + r0, out[i]);
}

__global__ __launch_bounds__(kThreads) void transpose_f16_scalar_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows, uint32_t columns,
    uint64_t total) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint64_t me = (uint64_t)rows * columns;
  const uint64_t matrix = idx / me;
  const uint64_t within = idx % me;  // index in the destination [columns][rows]
  const uint32_t c = (uint32_t)(within / rows);
  const uint32_t r = (uint32_t)(within % rows);
  dst[idx] = src[matrix * me + (uint64_t)r * columns + c];
}

// ---------------------------------------------------------------------------
// Row-major -> BlockMajor{row_block, column_block} without padding.  Inside a
// micro-panel the 16 rows of one column are contiguous, so an 8x8 register
// transpose turns 8 source rows into 8 destination runs of 8 rows.  A wave
// covers 16 rows x 256 columns: lane % 2 picks the row half, lane / 2 the
// 8-column chunk.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void block_major_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows, uint32_t columns,
    uint32_t row_block, uint32_t column_block, uint32_t tiles_c) {
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t r0 = (blockIdx.x / tiles_c) * 64 + wave * 16 + (lane % 2) * 8;
  const uint32_t c0 = (blockIdx.x % tiles_c) * 256 + (lane / 2) * 8;
  if (r0 >= rows || c0 >= columns) return;
  const uint64_t me = (uint64_t)rows * columns;
  const uint16_t* s = src + blockIdx.y * me;
  uint16_t* d = dst + blockIdx.y * me;
  u32x4 in[8], out[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) in[j] = load16(s + (uint64_t)(r0 + j) * columns + c0);
  transpose8x8_u16(in, out);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    store16(d + block_major_index(row_block, column_block, columns, r0, c0 + i), out[i]);
}

// Row-major -> BlockMajor{64, cb} with cb dividing 256, rows % 64 == 0 and
// columns % 256 == 0.  The destination of a 64 x 256 tile (tr, tc) is one
// contiguous run of 32 KiB starting at element tr * columns * 64 + tc * 16384
// (its 256 / cb column blocks are consecutive): the register-transposed 8x8
// blocks are placed in LDS at their offsets in that run, and the run is then
// written with whole-line streaming stores.  At most three workgroups share
// a CU (occupancy_lds; five by LDS: 5.96-5.99 TB/s, three 6.09, two 6.08-6.11).
// LDS slot of 16-byte chunk p of the staged run: XOR-swizzled so that the
// transposed 8x8 blocks a 16-lane group stores (8 column chunks x 2 row
// halves) hit distinct bank groups for column blocks 16 and 64 (unswizzled:
// 8-way conflicts), while the sequential read-back stays conflict-free.
__device__ __forceinline__ uint32_t stage_chunk(uint32_t p) {
  return p ^ ((((p >> 4) ^ (p >> 6)) & 7u) << 1);
}

constexpr uint32_t kBlockMajorStaticLds = 64 * 256 * 2;
__global__ __launch_bounds__(kThreads) void block_major64_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t columns,
    uint32_t column_block, uint32_t tiles_c) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[kBlockMajorStaticLds];
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const uint32_t rl = wave * 16 + (lane % 2) * 8;  // tile-local row of this lane's 8x8 block
  const uint32_t cl = (lane / 2) * 8;              // tile-local column
  const uint64_t me = (uint64_t)gridDim.x * 64 * 256;  // elements per matrix
  const uint16_t* s = src + blockIdx.y * me;
  uint16_t* d = dst + blockIdx.y * me;
  u32x4 in[8], out[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    in[j] = load16_nt(s + (uint64_t)(tr * 64 + rl + j) * columns + tc * 256 + cl);
  transpose8x8_u16(in, out);
  const uint32_t cb = column_block;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t c = cl + i;
    const uint32_t off = ((c / cb) * 4 + rl / 16) * 16 * cb + (c % cb) * 16 + rl % 16;
    *reinterpret_cast<u32x4*>(stage + stage_chunk(off / 8) * 16) = out[i];
  }
  __syncthreads();
  uint16_t* run = d + (uint64_t)tr * columns * 64 + (uint64_t)tc * 16384;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t v = k * kThreads + threadIdx.x;
    store16_nt(run + v * 8, *reinterpret_cast<const u32x4*>(stage + stage_chunk(v) * 16));
  }
}

// ---------------------------------------------------------------------------
// General rearrange / unpack: one thread per destination element, gathering
// from the source through the inverse (or forward) storage map, zero-filling
// padding.  Used for padded or unaligned shapes and the AMP orders.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void rearrange_f16_general_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t target_order,
    uint32_t row_block, uint32_t column_block, uint32_t matrices, uint32_t logical_rows,
    uint32_t physical_rows, uint32_t logical_columns, uint32_t physical_columns, uint64_t total) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint64_t me = (uint64_t)physical_rows * physical_columns;
  uint32_t matrix, row, column;
  if (target_order == kOrderAmpLeft) {
    // Outer matrices fold into the row axis (storage.rs:250-266).
    uint32_t flat_row;
    amp_left_coordinates(matrices * physical_rows, idx, &flat_row, &column);
    matrix = flat_row / physical_rows;
    row = flat_row % physical_rows;
  } else {
    matrix = (uint32_t)(idx / me);
    const uint64_t within = idx % me;
    if (target_order == kOrderAmpTransposedRight)
      amp_transposed_right_coordinates(physical_rows, physical_columns, within, &row, &column);
    else
      block_major_coordinates(row_block, column_block, physical_columns, within, &row, &column);
  }
  uint16_t v = 0;
  if (row < logical_rows && column < logical_columns)
    v = src[((uint64_t)matrix * logical_rows + row) * logical_columns + column];
  dst[idx] = v;
}

__global__ __launch_bounds__(kThreads) void unpack_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t source_order,
    uint32_t logical_rows, uint32_t physical_rows, uint32_t logical_columns,
    uint32_t physical_columns, uint64_t total) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint64_t me = (uint64_t)physical_rows * physical_columns;
  const uint64_t matrix = idx / me;
  const uint64_t within = idx % me;
  const uint32_t row = (uint32_t)(within / physical_columns);
  const uint32_t column = (uint32_t)(within % physical_columns);
  uint16_t v = 0;
  if (row < logical_rows && column < logical_columns) {
    const uint64_t physical =
        source_order == kUnpackAmpOutput
            ? amp_output_index(physical_rows, row, column)
            : amp_transposed_left_index(physical_rows, physical_columns, row, column);
    v = src[matrix * me + physical];
  }
  dst[idx] = v;
}

// ---------------------------------------------------------------------------
// AMP orders, unpadded and 16-byte aligned: 16-byte chunks instead of
// elements.  AMP-Left and AMP-TransposedRight keep every run of 8 columns
// (8-aligned) contiguous (panels of 16 columns, 16 x 16 blocks stored row by
// row), so a chunk of a row-major row is a chunk of the stored tensor.  A
// workgroup takes a tile of kAmpTileRows rows x 64 columns: each row-major
// row of the tile is one 128-byte line, and the stored side is 4 panels of
// kAmpTileRows rows x 32 bytes (AMP-Left) or runs of 4 blocks of 512 bytes
// (TransposedRight), so both sides are read and written in runs of 256
// bytes or more per wave instruction.  Each thread loads its 8 chunks before
// it stores any (64 x 64 tiles, 2 chunks per thread: 5.0 / 5.8 TB/s).
// ToRowMajor runs the same map the other way (stored -> row-major).
// AMP-Left folds matrices into the rows (storage.rs:250-266), so `rows` is
// all matrices' rows and blockIdx.y is 0; TransposedRight is per matrix.
// ---------------------------------------------------------------------------
template <uint32_t Order, bool ToRowMajor, uint32_t TileRows, uint32_t TileCols>
__global__ __launch_bounds__(kThreads) void amp_tile_f16_kernel(uint16_t* __restrict__ dst,
                                                                const uint16_t* __restrict__ src,
                                                                uint32_t rows, uint32_t columns,
                                                                uint32_t tiles_c) {
  constexpr uint32_t kRowChunks = TileCols / 8;
  constexpr uint32_t kPer = TileRows * kRowChunks / kThreads;  // chunks per thread, all in flight
  static_assert(kPer >= 1 && TileRows * kRowChunks % kThreads == 0, "whole chunks per thread");
  uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  // AMP-Left: XCD-regrouped diagonal order, as the transpose (its stored
  // side is a transpose of 32-byte pieces; plain order 5.0 TB/s, 5.35 so).
  if (Order == kOrderAmpLeft) tile_of_block(tiles_c, 7, &tr, &tc);
  const uint64_t me = (uint64_t)rows * columns;
  src += blockIdx.y * me;
  dst += blockIdx.y * me;
  u32x4 v[kPer];
  uint64_t to[kPer];
  bool ok[kPer];
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i) {
    const uint32_t k = threadIdx.x + kThreads * i;
    const uint32_t r = tr * TileRows + k / kRowChunks, c = tc * TileCols + (k % kRowChunks) * 8;
    ok[i] = r < rows && c < columns;
    const uint64_t row_major = (uint64_t)r * columns + c;
    const uint64_t stored = Order == kOrderAmpLeft
                                ? amp_left_index(rows, r, c)
                                : amp_transposed_right_index(rows, columns, r, c);
    to[i] = ToRowMajor ? row_major : stored;
    if (ok[i]) v[i] = load16_nt(src + (ToRowMajor ? stored : row_major));
  }
#pragma unroll
  for (uint32_t i = 0; i < kPer; ++i)
    if (ok[i]) store16_nt(dst + to[i], v[i]);
}

// Unpack AMP-Output (pair-permuted 16-column micros, storage.rs:329-340),
// unpadded and aligned.  Logical pair p of a micro sits at physical pair
// (p % 4) * 2 + p / 4, so each 16-byte half of the row-major micro takes two
// words from each stored half.  Two adjacent lanes take one micro, one
// stored half each, and swap two words (DPP within the lane pair); then
// eight lanes write one whole 128-byte row line (64 columns), and a wave
// instruction writes 8 whole lines and reads 4 runs of 256 bytes (8 rows of
// each of the tile's 4 panels).  A workgroup takes 256 rows x 64 columns,
// 8 loads in flight per thread.
__global__ __launch_bounds__(kThreads) void unpack_amp_output_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows,
    uint32_t columns, uint32_t tiles_c) {
  constexpr uint32_t kPasses = kAmpTileRows / 32;
  const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const uint32_t half = threadIdx.x % 2, micro = threadIdx.x / 2 % 4;
  const uint32_t c = tc * 64 + micro * kMicro;
  const uint64_t me = (uint64_t)rows * columns;
  const uint16_t* s = src + blockIdx.y * me;
  uint16_t* d = dst + blockIdx.y * me;
  u32x4 v[kPasses];
#pragma unroll
  for (uint32_t i = 0; i < kPasses; ++i) {
    const uint32_t r = tr * kAmpTileRows + 32 * i + threadIdx.x / 8;
    if (r < rows && c < columns) v[i] = load16_nt(s + amp_output_index(rows, r, c) + half * 8);
  }
#pragma unroll
  for (uint32_t i = 0; i < kPasses; ++i) {
    const uint32_t r = tr * kAmpTileRows + 32 * i + threadIdx.x / 8;
    // Half 0 holds logical pairs 0, 4, 1, 5 and keeps 0, 1 (words 0, 2);
    // half 1 holds 2, 6, 3, 7 and keeps 6, 7 (words 1, 3).  Each sends the
    // other two words to its partner (quad_perm [1, 0, 3, 2]).
    const uint32_t x0 = half == 0 ? v[i][1] : v[i][0];
    const uint32_t x1 = half == 0 ? v[i][3] : v[i][2];
    const uint32_t y0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x0, 0xB1, 0xF, 0xF, true);
    const uint32_t y1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x1, 0xB1, 0xF, 0xF, true);
    const u32x4 out = half == 0 ? u32x4{v[i][0], v[i][2], y0, y1} : u32x4{y0, y1, v[i][1], v[i][3]};
    if (r < rows && c < columns) store16_nt(d + (uint64_t)r * columns + c + half * 8, out);
  }
}

// Unpack AMP-TransposedLeft (AMP-Left of the transpose, storage.rs:326-328),
// unpadded and aligned: the 16 rows of panel q are stored [columns][16], a
// transposed strip.  A thread loads 8 columns x 8 rows of it (one half of
// each column's 16 rows), transposes the 8 x 8 block in registers and writes
// 8 row segments of 16 bytes; lanes pair up on the two halves, so a wave
// reads 8 KiB of one strip and writes 512-byte runs of 16 rows.  Each load
// instruction takes a quarter of every 128-byte line it touches and the next
// three take the rest, so the loads are ordinary (cached): non-temporal ones
// let L2 drop the lines in between (1.49x the algorithmic reads, 4.3 against
// 5.7 TB/s).
__global__ __launch_bounds__(kThreads) void unpack_amp_transposed_left_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows,
    uint32_t columns, uint32_t col_groups) {
  const uint32_t panel = blockIdx.x / col_groups, group = blockIdx.x % col_groups;
  const uint32_t half = threadIdx.x % 2;
  const uint32_t c0 = (group * (kThreads / 2) + threadIdx.x / 2) * 8;
  if (c0 >= columns) return;
  const uint64_t me = (uint64_t)rows * columns;
  const uint16_t* s = src + blockIdx.y * me + (uint64_t)panel * columns * kMicro + half * 8;
  uint16_t* d = dst + blockIdx.y * me + (uint64_t)(panel * kMicro + half * 8) * columns + c0;
  u32x4 in[8], out[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) in[i] = load16(s + (uint64_t)(c0 + i) * kMicro);
  transpose8x8_u16(in, out);
#pragma unroll
  for (int j = 0; j < 8; ++j) store16_nt(d + (uint64_t)j * columns, out[j]);
}

// ---------------------------------------------------------------------------
// Row sums of a row-major [rows, columns] fp16 matrix, fp32 accumulation.
// One block per row; 16-byte loads; wave shuffles then LDS across waves.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sum8_f16(u32x4 v) {
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = v[w];
    s += (float)__builtin_bit_cast(half_t, (uint16_t)(x & 0xffffu));
    s += (float)__builtin_bit_cast(half_t, (uint16_t)(x >> 16));
  }
  return s;
}

__device__ __forceinline__ float block_sum(float v, float* shared) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) shared[wave] = v;
  __syncthreads();
  float total = 0.0f;
  if (threadIdx.x == 0)
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) total += shared[w];
  return total;
}

__global__ __launch_bounds__(kThreads) void reduce_rows_f16_kernel(
    float* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t columns) {
  __shared__ float partial[kThreads / kWave];
  const uint16_t* row = src + (uint64_t)blockIdx.x * columns;
  float acc = 0.0f;
  const uint32_t vectors = columns / 8;
  uint32_t v = threadIdx.x;
  // Four loads in flight per thread.
  for (; v + 3 * kThreads < vectors; v += 4 * kThreads) {
    u32x4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = load16_nt(row + (v + u * kThreads) * 8);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += sum8_f16(x[u]);
  }
  for (; v < vectors; v += kThreads) acc += sum8_f16(load16_nt(row + v * 8));
  for (uint32_t c = vectors * 8 + threadIdx.x; c < columns; c += kThreads)
    acc += (float)__builtin_bit_cast(half_t, row[c]);
  const float total = block_sum(acc, partial);
  if (threadIdx.x == 0) dst[blockIdx.x] = total;
}

// Unaligned rows (columns not a multiple of 8): scalar loads.
__global__ __launch_bounds__(kThreads) void reduce_rows_f16_scalar_kernel(
    float* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t columns) {
  __shared__ float partial[kThreads / kWave];
  const uint16_t* row = src + (uint64_t)blockIdx.x * columns;
  float acc = 0.0f;
  for (uint32_t c = threadIdx.x; c < columns; c += kThreads)
    acc += (float)__builtin_bit_cast(half_t, row[c]);
  const float total = block_sum(acc, partial);
  if (threadIdx.x == 0) dst[blockIdx.x] = total;
}

// Row sums of a logical [rows, columns] matrix stored BlockMajor{rb, cb}.
// The 16 rows of one row group live in columns/cb panels of 16*cb elements
// (column-major inside a panel), panel stride rb/16 panels.  One 256-thread
// block per row group walks all of its panels with four 16-byte loads in
// flight per thread (measured on 8192^2: 5.6 TB/s, against 4.8 TB/s for
// 1024-thread blocks and 5.2 TB/s for four column splits summed by a second
// kernel); lane parity selects the row half, so each lane accumulates 8
// rows; waves combine through LDS.  One launch, no workspace.
constexpr uint32_t kReduceThreads = 256;
constexpr int kReduceDepth = 4;  // loads in flight per thread (8 measured 5.4 TB/s)

__global__ __launch_bounds__(kReduceThreads) void reduce_rows_block_major_kernel(
    float* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t columns,
    uint32_t row_block, uint32_t column_block) {
  __shared__ float partial[kReduceThreads / kWave][16];
  const uint32_t row0 = blockIdx.x * 16;
  const uint32_t row_groups = row_block / 16;
  const uint32_t column_blocks = columns / column_block;
  // First panel of this row group (column block 0).
  const uint64_t first_panel =
      (uint64_t)(row0 / row_block) * column_blocks * row_groups + (row0 % row_block) / 16;
  const uint32_t vectors_per_panel = column_block * 2;  // 16 rows x cb columns / 8
  const uint32_t total_vectors = column_blocks * vectors_per_panel;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  auto element_of = [&](uint32_t v) {
    const uint32_t panel_index = v / vectors_per_panel;
    const uint32_t within = v % vectors_per_panel;
    return (first_panel + (uint64_t)panel_index * row_groups) * 16 * column_block + within * 8;
  };
  auto add8 = [&](u32x4 x) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc[2 * w] += (float)__builtin_bit_cast(half_t, (uint16_t)(x[w] & 0xffffu));
      acc[2 * w + 1] += (float)__builtin_bit_cast(half_t, (uint16_t)(x[w] >> 16));
    }
  };
  // v % 2 == threadIdx.x % 2 for every v a thread visits (the stride is
  // even): each lane always sees the same row half.  kReduceDepth loads in
  // flight; each lane adds its vectors in increasing v whatever the depth.
  uint32_t v = threadIdx.x;
  for (; v + (kReduceDepth - 1) * kReduceThreads < total_vectors; v += kReduceDepth * kReduceThreads) {
    u32x4 x[kReduceDepth];
#pragma unroll
    for (int u = 0; u < kReduceDepth; ++u) x[u] = load16_nt(src + element_of(v + u * kReduceThreads));
#pragma unroll
    for (int u = 0; u < kReduceDepth; ++u) add8(x[u]);
  }
  for (; v < total_vectors; v += kReduceThreads) add8(load16_nt(src + element_of(v)));
  // Reduce over lanes of equal parity.
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t = acc[e];
#pragma unroll
    for (int offset = 32; offset >= 2; offset >>= 1) t += __shfl_xor(t, offset, kWave);
    acc[e] = t;
  }
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  if (lane < 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) partial[wave][lane * 8 + e] = acc[e];
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    float t = 0.0f;
    for (uint32_t w = 0; w < kReduceThreads / kWave; ++w) t += partial[w][threadIdx.x];
    dst[row0 + threadIdx.x] = t;
  }
}

// ---------------------------------------------------------------------------
// Reference ReductionSum: out = initial + remote[0] + ... + remote[P-1],
// each addition rounded to fp16 in order (device/reduce_add_f16.S:54-70).
// ---------------------------------------------------------------------------
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(kThreads) void reduce_sum_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ initial,
    const uint16_t* __restrict__ remote, uint32_t partials, uint32_t count) {
  const uint32_t vectors = count / 8;
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < vectors;
       v += gridDim.x * blockDim.x) {
    half8_t acc = __builtin_bit_cast(half8_t, load16(initial + (uint64_t)v * 8));
    for (uint32_t p = 0; p < partials; ++p)
      acc = acc + __builtin_bit_cast(half8_t, load16(remote + (uint64_t)p * count + (uint64_t)v * 8));
    store16(dst + (uint64_t)v * 8, __builtin_bit_cast(u32x4, acc));
  }
}

// ---------------------------------------------------------------------------
// tanh-approximate GELU (gelu_tanh, device_common.h) on fp16 pairs.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t gelu_pair(uint32_t bits) {
  const half2_t h = __builtin_bit_cast(half2_t, bits);
  half2_t r;
  r[0] = (half_t)gelu_tanh((float)h[0]);
  r[1] = (half_t)gelu_tanh((float)h[1]);
  return __builtin_bit_cast(uint32_t, r);
}

// Two 16-byte vectors per thread per iteration keep two loads in flight.
__global__ __launch_bounds__(kThreads) void gelu_f16_kernel(uint16_t* __restrict__ dst,
                                                            const uint16_t* __restrict__ src,
                                                            uint64_t count) {
  const uint64_t vectors = count / 8;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; v + stride < vectors; v += 2 * stride) {
    u32x4 x = load16_nt(src + v * 8), y = load16_nt(src + (v + stride) * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      x[w] = gelu_pair(x[w]);
      y[w] = gelu_pair(y[w]);
    }
    store16_nt(dst + v * 8, x);
    store16_nt(dst + (v + stride) * 8, y);
  }
  if (v < vectors) {
    u32x4 x = load16_nt(src + v * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) x[w] = gelu_pair(x[w]);
    store16_nt(dst + v * 8, x);
  }
  // Tail elements.
  const uint64_t tail = vectors * 8 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tail < count && tail < vectors * 8 + 8) {
    const half_t h = __builtin_bit_cast(half_t, src[tail]);
    dst[tail] = __builtin_bit_cast(uint16_t, (half_t)gelu_tanh((float)h));
  }
}

__global__ __launch_bounds__(kThreads) void gelu_f16_scalar_kernel(uint16_t* __restrict__ dst,
                                                                   const uint16_t* __restrict__ src,
                                                                   uint64_t count) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const half_t h = __builtin_bit_cast(half_t, src[i]);
    dst[i] = __builtin_bit_cast(uint16_t, (half_t)gelu_tanh((float)h));
  }
}

// ---------------------------------------------------------------------------
// Fill, casts, add, split_heads.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void fill_zero_kernel(uint8_t* __restrict__ dst,
                                                             uint64_t bytes) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t vectors = bytes / 16;
  for (uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; v < vectors; v += stride)
    store16_nt(dst + v * 16, u32x4{0, 0, 0, 0});
  const uint64_t tail = vectors * 16 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tail < bytes && tail < vectors * 16 + 16) dst[tail] = 0;
}

// Plain device copy: 16-byte vectors (both pointers 16-byte aligned), then
// the byte tail; `vectors` = 0 copies byte by byte.  Non-temporal loads and
// stores (whole lines per wave): 5.8 -> 6.3 TB/s on 256 MiB.
__global__ __launch_bounds__(kThreads) void copy_bytes_kernel(uint8_t* __restrict__ dst,
                                                              const uint8_t* __restrict__ src,
                                                              uint64_t vectors, uint64_t bytes) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t first = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (uint64_t v = first; v < vectors; v += stride) store16_nt(dst + v * 16, load16_nt(src + v * 16));
  for (uint64_t b = vectors * 16 + first; b < bytes; b += stride) dst[b] = src[b];
}

__global__ __launch_bounds__(kThreads) void cast_f32_f16_kernel(uint16_t* __restrict__ dst,
                                                                const float* __restrict__ src,
                                                                uint64_t count) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
    dst[i] = __builtin_bit_cast(uint16_t, (half_t)src[i]);
}

__global__ __launch_bounds__(kThreads) void cast_f16_f32_kernel(float* __restrict__ dst,
                                                                const uint16_t* __restrict__ src,
                                                                uint64_t count) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
    dst[i] = (float)__builtin_bit_cast(half_t, src[i]);
}

struct AddShape {
  int rank;
  uint32_t shape[6];
  uint64_t ls[6];
  uint64_t rs[6];
};

template <typename T>
__global__ __launch_bounds__(kThreads) void add_kernel(T* __restrict__ dst,
                                                       const T* __restrict__ left,
                                                       const T* __restrict__ right, AddShape s,
                                                       uint64_t total) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint64_t rem = i, lo = 0, ro = 0;
    for (int axis = s.rank - 1; axis >= 0; --axis) {
      const uint64_t c = rem % s.shape[axis];
      rem /= s.shape[axis];
      lo += c * s.ls[axis];
      ro += c * s.rs[axis];
    }
    if constexpr (sizeof(T) == 2) {
      const float v = (float)__builtin_bit_cast(half_t, left[lo]) +
                      (float)__builtin_bit_cast(half_t, right[ro]);
      dst[i] = __builtin_bit_cast(uint16_t, (half_t)v);
    } else {
      dst[i] = left[lo] + right[ro];
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void split_heads_kernel(
    T* __restrict__ dst, const T* __restrict__ src, uint32_t rows, uint32_t heads,
    uint32_t channels, uint64_t total) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    // i indexes the destination [batch*heads, rows, channels].
    const uint32_t c = (uint32_t)(i % channels);
    uint64_t rem = i / channels;
    const uint32_t r = (uint32_t)(rem % rows);
    rem /= rows;
    const uint32_t h = (uint32_t)(rem % heads);
    const uint64_t b = rem / heads;
    const uint64_t width = (uint64_t)heads * channels;
    dst[i] = src[(b * rows + r) * width + (uint64_t)h * channels + c];
  }
}

// Any stored order -> row-major [matrices][rows][columns], one thread per
// destination element (forward storage maps, storage.rs:301-426).
__global__ __launch_bounds__(kThreads) void to_row_major_f16_general_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t source_order,
    uint32_t row_block, uint32_t column_block, uint32_t matrices, uint32_t rows,
    uint32_t columns, uint64_t total) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint64_t me = (uint64_t)rows * columns;
  const uint32_t matrix = (uint32_t)(idx / me);
  const uint64_t within = idx % me;
  const uint32_t row = (uint32_t)(within / columns), column = (uint32_t)(within % columns);
  uint64_t physical;
  if (source_order == kOrderAmpLeft)
    physical = amp_left_index(matrices * rows, matrix * rows + row, column);
  else if (source_order == kOrderAmpTransposedRight)
    physical = matrix * me + amp_transposed_right_index(rows, columns, row, column);
  else
    physical = matrix * me + block_major_index(row_block, column_block, columns, row, column);
  dst[idx] = src[physical];
}

// Block-major -> row-major, the inverse of block_major_f16_kernel: 8 runs of
// 8 rows are read, transposed in registers and written as 8 row segments.
// Tiles go in plain dispatch order, so adjacent 512-byte segments of the same
// destination rows are written by different XCDs at the same time (8192^2,
// 64 x 64 blocks: 5.05-5.16 TB/s with the transpose's XCD-regrouped diagonal
// order, 5.37-5.50 plain).
__global__ __launch_bounds__(kThreads) void block_major_to_row_major_f16_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows, uint32_t columns,
    uint32_t row_block, uint32_t column_block, uint32_t tiles_c) {
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const uint32_t r0 = tr * 64 + wave * 16 + (lane % 2) * 8;
  const uint32_t c0 = tc * 256 + (lane / 2) * 8;
  if (r0 >= rows || c0 >= columns) return;
  const uint64_t me = (uint64_t)rows * columns;
  const uint16_t* s = src + blockIdx.y * me;
  uint16_t* d = dst + blockIdx.y * me;
  u32x4 in[8], out[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    in[i] = load16(s + block_major_index(row_block, column_block, columns, r0, c0 + i));
  transpose8x8_u16(in, out);
#pragma unroll
  for (int j = 0; j < 8; ++j) store16_nt(d + (uint64_t)(r0 + j) * columns + c0, out[j]);
}

// Unshard: host bytes of a declared input format (the shards of a tiled
// tensor in logical tile order, each stored in an element order with zero
// padding; package.rs:2101-2137, storage.rs:201-285) -> the row-major
// logical tensor.  Workgroup row y handles table shard y; its threads walk
// the shard's logical region in row-major order (so each thread's writes go
// to consecutive destination elements of a row) and read each element at its
// physical index inside the shard.  Element orders: IPUS_ORDER_* codes.
// Table: kShardHeaderWords words (dims[8], reserved[8]), then per shard
// 26 words: file element offset lo, hi, start[8], logical width[8],
// physical width[8].
constexpr uint32_t kUnshardHeader = 16, kUnshardShard = 26, kUnshardMaxRank = 8;

__device__ __forceinline__ uint64_t shard_physical_index(uint32_t order, uint32_t rank,
                                                         const uint32_t* c, const uint32_t* pw,
                                                         uint32_t row_block,
                                                         uint32_t column_block) {
  if (order == 3) {  // row-major
    uint64_t p = 0;
    for (uint32_t a = 0; a < rank; ++a) p = p * pw[a] + c[a];
    return p;
  }
  uint64_t outer = 0, outer_count = 1;
  for (uint32_t a = 0; a + 2 < rank; ++a) {
    outer = outer * pw[a] + c[a];
    outer_count *= pw[a];
  }
  const uint32_t R = pw[rank - 2], C = pw[rank - 1], r = c[rank - 2], col = c[rank - 1];
  const uint64_t matrix = outer * (uint64_t)R * C;
  switch (order) {
    case 0:  // AMP-Left: outer axes fold into the rows
      return amp_left_index((uint32_t)(outer_count * R), (uint32_t)(outer * R + r), col);
    case 4:  // AMP-Output
      return amp_output_index((uint32_t)(outer_count * R), (uint32_t)(outer * R + r), col);
    case 1:  // AMP-TransposedRight
      return matrix + amp_transposed_right_index(R, C, r, col);
    case 5:  // AMP-TransposedLeft
      return matrix + amp_left_index(C, col, r);
    case 6:  // AMP-TransposedOutput
      return matrix + amp_output_index(C, col, r);
    case 2:  // block-major Matrix
      return matrix + block_major_index(row_block, column_block, C, r, col);
    default:  // 7: block-major TransposedMatrix
      return matrix + block_major_index(row_block, column_block, R, col, r);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void unshard_kernel(T* __restrict__ dst,
                                                           const T* __restrict__ src,
                                                           const uint32_t* __restrict__ table,
                                                           uint32_t rank, uint32_t order,
                                                           uint32_t row_block,
                                                           uint32_t column_block) {
  const uint32_t* sh = table + kUnshardHeader + (uint64_t)blockIdx.y * kUnshardShard;
  const uint64_t offset = (uint64_t)sh[0] | ((uint64_t)sh[1] << 32);
  uint32_t dims[kUnshardMaxRank], start[kUnshardMaxRank], lw[kUnshardMaxRank],
      pw[kUnshardMaxRank], c[kUnshardMaxRank];
  uint64_t n = 1;
  for (uint32_t a = 0; a < rank; ++a) {
    dims[a] = table[a];
    start[a] = sh[2 + a];
    lw[a] = sh[2 + kUnshardMaxRank + a];
    pw[a] = sh[2 + 2 * kUnshardMaxRank + a];
    n *= lw[a];
  }
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t rem = i;
    for (int a = (int)rank - 1; a >= 0; --a) {
      c[a] = (uint32_t)(rem % lw[a]);
      rem /= lw[a];
    }
    uint64_t d = 0;
    for (uint32_t a = 0; a < rank; ++a) d = d * dims[a] + start[a] + c[a];
    dst[d] = src[offset + shard_physical_index(order, rank, c, pw, row_block, column_block)];
  }
}

// Grid for a grid-stride kernel: one work item per thread up to 2^24
// workgroups.  A one-shot grid keeps every wave's loads independent (a
// 256 MiB copy: 5.7 TB/s with 2,048 workgroups looping, 6.5 one-shot).
inline uint32_t grid_for(uint64_t work_items, uint32_t cap = 1u << 24) {
  uint64_t g = (work_items + kThreads - 1) / kThreads;
  if (g == 0) g = 1;
  return (uint32_t)(g < cap ? g : cap);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

int launch_transpose_f16(hipStream_t stream, void* dst, const void* src, uint32_t matrices,
                         uint32_t rows, uint32_t columns) {
  if (matrices == 0 || rows == 0 || columns == 0) return 0;
  if (rows % 8 == 0 && columns % 8 == 0 && aligned16(dst) && aligned16(src) && matrices <= 65535) {
    const uint32_t tiles_r = ceil_div(rows, 64 * kTransposeWaves), tiles_c = ceil_div(columns, 64);
    hipLaunchKernelGGL(transpose_f16_kernel, dim3(tiles_r * tiles_c, matrices),
                       dim3(64 * kTransposeWaves), occupancy_lds(1, 0), stream, (uint16_t*)dst,
                       (const uint16_t*)src, rows, columns, tiles_c);
  } else {
    const uint64_t total = (uint64_t)matrices * rows * columns;
    hipLaunchKernelGGL(transpose_f16_scalar_kernel, dim3(ceil_div(total, kThreads)), dim3(kThreads),
                       0, stream, (uint16_t*)dst, (const uint16_t*)src, rows, columns, total);
  }
  return hip_status(hipGetLastError());
}

// The chunked AMP-Left / AMP-TransposedRight kernels for an unpadded,
// aligned tensor (columns a multiple of 16, and rows too for
// TransposedRight, as the orders require); false when the grid does not fit.
template <bool ToRowMajor>
bool launch_amp_tile(hipStream_t stream, void* dst, const void* src, uint32_t order,
                     uint32_t matrices, uint32_t rows, uint32_t columns) {
  if (order == kOrderAmpLeft) {
    // Row-major -> AMP-Left: 96 x 64 tiles at five workgroups per CU
    // (8192^2: 5.34-5.37 -> 5.60-5.62 TB/s against 64 x 64 tiles at the
    // default occupancy; 128 x 64 at four or five per CU 5.51-5.57, 96 x 64
    // at four or six 5.42-5.55).  The reverse keeps 64 x 64.
    constexpr uint32_t kRows = ToRowMajor ? 64 : 96;
    const uint32_t tiles_c = ceil_div(columns, 64);
    const uint64_t flat = (uint64_t)matrices * rows;
    const uint64_t tiles = ceil_div(flat, kRows) * (uint64_t)tiles_c;
    if (flat > 0xffffffffull || tiles > 0x7fffffffull) return false;
    hipLaunchKernelGGL((amp_tile_f16_kernel<kOrderAmpLeft, ToRowMajor, kRows, 64>),
                       dim3((uint32_t)tiles), dim3(kThreads), ToRowMajor ? 0 : occupancy_lds(5, 0),
                       stream, (uint16_t*)dst, (const uint16_t*)src, (uint32_t)flat, columns,
                       tiles_c);
    return true;
  }
  const uint32_t tiles_c = ceil_div(columns, 64);
  const uint64_t tiles = (uint64_t)ceil_div(rows, 32) * tiles_c;
  if (tiles > 0x7fffffffull || matrices > 65535) return false;
  hipLaunchKernelGGL((amp_tile_f16_kernel<kOrderAmpTransposedRight, ToRowMajor, 32, 64>),
                     dim3((uint32_t)tiles, matrices), dim3(kThreads), 0, stream, (uint16_t*)dst,
                     (const uint16_t*)src, rows, columns, tiles_c);
  return true;
}

int launch_rearrange_f16(hipStream_t stream, void* dst, const void* src, uint32_t target_order,
                         uint32_t row_block, uint32_t column_block, uint32_t matrices,
                         uint32_t logical_rows, uint32_t physical_rows, uint32_t logical_columns,
                         uint32_t physical_columns) {
  if (target_order > kOrderBlockMajor) return IPUS_ERROR_UNAVAILABLE;
  if (logical_rows > physical_rows || logical_columns > physical_columns)
    return IPUS_ERROR_INVALID_ARGUMENT;
  // Storage constraints of each order (storage.rs:314-425).
  if (target_order == kOrderAmpLeft && physical_columns % kMicro != 0)
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (target_order == kOrderAmpTransposedRight &&
      (physical_rows % kMicro != 0 || physical_columns % kMicro != 0))
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (target_order == kOrderBlockMajor &&
      (row_block == 0 || column_block == 0 || row_block % kMicro != 0 ||
       physical_rows % row_block != 0 || physical_columns % column_block != 0))
    return IPUS_ERROR_INVALID_ARGUMENT;
  const uint64_t total = (uint64_t)matrices * physical_rows * physical_columns;
  if (total == 0) return 0;
  const bool fast_block_major = target_order == kOrderBlockMajor &&
                                logical_rows == physical_rows &&
                                logical_columns == physical_columns && column_block % 8 == 0 &&
                                aligned16(dst) && aligned16(src) && matrices <= 65535;
  if (fast_block_major && row_block == 64 && 256 % column_block == 0 && physical_rows % 64 == 0 &&
      physical_columns % 256 == 0) {
    const uint32_t tiles_r = physical_rows / 64, tiles_c = physical_columns / 256;
    hipLaunchKernelGGL(block_major64_f16_kernel, dim3(tiles_r * tiles_c, matrices), dim3(kThreads),
                       occupancy_lds(3, kBlockMajorStaticLds), stream, (uint16_t*)dst, (const uint16_t*)src, physical_columns,
                       column_block, tiles_c);
  } else if (fast_block_major) {
    const uint32_t tiles_r = ceil_div(physical_rows, 64), tiles_c = ceil_div(physical_columns, 256);
    hipLaunchKernelGGL(block_major_f16_kernel, dim3(tiles_r * tiles_c, matrices), dim3(kThreads), 0,
                       stream, (uint16_t*)dst, (const uint16_t*)src, physical_rows,
                       physical_columns, row_block, column_block, tiles_c);
  } else if (target_order != kOrderBlockMajor && logical_rows == physical_rows &&
             logical_columns == physical_columns && aligned16(dst) && aligned16(src) &&
             launch_amp_tile<false>(stream, dst, src, target_order, matrices, physical_rows,
                                    physical_columns)) {
    // launched by launch_amp_tile
  } else {
    hipLaunchKernelGGL(rearrange_f16_general_kernel, dim3(ceil_div(total, kThreads)),
                       dim3(kThreads), 0, stream, (uint16_t*)dst, (const uint16_t*)src,
                       target_order, row_block, column_block, matrices, logical_rows,
                       physical_rows, logical_columns, physical_columns, total);
  }
  return hip_status(hipGetLastError());
}

int launch_unpack_f16(hipStream_t stream, void* dst, const void* src, uint32_t source_order,
                      uint32_t matrices, uint32_t logical_rows, uint32_t physical_rows,
                      uint32_t logical_columns, uint32_t physical_columns) {
  if (source_order > kUnpackAmpTransposedLeft) return IPUS_ERROR_UNAVAILABLE;
  if (logical_rows > physical_rows || logical_columns > physical_columns)
    return IPUS_ERROR_INVALID_ARGUMENT;
  // device/unpack_amp_f16.cpp:24-27 static asserts.
  if (source_order == kUnpackAmpOutput && physical_columns % kMicro != 0)
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (source_order == kUnpackAmpTransposedLeft && physical_rows % kMicro != 0)
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (physical_columns % 2 != 0) return IPUS_ERROR_INVALID_ARGUMENT;
  const uint64_t total = (uint64_t)matrices * physical_rows * physical_columns;
  if (total == 0) return 0;
  const bool unpadded = logical_rows == physical_rows && logical_columns == physical_columns &&
                        aligned16(dst) && aligned16(src);
  const uint64_t out_tiles =
      (uint64_t)ceil_div(physical_rows, kAmpTileRows) * ceil_div(physical_columns, 64);
  if (unpadded && source_order == kUnpackAmpOutput && out_tiles <= 0x7fffffffull &&
      matrices <= 65535) {
    const uint32_t tiles_c = ceil_div(physical_columns, 64);
    // Six workgroups per CU (8192^2: 5.36-5.39 -> 5.53-5.56 TB/s; five
    // 5.46-5.49, seven 5.45-5.47, four with 64-row tiles 5.47).
    hipLaunchKernelGGL(unpack_amp_output_f16_kernel, dim3((uint32_t)out_tiles, matrices),
                       dim3(kThreads), occupancy_lds(6, 0), stream, (uint16_t*)dst, (const uint16_t*)src,
                       physical_rows, physical_columns, tiles_c);
  } else if (unpadded && source_order == kUnpackAmpTransposedLeft && physical_columns % 8 == 0 &&
             matrices <= 65535 &&
             (uint64_t)(physical_rows / kMicro) * ceil_div(physical_columns, 8 * (kThreads / 2)) <=
                 0x7fffffffull) {
    const uint32_t col_groups = ceil_div(physical_columns, 8 * (kThreads / 2));
    // Two workgroups per CU (8192^2: 5.71-5.72 -> 5.78-5.80 TB/s; one
    // 5.55-5.58, three 5.75-5.77).
    hipLaunchKernelGGL(unpack_amp_transposed_left_f16_kernel,
                       dim3(physical_rows / kMicro * col_groups, matrices), dim3(kThreads),
                       occupancy_lds(2, 0),
                       stream, (uint16_t*)dst, (const uint16_t*)src, physical_rows,
                       physical_columns, col_groups);
  } else {
    hipLaunchKernelGGL(unpack_f16_kernel, dim3(ceil_div(total, kThreads)), dim3(kThreads), 0,
                       stream, (uint16_t*)dst, (const uint16_t*)src, source_order, logical_rows,
                       physical_rows, logical_columns, physical_columns, total);
  }
  return hip_status(hipGetLastError());
}

int launch_reduce_rows_f16(hipStream_t stream, float* dst, const void* src, uint32_t source_order,
                           uint32_t row_block, uint32_t column_block, uint32_t rows,
                           uint32_t columns) {
  if (rows == 0) return 0;
  if (source_order == kOrderRowMajor) {
    if (columns % 8 == 0 && aligned16(src))
      hipLaunchKernelGGL(reduce_rows_f16_kernel, dim3(rows), dim3(kThreads), 0, stream, dst,
                         (const uint16_t*)src, columns);
    else
      hipLaunchKernelGGL(reduce_rows_f16_scalar_kernel, dim3(rows), dim3(kThreads), 0, stream, dst,
                         (const uint16_t*)src, columns);
    return hip_status(hipGetLastError());
  }
  if (source_order != kOrderBlockMajor) return IPUS_ERROR_UNAVAILABLE;
  if (row_block == 0 || column_block == 0 || row_block % kMicro != 0 || rows % row_block != 0 ||
      columns % column_block != 0 || column_block % 2 != 0 || !aligned16(src))
    return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(reduce_rows_block_major_kernel, dim3(rows / 16), dim3(kReduceThreads), 0,
                     stream, dst, (const uint16_t*)src, columns, row_block, column_block);
  return hip_status(hipGetLastError());
}

int launch_reduce_sum_f16(hipStream_t stream, void* dst, const void* initial, const void* remote,
                          uint32_t remote_partials, uint32_t count) {
  if (count % 8 != 0) return IPUS_ERROR_UNSUPPORTED_COUNT;
  if (!aligned16(dst) || !aligned16(initial) || !aligned16(remote))
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (count == 0) return 0;
  hipLaunchKernelGGL(reduce_sum_f16_kernel, dim3(grid_for(count / 8)), dim3(kThreads), 0, stream,
                     (uint16_t*)dst, (const uint16_t*)initial, (const uint16_t*)remote,
                     remote_partials, count);
  return hip_status(hipGetLastError());
}

int launch_gelu_f16(hipStream_t stream, void* dst, const void* src, uint64_t count) {
  if (count == 0) return 0;
  if (aligned16(dst) && aligned16(src))
    hipLaunchKernelGGL(gelu_f16_kernel, dim3(grid_for(count / 8 + 1)), dim3(kThreads), 0, stream,
                       (uint16_t*)dst, (const uint16_t*)src, count);
  else
    hipLaunchKernelGGL(gelu_f16_scalar_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream,
                       (uint16_t*)dst, (const uint16_t*)src, count);
  return hip_status(hipGetLastError());
}

int launch_copy(hipStream_t stream, void* dst, const void* src, uint64_t bytes) {
  if (bytes == 0) return 0;
  const uint64_t vectors = aligned16(dst) && aligned16(src) ? bytes / 16 : 0;
  hipLaunchKernelGGL(copy_bytes_kernel, dim3(grid_for(vectors ? vectors : bytes)), dim3(kThreads),
                     0, stream, (uint8_t*)dst, (const uint8_t*)src, vectors, bytes);
  return hip_status(hipGetLastError());
}

int launch_fill_zero(hipStream_t stream, void* dst, uint64_t bytes) {
  if (bytes == 0) return 0;
  if (!aligned16(dst)) return IPUS_ERROR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(bytes / 16 + 1)), dim3(kThreads), 0, stream,
                     (uint8_t*)dst, bytes);
  return hip_status(hipGetLastError());
}

int launch_cast_f32_to_f16(hipStream_t stream, void* dst, const void* src, uint64_t count) {
  if (count == 0) return 0;
  hipLaunchKernelGGL(cast_f32_f16_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream,
                     (uint16_t*)dst, (const float*)src, count);
  return hip_status(hipGetLastError());
}

int launch_cast_f16_to_f32(hipStream_t stream, void* dst, const void* src, uint64_t count) {
  if (count == 0) return 0;
  hipLaunchKernelGGL(cast_f16_f32_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream,
                     (float*)dst, (const uint16_t*)src, count);
  return hip_status(hipGetLastError());
}

int launch_add(hipStream_t stream, const AddArgs& a) {
  if (a.rank < 0 || a.rank > 6) return IPUS_ERROR_INVALID_ARGUMENT;
  AddShape s;
  s.rank = a.rank;
  uint64_t total = 1;
  for (int i = 0; i < a.rank; ++i) {
    s.shape[i] = a.shape[i];
    s.ls[i] = a.left_strides[i];
    s.rs[i] = a.right_strides[i];
    total *= a.shape[i];
  }
  if (total == 0) return 0;
  if (a.precision == 1)
    hipLaunchKernelGGL(add_kernel<uint16_t>, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                       (uint16_t*)a.out, (const uint16_t*)a.left, (const uint16_t*)a.right, s,
                       total);
  else if (a.precision == 2)
    hipLaunchKernelGGL(add_kernel<float>, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                       (float*)a.out, (const float*)a.left, (const float*)a.right, s, total);
  else
    return IPUS_ERROR_INVALID_ARGUMENT;
  return hip_status(hipGetLastError());
}

int launch_split_heads(hipStream_t stream, void* dst, const void* src, uint32_t batch,
                       uint32_t rows, uint32_t heads, uint32_t channels, uint32_t element_bytes) {
  const uint64_t total = (uint64_t)batch * rows * heads * channels;
  if (total == 0) return 0;
  if (element_bytes == 2)
    hipLaunchKernelGGL(split_heads_kernel<uint16_t>, dim3(grid_for(total)), dim3(kThreads), 0,
                       stream, (uint16_t*)dst, (const uint16_t*)src, rows, heads, channels, total);
  else if (element_bytes == 4)
    hipLaunchKernelGGL(split_heads_kernel<uint32_t>, dim3(grid_for(total)), dim3(kThreads), 0,
                       stream, (uint32_t*)dst, (const uint32_t*)src, rows, heads, channels, total);
  else
    return IPUS_ERROR_INVALID_ARGUMENT;
  return hip_status(hipGetLastError());
}

int launch_unshard(hipStream_t stream, void* dst, const void* src, const void* table,
                   uint32_t shards, uint32_t rank, uint32_t order, uint32_t row_block,
                   uint32_t column_block, uint32_t element_bytes, uint32_t max_shard_elements) {
  if (shards == 0 || max_shard_elements == 0) return 0;
  if (rank == 0 || rank > kUnshardMaxRank || order > 7 || shards > 65535 ||
      (element_bytes != 2 && element_bytes != 4) || (order != 3 && element_bytes != 2) ||
      ((order == 2 || order == 7) && (row_block == 0 || column_block == 0 || row_block % kMicro)))
    return IPUS_ERROR_INVALID_ARGUMENT;
  const dim3 grid(grid_for(max_shard_elements, 4096), shards);
  if (element_bytes == 2)
    hipLaunchKernelGGL(unshard_kernel<uint16_t>, grid, dim3(kThreads), 0, stream, (uint16_t*)dst,
                       (const uint16_t*)src, (const uint32_t*)table, rank, order, row_block,
                       column_block);
  else
    hipLaunchKernelGGL(unshard_kernel<uint32_t>, grid, dim3(kThreads), 0, stream, (uint32_t*)dst,
                       (const uint32_t*)src, (const uint32_t*)table, rank, order, row_block,
                       column_block);
  return hip_status(hipGetLastError());
}

int launch_to_row_major_f16(hipStream_t stream, void* dst, const void* src, uint32_t source_order,
                            uint32_t row_block, uint32_t column_block, uint32_t matrices,
                            uint32_t rows, uint32_t columns) {
  if (source_order > kOrderBlockMajor) return IPUS_ERROR_UNAVAILABLE;
  if (source_order == kOrderAmpLeft && columns % kMicro != 0) return IPUS_ERROR_INVALID_ARGUMENT;
  if (source_order == kOrderAmpTransposedRight && (rows % kMicro != 0 || columns % kMicro != 0))
    return IPUS_ERROR_INVALID_ARGUMENT;
  if (source_order == kOrderBlockMajor &&
      (row_block == 0 || column_block == 0 || row_block % kMicro != 0 || rows % row_block != 0 ||
       columns % column_block != 0))
    return IPUS_ERROR_INVALID_ARGUMENT;
  const uint64_t total = (uint64_t)matrices * rows * columns;
  if (total == 0) return 0;
  if (source_order == kOrderBlockMajor && column_block % 8 == 0 && aligned16(dst) &&
      aligned16(src) && matrices <= 65535) {
    const uint32_t tiles_r = ceil_div(rows, 64), tiles_c = ceil_div(columns, 256);
    hipLaunchKernelGGL(block_major_to_row_major_f16_kernel, dim3(tiles_r * tiles_c, matrices),
                       dim3(kThreads), 0, stream, (uint16_t*)dst, (const uint16_t*)src, rows,
                       columns, row_block, column_block, tiles_c);
  } else if (source_order != kOrderBlockMajor && aligned16(dst) && aligned16(src) &&
             launch_amp_tile<true>(stream, dst, src, source_order, matrices, rows, columns)) {
    // launched by launch_amp_tile
  } else {
    hipLaunchKernelGGL(to_row_major_f16_general_kernel, dim3(ceil_div(total, kThreads)),
                       dim3(kThreads), 0, stream, (uint16_t*)dst, (const uint16_t*)src,
                       source_order, row_block, column_block, matrices, rows, columns, total);
  }
  return hip_status(hipGetLastError());
}

}  // namespace ipus

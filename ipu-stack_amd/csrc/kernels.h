// Host-side launchers of the gfx950 kernels.  Each launcher validates the
// shape it needs, picks a grid, and enqueues on the given stream.  They return
// 0 or a negative ipus status (see include/ipus.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ipus {

struct GemmArgs {
  void* out;
  const void* left;
  const void* right;
  uint32_t batches;
  uint64_t left_batch_stride;   // elements; 0 broadcasts one matrix
  uint64_t right_batch_stride;  // elements; 0 broadcasts one matrix
  uint32_t rows, columns, inner;
  bool transpose_left, transpose_right;
  bool gelu = false;  // fp16 GEMM only: GELU of the fp16 result in the epilogue
  // fp16 GEMM only, exclusive with gelu: out = add_f16(addend, fp16 product)
  // with the addend element at batch * addend_batch_stride + row *
  // addend_row_stride + column (0 strides broadcast); out may be the addend.
  const void* addend = nullptr;
  uint64_t addend_batch_stride = 0;
  uint32_t addend_row_stride = 0;
};

// The addend of a split-K reduction (launch_reduce_splits_f16): the partials
// are [splits][batches][rows][columns].
struct SplitAddend {
  const void* addend;
  uint32_t rows, columns;
  uint64_t batch_stride;
  uint32_t row_stride;
};

struct AttentionArgs {
  void* out;
  const void* query;
  const void* key;
  const void* value;
  uint32_t streams, query_rows, key_rows, width, value_width;
  float scale;
  bool causal;
  bool output_f16;  // false: fp32 output (reference), true: fp16
  // Per operand (query, key, value): stream s is head s % h of matrix s / h
  // of a [streams / h, rows, h * width] tensor; 1 = contiguous streams.
  uint32_t heads[3] = {1, 1, 1};
};

// Dense products (k_gemm_f16.hip, k_gemm_f32.hip).
int launch_gemm_f16(hipStream_t stream, const GemmArgs& a);
// Split-K: fp32 partials float[splits][batches][M][N] into a.out (a.gelu must
// be false), then launch_reduce_splits_f16 to fp16.  gemm_f16_split_chunk
// gives the k range per split (a multiple of 64); the plan picks splits so
// that every split owns some k.
int gemm_f16_split_chunk(uint32_t inner, uint32_t splits);
int launch_gemm_f16_split(hipStream_t stream, const GemmArgs& a, uint32_t splits);
int launch_reduce_splits_f16(hipStream_t stream, void* dst, const void* parts, uint32_t splits,
                             uint64_t count, bool gelu, const SplitAddend* add = nullptr);
// Declared input format -> row-major (k_memory.hip): `table` is the shard
// table of tiling.h in device memory; one workgroup row per table shard,
// `max_shard_elements` sizes the grid.
int launch_unshard(hipStream_t stream, void* dst, const void* src, const void* table,
                   uint32_t shards, uint32_t rank, uint32_t order, uint32_t row_block,
                   uint32_t column_block, uint32_t element_bytes, uint32_t max_shard_elements);
// Split-K with the partials in the library's per-device scratch array
// (no allocation): split_scratch_init(device) looks up the device's copy
// once, with that device current; the launch then runs the split GEMM into
// it and the reduction into a.out (GELU when a.gelu).  Partials beyond
// IPUS_SPLIT_SCRATCH_BYTES return IPUS_ERROR_UNSUPPORTED_COUNT.
int split_scratch_init(int device);
int launch_gemm_f16_split_noalloc(hipStream_t stream, int device, const GemmArgs& a,
                                  uint32_t splits);
int launch_gemm_f32(hipStream_t stream, const GemmArgs& a);

// Fused online-softmax attention (k_attention.hip).
int launch_attention_f16(hipStream_t stream, const AttentionArgs& a);

// Bandwidth kernels (k_memory.hip).
int launch_transpose_f16(hipStream_t stream, void* dst, const void* src, uint32_t matrices,
                         uint32_t rows, uint32_t columns);
int launch_rearrange_f16(hipStream_t stream, void* dst, const void* src, uint32_t target_order,
                         uint32_t row_block, uint32_t column_block, uint32_t matrices,
                         uint32_t logical_rows, uint32_t physical_rows, uint32_t logical_columns,
                         uint32_t physical_columns);
int launch_unpack_f16(hipStream_t stream, void* dst, const void* src, uint32_t source_order,
                      uint32_t matrices, uint32_t logical_rows, uint32_t physical_rows,
                      uint32_t logical_columns, uint32_t physical_columns);
// Row sums with fp32 accumulation of a logical [rows, columns] fp16 matrix
// stored row-major (source_order = 3) or block-major (source_order = 2).
int launch_reduce_rows_f16(hipStream_t stream, float* dst, const void* src, uint32_t source_order,
                           uint32_t row_block, uint32_t column_block, uint32_t rows,
                           uint32_t columns);
int launch_reduce_sum_f16(hipStream_t stream, void* dst, const void* initial, const void* remote,
                          uint32_t remote_partials, uint32_t count);
int launch_gelu_f16(hipStream_t stream, void* dst, const void* src, uint64_t count);
int launch_fill_zero(hipStream_t stream, void* dst, uint64_t bytes);
int launch_copy(hipStream_t stream, void* dst, const void* src, uint64_t bytes);
int launch_cast_f32_to_f16(hipStream_t stream, void* dst, const void* src, uint64_t count);
int launch_cast_f16_to_f32(hipStream_t stream, void* dst, const void* src, uint64_t count);
// out = left + right with numpy broadcasting over up to 6 axes; strides are
// in elements, 0 on broadcast axes.  precision: 1 = f16, 2 = f32.
struct AddArgs {
  void* out;
  const void* left;
  const void* right;
  int rank;
  uint32_t shape[6];
  uint64_t left_strides[6];
  uint64_t right_strides[6];
  int precision;
};
int launch_add(hipStream_t stream, const AddArgs& a);
// Streams = batch * heads: [batch, rows, heads*ch] -> [batch*heads, rows, ch];
// element_bytes 2 or 4.
int launch_split_heads(hipStream_t stream, void* dst, const void* src, uint32_t batch,
                       uint32_t rows, uint32_t heads, uint32_t channels, uint32_t element_bytes);
// Roofline calibration (k_calibrate.hip): `out` receives two u64 (shader
// clock cycles, 100 MHz ticks of lane 0 of block 0) and a float sink of
// blocks * 256 values; `operands` holds operand_count fragments of 8 fp16.
uint64_t calibrate_output_bytes(uint32_t blocks);
// Plain 16-byte-vector copy with ordinary loads and stores (bytes % 16 == 0,
// both pointers 16-byte aligned): the HBM traffic counters' calibration.
int launch_calibrate_copy(hipStream_t stream, void* dst, const void* src, uint32_t bytes);
int launch_calibrate_mfma_f16(hipStream_t stream, void* out, const void* operands,
                              uint32_t operand_count, uint32_t iterations, uint32_t blocks,
                              bool form16 = false);
// Stored order (AmpLeft, AmpTransposedRight, BlockMajor) -> row-major.
int launch_to_row_major_f16(hipStream_t stream, void* dst, const void* src, uint32_t source_order,
                            uint32_t row_block, uint32_t column_block, uint32_t matrices,
                            uint32_t rows, uint32_t columns);

}  // namespace ipus

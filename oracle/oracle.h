/*
 * CPU oracle for the ipu-stack hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or as the timed CPU baseline.
 * The product library (ipu-stack_amd/) never links, loads or calls it.
 *
 * Every function restates the reference's semantics and cites the reference
 * file:line it follows (paths relative to the osmarks/ipu-stack root).
 * Return codes: 0 = ok, negative = invalid arguments (mirrors StorageError /
 * bail! in the reference).
 */
#ifndef IPUS_ORACLE_H
#define IPUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Precision codes, crates/ipu-codegen/src/operator.rs:14-21. */
enum { OR_F8 = 0, OR_F16 = 1, OR_F32 = 2 };

/* AmpOrder, crates/ipu-codegen/src/layout.rs:7-17. */
enum {
  OR_AMP_LEFT = 0,
  OR_AMP_TRANSPOSED_LEFT = 1,
  OR_AMP_TRANSPOSED_RIGHT = 2,
  OR_AMP_OUTPUT = 3,
  OR_AMP_TRANSPOSED_OUTPUT = 4
};

/* ---- binary16 <-> binary32 (half 2.7.1 semantics, main.rs:2040-2046) ---- */
uint16_t or_f32_to_f16(float value);
float or_f16_to_f32(uint16_t bits);
void or_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void or_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);
void or_quantize_f16_array(float *values, size_t n);

/* ---- storage index maps, crates/ipu-codegen/src/storage.rs ---- */
int64_t or_amp_matrix_index(int role, int precision, uint32_t rows,
                            uint32_t columns, uint32_t row, uint32_t column);
int or_amp_matrix_coordinates(int role, int precision, uint32_t rows,
                              uint32_t columns, uint32_t linear, uint32_t *row,
                              uint32_t *column);
int64_t or_right_matrix_index(int precision, uint32_t rows, uint32_t columns,
                              uint32_t row, uint32_t column);
int64_t or_block_major_matrix_index(int transposed, uint32_t row_block,
                                    uint32_t column_block, int precision,
                                    uint32_t rows, uint32_t columns,
                                    uint32_t row, uint32_t column);
int or_block_major_matrix_coordinates(int transposed, uint32_t row_block,
                                      uint32_t column_block, int precision,
                                      uint32_t rows, uint32_t columns,
                                      uint32_t linear, uint32_t *row,
                                      uint32_t *column);

/* ---- one shard of a tiled host binding, storage.rs:201-299
 * (physical_index) and package.rs:2101-2137 (shard bytes) ----
 * kind 0 row-major, 1 AMP (`variant` = AmpOrder role above), 2 block-major
 * (`variant` = 1 for TransposedMatrix).  The shard covers [start, logical_end)
 * of each of `rank` axes of a row-major logical tensor `dims`, stored with
 * physical widths physical_end - start; padding elements stay as the caller
 * left them (zero).  Returns 0, or < 0 when an index is invalid. */
int or_pack_shard(int kind, int variant, uint32_t row_block, uint32_t column_block,
                  int rank, const uint32_t *dims, const uint32_t *start,
                  const uint32_t *logical_end, const uint32_t *physical_end,
                  const uint16_t *logical, uint16_t *shard);

/* ---- rearrange / unpack kernels (device/rearrange_f16.cpp,
 *      device/unpack_amp_f16.cpp) on 16-bit payloads ---- */
int or_rearrange_row_major_f16(int target_order, uint32_t row_block,
                               uint32_t column_block, uint32_t matrices,
                               uint32_t logical_rows, uint32_t physical_rows,
                               uint32_t logical_columns,
                               uint32_t physical_columns, const uint16_t *src,
                               uint16_t *dst);
int or_unpack_to_row_major_f16(int source_order, uint32_t matrices,
                               uint32_t logical_rows, uint32_t physical_rows,
                               uint32_t logical_columns,
                               uint32_t physical_columns, const uint16_t *src,
                               uint16_t *dst);
void or_transpose_u16(uint32_t matrices, uint32_t rows, uint32_t columns,
                      const uint16_t *src, uint16_t *dst);

/* ---- arithmetic, crates/ipu-tests/src/diagnostic.rs ---- */
int or_gemm_f32(const float *left, const float *right, float *out,
                uint32_t batches, uint64_t left_batch_stride,
                uint64_t right_batch_stride, uint32_t rows, uint32_t columns,
                uint32_t inner, int transpose_left, int transpose_right,
                int threads);
int or_gemm_f16(const uint16_t *left, const uint16_t *right, uint16_t *out,
                uint32_t batches, uint64_t left_batch_stride,
                uint64_t right_batch_stride, uint32_t rows, uint32_t columns,
                uint32_t inner, int transpose_left, int transpose_right,
                int threads);
int or_gemm_f16_rows(const uint16_t *left, const uint16_t *right, float *out,
                     uint32_t rows, uint32_t columns, uint32_t inner,
                     const uint32_t *row_list, uint32_t row_count, int threads);
int or_attention(const float *query, const float *key, const float *value,
                 float *out, uint32_t streams, uint32_t query_rows,
                 uint32_t key_rows, uint32_t width, uint32_t value_width,
                 int causal, float scale, int use_scale,
                 const uint32_t *row_list, uint32_t row_count, int threads);
float or_gelu_reference(float value);
void or_gelu_f16(const uint16_t *src, uint16_t *dst, size_t n);
int or_add_f32(const float *left, const uint32_t *left_shape, int left_rank,
               const float *right, const uint32_t *right_shape, int right_rank,
               float *out, uint32_t *out_shape, int *out_rank);
int or_split_heads(const float *input, uint32_t batch, uint32_t rows,
                   uint32_t width, uint32_t heads, float *out);
void or_reduce_sum_f16(const uint16_t *initial, const uint16_t *remote,
                       uint32_t remote_partials, uint32_t count,
                       uint16_t *out);
void or_reduce_rows_f16(const uint16_t *src, uint32_t rows, uint32_t columns,
                        float *out, int threads);
int or_reduce_rows_block_major_f16(const uint16_t *src, uint32_t row_block,
                                   uint32_t column_block, uint32_t rows,
                                   uint32_t columns, float *out, int threads);

/* ---- synthetic inputs (same construction as bench/tests) ---- */
uint64_t or_splitmix64(uint64_t state);

#ifdef __cplusplus
}
#endif
#endif

// Physical element maps of the reference's storage orders, usable on the host
// and inside kernels.  These are the maps of
// crates/ipu-codegen/src/storage.rs:301-426 (logical -> physical) and
// storage.rs:656-782 (physical -> logical) for 16-bit elements (micro = 16).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define IPUS_HD __host__ __device__ __forceinline__
#else
#define IPUS_HD inline
#endif

namespace ipus {

// Target / source order codes.  The first three match the reference's
// rearrange codelet indices (crates/ipu-codegen/src/kernel.rs:113-119); the
// unpack sources match kernel.rs:91-96.
enum Order : uint32_t {
  kOrderAmpLeft = 0,
  kOrderAmpTransposedRight = 1,
  kOrderBlockMajor = 2,
  kOrderRowMajor = 3,
};
enum UnpackSource : uint32_t {
  kUnpackAmpOutput = 0,
  kUnpackAmpTransposedLeft = 1,
};

constexpr uint32_t kMicro = 16;  // AMP_COLUMN_MICRO and the f16 inner micro

// AMP-Left [rows, columns]: storage.rs:314-324.
IPUS_HD uint64_t amp_left_index(uint32_t rows, uint32_t row, uint32_t column) {
  return (uint64_t)(column / kMicro) * rows * kMicro + (uint64_t)row * kMicro + column % kMicro;
}
IPUS_HD void amp_left_coordinates(uint32_t rows, uint64_t linear, uint32_t* row, uint32_t* column) {
  const uint64_t panel_elements = (uint64_t)rows * kMicro;
  const uint64_t panel = linear / panel_elements;
  const uint64_t offset = linear % panel_elements;
  *row = (uint32_t)(offset / kMicro);
  *column = (uint32_t)(panel * kMicro + offset % kMicro);
}

// AMP-Output [rows, columns]: pair-permuted columns, storage.rs:329-340.
IPUS_HD uint64_t amp_output_index(uint32_t rows, uint32_t row, uint32_t column) {
  const uint32_t logical_pair = column % kMicro / 2;
  const uint32_t physical_pair = logical_pair % 4 * 2 + logical_pair / 4;
  const uint32_t physical_column = physical_pair * 2 + column % 2;
  return (uint64_t)(column / kMicro) * rows * kMicro + (uint64_t)row * kMicro + physical_column;
}

// right_matrix_index (storage.rs:347-370) for semantic [rows, columns].
IPUS_HD uint64_t right_matrix_index(uint32_t rows, uint32_t row, uint32_t column) {
  const uint64_t panel = (uint64_t)(column / kMicro) * (rows / kMicro) + row / kMicro;
  return panel * kMicro * kMicro + (uint64_t)(column % kMicro) * kMicro + row % kMicro;
}
IPUS_HD void right_matrix_coordinates(uint32_t rows, uint64_t linear, uint32_t* row,
                                      uint32_t* column) {
  const uint64_t panel = linear / (kMicro * kMicro);
  const uint32_t offset = (uint32_t)(linear % (kMicro * kMicro));
  const uint32_t inner_groups = rows / kMicro;
  const uint32_t column_group = (uint32_t)(panel / inner_groups);
  const uint32_t inner_group = (uint32_t)(panel % inner_groups);
  *row = inner_group * kMicro + offset % kMicro;
  *column = column_group * kMicro + offset / kMicro;
}

// AMP-TransposedRight, semantic [keys, channels] stored as the right operand
// [channels, keys] (storage.rs:325 via 242-249).
IPUS_HD uint64_t amp_transposed_right_index(uint32_t rows, uint32_t columns, uint32_t row,
                                            uint32_t column) {
  (void)rows;
  return right_matrix_index(columns, column, row);
}
IPUS_HD void amp_transposed_right_coordinates(uint32_t rows, uint32_t columns, uint64_t linear,
                                              uint32_t* row, uint32_t* column) {
  (void)rows;
  uint32_t a, b;
  right_matrix_coordinates(columns, linear, &a, &b);
  *column = a;
  *row = b;
}

// AMP-TransposedLeft = AMP-Left of the transposed matrix (storage.rs:326-328).
IPUS_HD uint64_t amp_transposed_left_index(uint32_t rows, uint32_t columns, uint32_t row,
                                           uint32_t column) {
  (void)rows;
  return amp_left_index(columns, column, row);
}

// Block-major Matrix{row_block, column_block}: storage.rs:403-425.
IPUS_HD uint64_t block_major_index(uint32_t row_block, uint32_t column_block, uint32_t columns,
                                   uint32_t row, uint32_t column) {
  const uint64_t row_groups = row_block / kMicro;
  const uint64_t panel = (uint64_t)(row / row_block) * (columns / column_block) * row_groups +
                         (uint64_t)(column / column_block) * row_groups +
                         (row % row_block) / kMicro;
  return panel * kMicro * column_block + (uint64_t)(column % column_block) * kMicro +
         row % kMicro;
}
IPUS_HD void block_major_coordinates(uint32_t row_block, uint32_t column_block, uint32_t columns,
                                     uint64_t linear, uint32_t* row, uint32_t* column) {
  const uint64_t panel_elements = (uint64_t)kMicro * column_block;
  const uint64_t panel = linear / panel_elements;
  const uint32_t offset = (uint32_t)(linear % panel_elements);
  const uint32_t row_groups = row_block / kMicro;
  const uint64_t panels_per_row_block = (uint64_t)(columns / column_block) * row_groups;
  const uint64_t row_block_index = panel / panels_per_row_block;
  const uint32_t within_block = (uint32_t)(panel % panels_per_row_block);
  const uint32_t column_group = within_block / row_groups;
  const uint32_t row_group = within_block % row_groups;
  *row = (uint32_t)(row_block_index * row_block) + row_group * kMicro + offset % kMicro;
  *column = column_group * column_block + offset / kMicro;
}

}  // namespace ipus

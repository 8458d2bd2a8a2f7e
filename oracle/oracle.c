/*
 * CPU oracle for the ipu-stack hot path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker (or the timed CPU baseline),
 * never as the product path.  The product library does not link or load it.
 *
 * It restates the reference's CPU evaluator
 * (crates/ipu-tests/src/diagnostic.rs:411-847), its fp16 conversion
 * (crates/ipu-tests/src/main.rs:2040-2046), its GELU reference
 * (main.rs:1985-1987), the storage index maps
 * (crates/ipu-codegen/src/storage.rs:301-426, 656-790) and the device kernel
 * semantics of device/rearrange_f16.cpp:72-153, device/unpack_amp_f16.cpp:40-82
 * and device/reduce_add_f16.S:54-70.
 *
 * Pinning (what each function is checked against) is listed in the tests:
 * tests/test_oracle.py.  The reference itself (Rust + Graphcore SDK) cannot be
 * built in this environment, so there is no oracle/_ref build.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Small parallel-for helper.                                                */
/* ------------------------------------------------------------------------- */
typedef void (*range_fn)(void *ctx, uint64_t begin, uint64_t end);
typedef struct {
  range_fn fn;
  void *ctx;
  uint64_t begin, end;
} range_job;

static void *range_thread(void *arg) {
  range_job *job = (range_job *)arg;
  job->fn(job->ctx, job->begin, job->end);
  return NULL;
}

static void parallel_for(uint64_t total, int threads, range_fn fn, void *ctx) {
  if (threads < 1) threads = 1;
  if ((uint64_t)threads > total) threads = (int)(total ? total : 1);
  if (threads == 1) {
    fn(ctx, 0, total);
    return;
  }
  pthread_t *ids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  range_job *jobs = (range_job *)malloc(sizeof(range_job) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].begin = total * (uint64_t)t / (uint64_t)threads;
    jobs[t].end = total * (uint64_t)(t + 1) / (uint64_t)threads;
    pthread_create(&ids[t], NULL, range_thread, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(ids[t], NULL);
  free(ids);
  free(jobs);
}

/* ------------------------------------------------------------------------- */
/* IEEE binary16, round to nearest even (the `half` crate's from_f32, used by */
/* f32_to_half at crates/ipu-tests/src/main.rs:2040-2042).                   */
/* ------------------------------------------------------------------------- */
uint16_t or_f32_to_f16(float value) {
  uint32_t x;
  memcpy(&x, &value, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exponent = (x >> 23) & 0xffu;
  uint32_t mantissa = x & 0x7fffffu;
  if (exponent == 0xffu) {
    if (mantissa == 0) return (uint16_t)(sign | 0x7c00u);
    /* NaN: keep the top mantissa bits and force a quiet NaN. */
    return (uint16_t)(sign | 0x7e00u | (mantissa >> 13));
  }
  const int32_t half_exponent = (int32_t)exponent - 127 + 15;
  if (half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  if (half_exponent <= 0) {
    /* Subnormal or zero result. */
    if (half_exponent < -10) return (uint16_t)sign;
    mantissa |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - half_exponent);
    uint32_t result = mantissa >> shift;
    const uint32_t remainder = mantissa & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (remainder > halfway || (remainder == halfway && (result & 1u)))
      result += 1u;
    return (uint16_t)(sign | result);
  }
  uint32_t result = ((uint32_t)half_exponent << 10) | (mantissa >> 13);
  const uint32_t remainder = mantissa & 0x1fffu;
  if (remainder > 0x1000u || (remainder == 0x1000u && (result & 1u)))
    result += 1u; /* may carry into the exponent, giving inf: correct */
  return (uint16_t)(sign | result);
}

float or_f16_to_f32(uint16_t bits) {
  const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
  uint32_t mantissa = (uint32_t)bits & 0x3ffu;
  uint32_t out;
  if (exponent == 0x1fu) {
    out = sign | 0x7f800000u | (mantissa << 13);
  } else if (exponent == 0) {
    if (mantissa == 0) {
      out = sign;
    } else {
      int e = -1;
      do {
        ++e;
        mantissa <<= 1;
      } while ((mantissa & 0x400u) == 0);
      out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mantissa & 0x3ffu) << 13);
    }
  } else {
    out = sign | ((exponent + 127 - 15) << 23) | (mantissa << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void or_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* diagnostic.rs:841-847 quantize(value, F16). */
void or_quantize_f16_array(float *values, size_t n) {
  for (size_t i = 0; i < n; ++i) values[i] = or_f16_to_f32(or_f32_to_f16(values[i]));
}

/* ------------------------------------------------------------------------- */
/* Storage index maps.                                                        */
/* ------------------------------------------------------------------------- */
#define AMP_COLUMN_MICRO 16u /* crates/ipu-codegen/src/layout.rs:36 */

/* storage.rs:784-790 */
static uint32_t amp_micro_dimension(int precision) {
  switch (precision) {
    case OR_F8: return 32u;
    case OR_F16: return 16u;
    default: return 8u;
  }
}

/* storage.rs:347-370 */
int64_t or_right_matrix_index(int precision, uint32_t rows, uint32_t columns,
                              uint32_t row, uint32_t column) {
  const uint32_t inner = amp_micro_dimension(precision);
  if (row >= rows || column >= columns || rows % inner != 0 ||
      columns % AMP_COLUMN_MICRO != 0)
    return -1;
  const uint64_t panel =
      (uint64_t)(column / AMP_COLUMN_MICRO) * (rows / inner) + row / inner;
  return (int64_t)(panel * inner * AMP_COLUMN_MICRO +
                   (uint64_t)(column % AMP_COLUMN_MICRO) * inner + row % inner);
}

/* storage.rs:301-345 */
int64_t or_amp_matrix_index(int role, int precision, uint32_t rows,
                            uint32_t columns, uint32_t row, uint32_t column) {
  if (row >= rows || column >= columns) return -1;
  switch (role) {
    case OR_AMP_LEFT: {
      const uint32_t inner = amp_micro_dimension(precision);
      if (columns % inner != 0) return -2;
      return (int64_t)((uint64_t)(column / inner) * rows * inner +
                       (uint64_t)row * inner + column % inner);
    }
    case OR_AMP_TRANSPOSED_RIGHT:
      return or_right_matrix_index(precision, columns, rows, column, row);
    case OR_AMP_TRANSPOSED_LEFT:
      return or_amp_matrix_index(OR_AMP_LEFT, precision, columns, rows, column, row);
    case OR_AMP_OUTPUT: {
      if (columns % AMP_COLUMN_MICRO != 0) return -2;
      const uint32_t logical_pair = column % AMP_COLUMN_MICRO / 2;
      const uint32_t physical_pair = logical_pair % 4 * 2 + logical_pair / 4;
      const uint32_t physical_column = physical_pair * 2 + column % 2;
      return (int64_t)((uint64_t)(column / AMP_COLUMN_MICRO) * rows * AMP_COLUMN_MICRO +
                       (uint64_t)row * AMP_COLUMN_MICRO + physical_column);
    }
    case OR_AMP_TRANSPOSED_OUTPUT:
      return or_amp_matrix_index(OR_AMP_OUTPUT, precision, columns, rows, column, row);
    default:
      return -3;
  }
}

/* storage.rs:705-725 */
static int right_matrix_coordinates(int precision, uint32_t rows, uint32_t columns,
                                    uint32_t linear, uint32_t *row, uint32_t *column) {
  const uint32_t inner = amp_micro_dimension(precision);
  if (rows % inner != 0 || columns % AMP_COLUMN_MICRO != 0) return -1;
  const uint32_t panel_elements = inner * AMP_COLUMN_MICRO;
  const uint32_t panel = linear / panel_elements;
  const uint32_t offset = linear % panel_elements;
  const uint32_t inner_groups = rows / inner;
  const uint32_t column_group = panel / inner_groups;
  const uint32_t inner_group = panel % inner_groups;
  *row = inner_group * inner + offset % inner;
  *column = column_group * AMP_COLUMN_MICRO + offset / inner;
  return 0;
}

/* storage.rs:656-703 */
int or_amp_matrix_coordinates(int role, int precision, uint32_t rows,
                              uint32_t columns, uint32_t linear, uint32_t *row,
                              uint32_t *column) {
  uint32_t a = 0, b = 0;
  int status;
  switch (role) {
    case OR_AMP_LEFT: {
      const uint32_t inner = amp_micro_dimension(precision);
      if (columns % inner != 0) return -2;
      const uint32_t panel_elements = rows * inner;
      const uint32_t panel = linear / panel_elements;
      const uint32_t offset = linear % panel_elements;
      *row = offset / inner;
      *column = panel * inner + offset % inner;
      return 0;
    }
    case OR_AMP_TRANSPOSED_RIGHT:
      status = right_matrix_coordinates(precision, columns, rows, linear, &a, &b);
      *column = a;
      *row = b;
      return status;
    case OR_AMP_TRANSPOSED_LEFT:
      status = or_amp_matrix_coordinates(OR_AMP_LEFT, precision, columns, rows,
                                         linear, &a, &b);
      *column = a;
      *row = b;
      return status;
    case OR_AMP_OUTPUT: {
      if (columns % AMP_COLUMN_MICRO != 0) return -2;
      const uint32_t panel_elements = rows * AMP_COLUMN_MICRO;
      const uint32_t panel = linear / panel_elements;
      const uint32_t offset = linear % panel_elements;
      const uint32_t physical_column = offset % AMP_COLUMN_MICRO;
      const uint32_t physical_pair = physical_column / 2;
      const uint32_t logical_pair = (physical_pair % 2) * 4 + physical_pair / 2;
      *row = offset / AMP_COLUMN_MICRO;
      *column = panel * AMP_COLUMN_MICRO + logical_pair * 2 + physical_column % 2;
      return 0;
    }
    case OR_AMP_TRANSPOSED_OUTPUT:
      status = or_amp_matrix_coordinates(OR_AMP_OUTPUT, precision, columns, rows,
                                         linear, &a, &b);
      *column = a;
      *row = b;
      return status;
    default:
      return -3;
  }
}

/* storage.rs:372-426 */
int64_t or_block_major_matrix_index(int transposed, uint32_t row_block,
                                    uint32_t column_block, int precision,
                                    uint32_t rows, uint32_t columns,
                                    uint32_t row, uint32_t column) {
  if (transposed)
    return or_block_major_matrix_index(0, row_block, column_block, precision,
                                       columns, rows, column, row);
  const uint32_t row_micro = amp_micro_dimension(precision);
  if (row >= rows || column >= columns || row_block == 0 || column_block == 0 ||
      rows % row_block != 0 || columns % column_block != 0 ||
      row_block % row_micro != 0)
    return -1;
  const uint64_t row_groups = row_block / row_micro;
  const uint64_t panel = (uint64_t)(row / row_block) * (columns / column_block) * row_groups +
                         (uint64_t)(column / column_block) * row_groups +
                         (row % row_block) / row_micro;
  return (int64_t)(panel * row_micro * column_block +
                   (uint64_t)(column % column_block) * row_micro + row % row_micro);
}

/* storage.rs:727-782 */
int or_block_major_matrix_coordinates(int transposed, uint32_t row_block,
                                      uint32_t column_block, int precision,
                                      uint32_t rows, uint32_t columns,
                                      uint32_t linear, uint32_t *row,
                                      uint32_t *column) {
  if (transposed) {
    uint32_t a = 0, b = 0;
    const int status = or_block_major_matrix_coordinates(
        0, row_block, column_block, precision, columns, rows, linear, &a, &b);
    *column = a;
    *row = b;
    return status;
  }
  const uint32_t row_micro = amp_micro_dimension(precision);
  if (row_block == 0 || column_block == 0 || rows % row_block != 0 ||
      columns % column_block != 0 || row_block % row_micro != 0)
    return -1;
  const uint32_t panel_elements = row_micro * column_block;
  const uint32_t panel = linear / panel_elements;
  const uint32_t offset = linear % panel_elements;
  const uint32_t row_groups = row_block / row_micro;
  const uint32_t column_groups = columns / column_block;
  const uint32_t panels_per_row_block = column_groups * row_groups;
  const uint32_t row_block_index = panel / panels_per_row_block;
  const uint32_t within_block = panel % panels_per_row_block;
  const uint32_t column_group = within_block / row_groups;
  const uint32_t row_group = within_block % row_groups;
  *row = row_block_index * row_block + row_group * row_micro + offset % row_micro;
  *column = column_group * column_block + offset / row_micro;
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Rearrange kernels on 16-bit payloads.                                     */
/* ------------------------------------------------------------------------- */

/*
 * Row-major [logical_rows, logical_columns] per matrix -> target order with
 * zero padding up to [physical_rows, physical_columns]
 * (device/rearrange_f16.cpp:72-153, target orders at crates/ipu-codegen/src/
 * kernel.rs:113-119: 0 AmpLeft, 1 AmpTransposedRight, 2 BlockMajor).  The
 * element placement uses the storage.rs maps above; padding positions hold 0
 * (rearrange_f16.cpp:86-89, 97-102, rearrange_amp_left_f16.S:93-132).
 * For AmpLeft the outer matrices fold into the row axis (storage.rs:250-266);
 * the other orders pack each matrix independently (storage.rs:216-249).
 */
int or_rearrange_row_major_f16(int target_order, uint32_t row_block,
                               uint32_t column_block, uint32_t matrices,
                               uint32_t logical_rows, uint32_t physical_rows,
                               uint32_t logical_columns,
                               uint32_t physical_columns, const uint16_t *src,
                               uint16_t *dst) {
  if (logical_rows > physical_rows || logical_columns > physical_columns) return -1;
  const uint64_t matrix_elements = (uint64_t)physical_rows * physical_columns;
  for (uint32_t m = 0; m < matrices; ++m) {
    for (uint32_t r = 0; r < physical_rows; ++r) {
      for (uint32_t c = 0; c < physical_columns; ++c) {
        int64_t physical;
        if (target_order == 0) {
          physical = or_amp_matrix_index(OR_AMP_LEFT, OR_F16, matrices * physical_rows,
                                         physical_columns, m * physical_rows + r, c);
        } else if (target_order == 1) {
          physical = or_amp_matrix_index(OR_AMP_TRANSPOSED_RIGHT, OR_F16, physical_rows,
                                         physical_columns, r, c);
          if (physical >= 0) physical += (int64_t)(m * matrix_elements);
        } else if (target_order == 2) {
          physical = or_block_major_matrix_index(0, row_block, column_block, OR_F16,
                                                 physical_rows, physical_columns, r, c);
          if (physical >= 0) physical += (int64_t)(m * matrix_elements);
        } else {
          return -3;
        }
        if (physical < 0) return -2;
        const uint16_t v =
            (r < logical_rows && c < logical_columns)
                ? src[(uint64_t)m * logical_rows * logical_columns +
                      (uint64_t)r * logical_columns + c]
                : (uint16_t)0;
        dst[physical] = v;
      }
    }
  }
  return 0;
}

/*
 * AMP-Output (0) or AMP-TransposedLeft (1) -> row-major with the physical
 * column pitch, device/unpack_amp_f16.cpp:53-79 (padding columns written 0).
 */
int or_unpack_to_row_major_f16(int source_order, uint32_t matrices,
                               uint32_t logical_rows, uint32_t physical_rows,
                               uint32_t logical_columns,
                               uint32_t physical_columns, const uint16_t *src,
                               uint16_t *dst) {
  if (source_order != 0 && source_order != 1) return -3;
  if (source_order == 0 && physical_columns % 16 != 0) return -2;
  if (source_order == 1 && physical_rows % 16 != 0) return -2;
  const uint64_t matrix_elements = (uint64_t)physical_rows * physical_columns;
  for (uint32_t m = 0; m < matrices; ++m) {
    const uint64_t base = m * matrix_elements;
    for (uint32_t r = 0; r < physical_rows; ++r) {
      for (uint32_t c = 0; c < physical_columns; ++c) {
        uint16_t v = 0;
        if (r < logical_rows && c < logical_columns) {
          int64_t physical;
          if (source_order == 0)
            physical = or_amp_matrix_index(OR_AMP_OUTPUT, OR_F16, physical_rows,
                                           physical_columns, r, c);
          else
            physical = or_amp_matrix_index(OR_AMP_TRANSPOSED_LEFT, OR_F16, physical_rows,
                                           physical_columns, r, c);
          if (physical < 0) return -2;
          v = src[base + (uint64_t)physical];
        }
        dst[base + (uint64_t)r * physical_columns + c] = v;
      }
    }
  }
  return 0;
}

/*
 * One shard of a tiled binding: storage.rs:201-285 (physical_index over the
 * shard's physical widths: row-major; block-major matrices matrix-major over
 * the outer axes; AMP Left / Output with the outer axes folded into the
 * rows; the transposed AMP roles matrix-major).
 */
int or_pack_shard(int kind, int variant, uint32_t row_block, uint32_t column_block,
                  int rank, const uint32_t *dims, const uint32_t *start,
                  const uint32_t *logical_end, const uint32_t *physical_end,
                  const uint16_t *logical, uint16_t *shard) {
  if (rank < 1 || rank > 8) return -1;
  if (kind != 0 && rank < 2) return -1;
  uint32_t w[8], lw[8], c[8];
  uint64_t total = 1, logical_total = 1;
  for (int a = 0; a < rank; ++a) {
    w[a] = physical_end[a] - start[a];
    lw[a] = logical_end[a] - start[a];
    total *= w[a];
    logical_total *= lw[a];
  }
  for (uint64_t i = 0; i < logical_total; ++i) {
    uint64_t rem = i;
    for (int a = rank - 1; a >= 0; --a) {
      c[a] = (uint32_t)(rem % lw[a]);
      rem /= lw[a];
    }
    uint64_t src = 0;
    for (int a = 0; a < rank; ++a) src = src * dims[a] + start[a] + c[a];
    int64_t phys;
    if (kind == 0) {
      uint64_t p = 0;
      for (int a = 0; a < rank; ++a) p = p * w[a] + c[a];
      phys = (int64_t)p;
    } else {
      uint64_t outer = 0, outer_count = 1;
      for (int a = 0; a + 2 < rank; ++a) {
        outer = outer * w[a] + c[a];
        outer_count *= w[a];
      }
      const uint32_t R = w[rank - 2], C = w[rank - 1];
      const uint32_t r = c[rank - 2], col = c[rank - 1];
      const uint64_t matrix = outer * (uint64_t)R * C;
      if (kind == 2) {
        const int64_t within = or_block_major_matrix_index(variant, row_block, column_block,
                                                           OR_F16, R, C, r, col);
        if (within < 0) return -2;
        phys = (int64_t)matrix + within;
      } else if (variant == OR_AMP_LEFT || variant == OR_AMP_OUTPUT) {
        phys = or_amp_matrix_index(variant, OR_F16, (uint32_t)(outer_count * R), C,
                                   (uint32_t)(outer * R + r), col);
        if (phys < 0) return -2;
      } else {
        const int64_t within = or_amp_matrix_index(variant, OR_F16, R, C, r, col);
        if (within < 0) return -2;
        phys = (int64_t)matrix + within;
      }
    }
    if (phys < 0 || (uint64_t)phys >= total) return -3;
    shard[phys] = logical[src];
  }
  return 0;
}

/* Plain transpose: row-major [rows, columns] -> row-major [columns, rows]. */
void or_transpose_u16(uint32_t matrices, uint32_t rows, uint32_t columns,
                      const uint16_t *src, uint16_t *dst) {
  const uint64_t me = (uint64_t)rows * columns;
  for (uint32_t m = 0; m < matrices; ++m)
    for (uint32_t r = 0; r < rows; ++r)
      for (uint32_t c = 0; c < columns; ++c)
        dst[m * me + (uint64_t)c * rows + r] = src[m * me + (uint64_t)r * columns + c];
}

/* ------------------------------------------------------------------------- */
/* GEMM: diagnostic.rs:533-654.  fp32 multiply-accumulate of row-major       */
/* operands with optional transposes (cblas_sgemm semantics: leading         */
/* dimension = last stored axis, diagnostic.rs:550-551).                      */
/* ------------------------------------------------------------------------- */
typedef float v8f __attribute__((vector_size(32)));

#define GEMM_MR 6
#define GEMM_NR 16
#define GEMM_KC 256
#define GEMM_MC 96
#define GEMM_NC 1024

typedef struct {
  const float *left, *right;
  float *out;
  uint32_t rows, columns, inner;
  uint32_t lda, ldb;
  int tl, tr;
} gemm_ctx;

static inline float left_at(const gemm_ctx *g, uint32_t i, uint32_t k) {
  return g->tl ? g->left[(uint64_t)k * g->lda + i] : g->left[(uint64_t)i * g->lda + k];
}
static inline float right_at(const gemm_ctx *g, uint32_t k, uint32_t j) {
  return g->tr ? g->right[(uint64_t)j * g->ldb + k] : g->right[(uint64_t)k * g->ldb + j];
}

static void gemm_micro(uint32_t kc, const float *ap, const float *bp, float *c,
                       uint32_t ldc, uint32_t mr, uint32_t nr, int first) {
  v8f acc[GEMM_MR][2];
  memset(acc, 0, sizeof(acc));
  for (uint32_t k = 0; k < kc; ++k) {
    v8f b0, b1;
    memcpy(&b0, bp + (uint64_t)k * GEMM_NR, 32);
    memcpy(&b1, bp + (uint64_t)k * GEMM_NR + 8, 32);
    const float *a = ap + (uint64_t)k * GEMM_MR;
    for (int i = 0; i < GEMM_MR; ++i) {
      const v8f av = {a[i], a[i], a[i], a[i], a[i], a[i], a[i], a[i]};
      acc[i][0] += av * b0;
      acc[i][1] += av * b1;
    }
  }
  for (uint32_t i = 0; i < mr; ++i) {
    float tmp[16];
    memcpy(tmp, &acc[i][0], 32);
    memcpy(tmp + 8, &acc[i][1], 32);
    float *row = c + (uint64_t)i * ldc;
    if (first)
      for (uint32_t j = 0; j < nr; ++j) row[j] = tmp[j];
    else
      for (uint32_t j = 0; j < nr; ++j) row[j] += tmp[j];
  }
}

static void gemm_rows_range(void *vctx, uint64_t begin_block, uint64_t end_block) {
  const gemm_ctx *g = (const gemm_ctx *)vctx;
  const uint32_t row_begin = (uint32_t)(begin_block * GEMM_MC);
  uint32_t row_end = (uint32_t)(end_block * GEMM_MC);
  if (row_end > g->rows) row_end = g->rows;
  if (row_begin >= row_end) return;
  float *bp = (float *)aligned_alloc(64, sizeof(float) * GEMM_KC * GEMM_NC);
  float *ap = (float *)aligned_alloc(64, sizeof(float) * GEMM_KC * GEMM_MC);
  if (g->inner == 0) {
    for (uint32_t i = row_begin; i < row_end; ++i)
      memset(g->out + (uint64_t)i * g->columns, 0, sizeof(float) * g->columns);
  }
  for (uint32_t jc = 0; jc < g->columns; jc += GEMM_NC) {
    const uint32_t nc = (g->columns - jc < GEMM_NC) ? g->columns - jc : GEMM_NC;
    for (uint32_t pc = 0; pc < g->inner; pc += GEMM_KC) {
      const uint32_t kc = (g->inner - pc < GEMM_KC) ? g->inner - pc : GEMM_KC;
      /* pack B[pc:pc+kc, jc:jc+nc] into NR-wide panels, zero padded */
      for (uint32_t jr = 0; jr < nc; jr += GEMM_NR) {
        float *panel = bp + (uint64_t)jr * kc;
        for (uint32_t k = 0; k < kc; ++k)
          for (uint32_t j = 0; j < GEMM_NR; ++j)
            panel[(uint64_t)k * GEMM_NR + j] =
                (jr + j < nc) ? right_at(g, pc + k, jc + jr + j) : 0.0f;
      }
      for (uint32_t ic = row_begin; ic < row_end; ic += GEMM_MC) {
        const uint32_t mc = (row_end - ic < GEMM_MC) ? row_end - ic : GEMM_MC;
        for (uint32_t ir = 0; ir < mc; ir += GEMM_MR) {
          float *panel = ap + (uint64_t)ir * kc;
          for (uint32_t k = 0; k < kc; ++k)
            for (uint32_t i = 0; i < GEMM_MR; ++i)
              panel[(uint64_t)k * GEMM_MR + i] =
                  (ir + i < mc) ? left_at(g, ic + ir + i, pc + k) : 0.0f;
        }
        for (uint32_t jr = 0; jr < nc; jr += GEMM_NR) {
          const uint32_t nr = (nc - jr < GEMM_NR) ? nc - jr : GEMM_NR;
          for (uint32_t ir = 0; ir < mc; ir += GEMM_MR) {
            const uint32_t mr = (mc - ir < GEMM_MR) ? mc - ir : GEMM_MR;
            gemm_micro(kc, ap + (uint64_t)ir * kc, bp + (uint64_t)jr * kc,
                       g->out + (uint64_t)(ic + ir) * g->columns + jc + jr,
                       g->columns, mr, nr, pc == 0);
          }
        }
      }
    }
  }
  free(bp);
  free(ap);
}

static void gemm_one(const float *left, const float *right, float *out,
                     uint32_t rows, uint32_t columns, uint32_t inner, int tl,
                     int tr, int threads) {
  gemm_ctx g;
  g.left = left;
  g.right = right;
  g.out = out;
  g.rows = rows;
  g.columns = columns;
  g.inner = inner;
  g.tl = tl;
  g.tr = tr;
  g.lda = tl ? rows : inner;
  g.ldb = tr ? inner : columns;
  const uint64_t blocks = (rows + GEMM_MC - 1) / GEMM_MC;
  parallel_for(blocks, threads, gemm_rows_range, &g);
}

/* diagnostic.rs:533-579 for a flat batch (broadcast strides of 0 allowed). */
int or_gemm_f32(const float *left, const float *right, float *out,
                uint32_t batches, uint64_t left_batch_stride,
                uint64_t right_batch_stride, uint32_t rows, uint32_t columns,
                uint32_t inner, int transpose_left, int transpose_right,
                int threads) {
  for (uint32_t b = 0; b < batches; ++b)
    gemm_one(left + b * left_batch_stride, right + b * right_batch_stride,
             out + (uint64_t)b * rows * columns, rows, columns, inner,
             transpose_left, transpose_right, threads);
  return 0;
}

/* fp16 operands dequantized exactly, fp32 GEMM, result quantized to fp16
 * (diagnostic.rs:454-460 with the F16 output precision, 841-847). */
int or_gemm_f16(const uint16_t *left, const uint16_t *right, uint16_t *out,
                uint32_t batches, uint64_t left_batch_stride,
                uint64_t right_batch_stride, uint32_t rows, uint32_t columns,
                uint32_t inner, int transpose_left, int transpose_right,
                int threads) {
  const uint64_t left_elems = (uint64_t)(left_batch_stride ? batches : 1) * rows * inner;
  const uint64_t right_elems = (uint64_t)(right_batch_stride ? batches : 1) * inner * columns;
  const uint64_t out_elems = (uint64_t)batches * rows * columns;
  float *lf = (float *)malloc(sizeof(float) * (left_elems ? left_elems : 1));
  float *rf = (float *)malloc(sizeof(float) * (right_elems ? right_elems : 1));
  float *of = (float *)malloc(sizeof(float) * (out_elems ? out_elems : 1));
  if (!lf || !rf || !of) {
    free(lf);
    free(rf);
    free(of);
    return -4;
  }
  or_f16_to_f32_array(left, lf, left_elems);
  or_f16_to_f32_array(right, rf, right_elems);
  or_gemm_f32(lf, rf, of, batches, left_batch_stride, right_batch_stride, rows,
              columns, inner, transpose_left, transpose_right, threads);
  or_f32_to_f16_array(of, out, out_elems);
  free(lf);
  free(rf);
  free(of);
  return 0;
}

/* Sampled rows of a row-major fp16 GEMM (no transposes), fp32 results (not
 * quantized) for sampled parity checks at sizes where the full CPU product
 * is too slow; sample selection mirrors diagnostic.rs:259-267. */
typedef struct {
  const uint16_t *left, *right;
  float *out;
  const float *right_f;
  uint32_t columns, inner;
  const uint32_t *rows;
} gemm_rows_ctx;

static void gemm_sample_range(void *vctx, uint64_t begin, uint64_t end) {
  const gemm_rows_ctx *g = (const gemm_rows_ctx *)vctx;
  float *a = (float *)malloc(sizeof(float) * g->inner);
  for (uint64_t s = begin; s < end; ++s) {
    const uint32_t r = g->rows[s];
    for (uint32_t k = 0; k < g->inner; ++k)
      a[k] = or_f16_to_f32(g->left[(uint64_t)r * g->inner + k]);
    float *o = g->out + s * g->columns;
    for (uint32_t j = 0; j < g->columns; ++j) o[j] = 0.0f;
    for (uint32_t k = 0; k < g->inner; ++k) {
      const float av = a[k];
      const float *b = g->right_f + (uint64_t)k * g->columns;
      for (uint32_t j = 0; j < g->columns; ++j) o[j] += av * b[j];
    }
  }
  free(a);
}

int or_gemm_f16_rows(const uint16_t *left, const uint16_t *right, float *out,
                     uint32_t rows, uint32_t columns, uint32_t inner,
                     const uint32_t *row_list, uint32_t row_count, int threads) {
  for (uint32_t s = 0; s < row_count; ++s)
    if (row_list[s] >= rows) return -1;
  float *rf = (float *)malloc(sizeof(float) * (uint64_t)inner * columns);
  if (!rf) return -4;
  or_f16_to_f32_array(right, rf, (uint64_t)inner * columns);
  gemm_rows_ctx g = {left, right, out, rf, columns, inner, row_list};
  parallel_for(row_count, threads, gemm_sample_range, &g);
  free(rf);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Attention: diagnostic.rs:711-780 (two-pass softmax in f32, causal key     */
/* limit at 741-745, scale at 733-736).                                       */
/* ------------------------------------------------------------------------- */
typedef struct {
  const float *q, *k, *v;
  float *out;
  uint32_t streams, query_rows, key_rows, width, value_width;
  int causal;
  float scale;
  const uint32_t *row_list; /* flat (stream * query_rows + row) indices */
  uint32_t row_count;
} attention_ctx;

static void attention_range(void *vctx, uint64_t begin, uint64_t end) {
  const attention_ctx *a = (const attention_ctx *)vctx;
  float *logits = (float *)malloc(sizeof(float) * (a->key_rows ? a->key_rows : 1));
  for (uint64_t s = begin; s < end; ++s) {
    const uint64_t flat = a->row_list ? a->row_list[s] : s;
    const uint32_t stream = (uint32_t)(flat / a->query_rows);
    const uint32_t row = (uint32_t)(flat % a->query_rows);
    uint32_t allowed = a->key_rows;
    if (a->causal) allowed = (row + 1 < a->key_rows) ? row + 1 : a->key_rows;
    const float *qrow = a->q + ((uint64_t)stream * a->query_rows + row) * a->width;
    for (uint32_t column = 0; column < allowed; ++column) {
      const float *krow = a->k + ((uint64_t)stream * a->key_rows + column) * a->width;
      float dot = 0.0f;
      for (uint32_t inner = 0; inner < a->width; ++inner) dot += qrow[inner] * krow[inner];
      logits[column] = dot * a->scale;
    }
    float maximum = -INFINITY;
    for (uint32_t c = 0; c < allowed; ++c) maximum = fmaxf(maximum, logits[c]);
    float sum = 0.0f;
    for (uint32_t c = 0; c < allowed; ++c) {
      logits[c] = expf(logits[c] - maximum);
      sum += logits[c];
    }
    float *o = a->out + s * a->value_width;
    for (uint32_t column = 0; column < a->value_width; ++column) {
      float result = 0.0f;
      for (uint32_t inner = 0; inner < allowed; ++inner)
        result += logits[inner] / sum *
                  a->v[((uint64_t)stream * a->key_rows + inner) * a->value_width + column];
      o[column] = result;
    }
  }
  free(logits);
}

int or_attention(const float *query, const float *key, const float *value,
                 float *out, uint32_t streams, uint32_t query_rows,
                 uint32_t key_rows, uint32_t width, uint32_t value_width,
                 int causal, float scale, int use_scale,
                 const uint32_t *row_list, uint32_t row_count, int threads) {
  attention_ctx a;
  a.q = query;
  a.k = key;
  a.v = value;
  a.out = out;
  a.streams = streams;
  a.query_rows = query_rows;
  a.key_rows = key_rows;
  a.width = width;
  a.value_width = value_width;
  a.causal = causal;
  a.scale = use_scale ? scale : 1.0f / sqrtf((float)width);
  a.row_list = row_list;
  a.row_count = row_list ? row_count : streams * query_rows;
  if (row_list)
    for (uint32_t i = 0; i < row_count; ++i)
      if (row_list[i] >= (uint64_t)streams * query_rows) return -1;
  parallel_for(a.row_count, threads, attention_range, &a);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* GELU tanh approximation, main.rs:1985-1987 applied by map_unary           */
/* (diagnostic.rs:433-436, 782-787) on fp16 inputs, then quantized to fp16.  */
/* ------------------------------------------------------------------------- */
float or_gelu_reference(float value) {
  return 0.5f * value * (1.0f + tanhf(0.7978846f * (value + 0.044715f * value * value * value)));
}

void or_gelu_f16(const uint16_t *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(or_gelu_reference(or_f16_to_f32(src[i])));
}

/* ------------------------------------------------------------------------- */
/* Add with numpy broadcasting (diagnostic.rs:673-683, 789-833).             */
/* ------------------------------------------------------------------------- */
int or_add_f32(const float *left, const uint32_t *left_shape, int left_rank,
               const float *right, const uint32_t *right_shape, int right_rank,
               float *out, uint32_t *out_shape, int *out_rank) {
  const int rank = left_rank > right_rank ? left_rank : right_rank;
  if (rank > 16) return -1;
  uint32_t shape[16], ls[16], rs[16];
  for (int axis = 0; axis < rank; ++axis) {
    const int la = axis - (rank - left_rank);
    const int ra = axis - (rank - right_rank);
    ls[axis] = la >= 0 ? left_shape[la] : 1;
    rs[axis] = ra >= 0 ? right_shape[ra] : 1;
    if (ls[axis] != rs[axis] && ls[axis] != 1 && rs[axis] != 1) return -2;
    shape[axis] = ls[axis] > rs[axis] ? ls[axis] : rs[axis];
    out_shape[axis] = shape[axis];
  }
  *out_rank = rank;
  uint64_t total = 1;
  for (int axis = 0; axis < rank; ++axis) total *= shape[axis];
  uint32_t coords[16];
  for (uint64_t index = 0; index < total; ++index) {
    uint64_t rem = index;
    for (int axis = rank - 1; axis >= 0; --axis) {
      coords[axis] = (uint32_t)(rem % shape[axis]);
      rem /= shape[axis];
    }
    uint64_t lo = 0, ro = 0;
    for (int axis = 0; axis < rank; ++axis) {
      lo = lo * ls[axis] + (ls[axis] == 1 ? 0 : coords[axis]);
      ro = ro * rs[axis] + (rs[axis] == 1 ? 0 : coords[axis]);
    }
    out[index] = left[lo] + right[ro];
  }
  return 0;
}

/* diagnostic.rs:685-709 */
int or_split_heads(const float *input, uint32_t batch, uint32_t rows,
                   uint32_t width, uint32_t heads, float *out) {
  if (heads == 0 || width % heads != 0) return -1;
  const uint32_t channels = width / heads;
  for (uint32_t b = 0; b < batch; ++b)
    for (uint32_t h = 0; h < heads; ++h)
      for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < channels; ++c) {
          const uint64_t source = ((uint64_t)b * rows + r) * width + (uint64_t)h * channels + c;
          const uint64_t target = (((uint64_t)b * heads + h) * rows + r) * channels + c;
          out[target] = input[source];
        }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Reductions.                                                                */
/* ------------------------------------------------------------------------- */

/* device/reduce_add_f16.S:54-70: out[i] = initial[i] + remote[0][i] + ...
 * + remote[P-1][i], evaluated left to right with an fp16 rounding after each
 * addition (f16v4add).  The fp32 sum of two fp16 values rounded once to fp16
 * is the correctly rounded fp16 sum (24 >= 2*11+2). */
void or_reduce_sum_f16(const uint16_t *initial, const uint16_t *remote,
                       uint32_t remote_partials, uint32_t count, uint16_t *out) {
  for (uint32_t i = 0; i < count; ++i) {
    uint16_t acc = initial[i];
    for (uint32_t p = 0; p < remote_partials; ++p)
      acc = or_f32_to_f16(or_f16_to_f32(acc) +
                          or_f16_to_f32(remote[(uint64_t)p * count + i]));
    out[i] = acc;
  }
}

/* Row reduction with fp32 accumulation, r[i] = sum_j X[i][j]: the
 * ReductionSum of crates/ipu-codegen/src/operator.rs:307-347 applied to the
 * rows of X with fp32 in place of fp16 accumulation.  Accumulated in f64 and
 * rounded once, so it is the exactly rounded row sum. */
typedef struct {
  const uint16_t *src;
  uint32_t columns;
  float *out;
} rows_ctx;

static void reduce_rows_range(void *vctx, uint64_t begin, uint64_t end) {
  const rows_ctx *r = (const rows_ctx *)vctx;
  for (uint64_t i = begin; i < end; ++i) {
    double acc = 0.0;
    const uint16_t *row = r->src + i * r->columns;
    for (uint32_t j = 0; j < r->columns; ++j) acc += (double)or_f16_to_f32(row[j]);
    r->out[i] = (float)acc;
  }
}

void or_reduce_rows_f16(const uint16_t *src, uint32_t rows, uint32_t columns,
                        float *out, int threads) {
  rows_ctx r = {src, columns, out};
  parallel_for(rows, threads, reduce_rows_range, &r);
}

int or_reduce_rows_block_major_f16(const uint16_t *src, uint32_t row_block,
                                   uint32_t column_block, uint32_t rows,
                                   uint32_t columns, float *out, int threads) {
  uint16_t *row_major = (uint16_t *)malloc(sizeof(uint16_t) * (uint64_t)rows * columns);
  if (!row_major) return -4;
  const uint64_t total = (uint64_t)rows * columns;
  for (uint64_t linear = 0; linear < total; ++linear) {
    uint32_t r, c;
    if (or_block_major_matrix_coordinates(0, row_block, column_block, OR_F16, rows,
                                          columns, (uint32_t)linear, &r, &c) != 0) {
      free(row_major);
      return -2;
    }
    row_major[(uint64_t)r * columns + c] = src[linear];
  }
  or_reduce_rows_f16(row_major, rows, columns, out, threads);
  free(row_major);
  return 0;
}

/* SplitMix64 output function (Steele, Lea, Flood 2014) applied to one state
 * advance: the generator behind gaussian(seed, index) at main.rs:2035-2038. */
uint64_t or_splitmix64(uint64_t state) {
  uint64_t z = state + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

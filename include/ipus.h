/*
 * libipus: C ABI of the MI355X (gfx950) backend for the ipu-stack hot path.
 *
 * This header is the drop-in boundary.  It replaces the roles that the
 * reference splits over four Rust crates:
 *   - ipu-runtime / ipu-driver (device open, host sessions, PCIe exchange):
 *       crates/ipu-runtime/src/lib.rs:17-47, crates/ipu-driver/src/lib.rs:1341-1600
 *     -> ipus_context_*, ipus_buffer_*, ipus_stream_sync, ipus_event_*
 *   - ipu-elf (compile + link, symbol lookup): crates/ipu-elf/src/lib.rs:86-170, 322
 *     -> kernels are compiled into this library; ipus_kernel_abi looks them up
 *   - ipu-target (ComputeStep emission: m2 = output, m3.. = inputs, then u32
 *     scalars): crates/ipu-target/src/program.rs:112-121,
 *     crates/ipu-target/src/emit.rs:514-551,
 *     crates/ipu-codegen/src/kernel.rs:14-16, 818-865
 *     -> ipus_launch(symbol, out, inputs, scalars)
 *   - the tile-kernel ABI registry and run validation:
 *     crates/ipu-codegen/src/kernel.rs:1215-1435 (tile_kernel_abi,
 *     validate_kernel_run) -> ipus_kernel_abi + the checks inside ipus_launch.
 *
 * Conventions (kernel.rs:14-16, crates/ipu-codegen/src/operator.rs:467-537):
 *   - The caller owns every buffer.  Kernels read inputs and write the output
 *     and allocate nothing.
 *   - Launches are ordered on the context's stream (replacing BSP phases).
 *   - Every call returns 0 on success or a negative IPUS_ERROR_* code;
 *     ipus_last_error() returns the message of the calling thread's last
 *     failure.  HIP runtime failures map to IPUS_ERROR_HIP_BASE - hipError_t.
 *   - Scalars are u32, as in the reference's PlannedKernelCall::arguments
 *     (kernel.rs:136-140).  f32 values travel as their bit patterns, as in
 *     AttentionScale::ValueBits (crates/ipu-codegen/src/graph.rs:147-165).
 */
#ifndef IPUS_H
#define IPUS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (KernelAbiError, kernel.rs:140-162) ---- */
#define IPUS_OK 0
#define IPUS_ERROR_INVALID_ARGUMENT (-1)   /* RequirementMismatch / bad shape */
#define IPUS_ERROR_POINTER_ARITY (-2)      /* PointerArity { expected, actual } */
#define IPUS_ERROR_UNAVAILABLE (-3)        /* Unavailable(spec): no device kernel */
#define IPUS_ERROR_UNSUPPORTED_COUNT (-4)  /* UnsupportedElementCount */
#define IPUS_ERROR_UNKNOWN_SYMBOL (-5)     /* symbol not in the registry */
#define IPUS_ERROR_GRAPH (-6)              /* GraphError (graph.rs:221-245) */
#define IPUS_ERROR_BUILD (-7)              /* PackageBuildError (package.rs:48-78) */
#define IPUS_ERROR_NO_DEVICE (-8)
#define IPUS_ERROR_OUT_OF_MEMORY (-9)
/* A reference symbol that names an IPU tile codelet with no per-tile GPU
 * counterpart (the tile GEMM codelets, the staged-attention codelets): the
 * caller translates the whole operator to one launch instead.  The message
 * names the replacement symbol. */
#define IPUS_ERROR_TRANSLATED (-10)
#define IPUS_ERROR_HIP_BASE (-1000)        /* IPUS_ERROR_HIP_BASE - hipError_t */

/* Message of the calling thread's most recent failure ("" if none). */
const char *ipus_last_error(void);
/* Library version string. */
const char *ipus_version(void);

/* ---- context: one device, one stream (Runtime::open / HostSession) ---- */
typedef struct ipus_context ipus_context;

typedef struct ipus_device_info {
  char name[64];          /* e.g. "AMD Instinct MI355X"; where the runtime
                             reports none, the driver's sysfs product_name
                             of the device's PCI function */
  char arch[32];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width;
  uint64_t global_memory_bytes;
  int lds_bytes_per_block;
} ipus_device_info;

int ipus_device_count(int *count);
int ipus_context_create(int device, ipus_context **out);
int ipus_context_destroy(ipus_context *context);
int ipus_context_device_info(ipus_context *context, ipus_device_info *info);
/* Stream handle (hipStream_t) of the context, for callers that interoperate
 * with other HIP code.  Launches through this library go to this stream. */
int ipus_context_stream(ipus_context *context, void **stream);

/* ---- buffers: replace SRAM placement, host exchange and FillZero ---- */
int ipus_buffer_alloc(ipus_context *context, size_t bytes, void **device_pointer);
int ipus_buffer_free(ipus_context *context, void *device_pointer);
/* Synchronous host <-> device copies (complete before returning). */
int ipus_buffer_upload(ipus_context *context, void *device_dst, const void *host_src,
                       size_t bytes);
int ipus_buffer_download(ipus_context *context, void *host_dst, const void *device_src,
                         size_t bytes);
/* Buffers allocated through the context and not yet freed (count, bytes).
 * ipus_context_destroy releases any that remain.  No reference counterpart:
 * it lets a caller check that an error path released what it allocated. */
int ipus_context_live_buffers(ipus_context *context, uint64_t *count, uint64_t *bytes);
/* Failure injection for tests of error propagation (the role of the
 * reference's device timeouts and retry path, crates/ipu-tests/src/
 * main.rs:985-1006, without a device fault): after `launches_before` more
 * ipus_launch calls on this context, the next one returns `status` (< 0)
 * without enqueuing work and the injection clears; status 0 cancels. */
int ipus_context_inject_launch_failure(ipus_context *context, uint32_t launches_before,
                                       int status);
/* Stream-ordered device copy and byte fill. */
int ipus_buffer_copy(ipus_context *context, void *device_dst, const void *device_src,
                     size_t bytes);
int ipus_buffer_memset(ipus_context *context, void *device_pointer, int value, size_t bytes);

/* ---- synchronisation and timing ---- */
int ipus_stream_sync(ipus_context *context);
typedef struct ipus_event ipus_event;
int ipus_event_create(ipus_context *context, ipus_event **event);
int ipus_event_destroy(ipus_event *event);
int ipus_event_record(ipus_context *context, ipus_event *event);
int ipus_event_elapsed_ms(ipus_event *start, ipus_event *end, float *milliseconds);

/* ---- kernel ABI registry (tile_kernel_abi, kernel.rs:1215-1382) ----
 *
 * Symbols (output, inputs, u32 scalars in order):
 *   ipu_stack_gemm_f16                 out f16 [B,M,N]; left, right f16;
 *        batches, rows, columns, inner, transpose_left, transpose_right,
 *        left_batch_stride, right_batch_stride  (strides in elements, 0 =
 *        broadcast).  Replaces gemm_f16_amp (device/gemm_f16_amp.S:186-440)
 *        with fp32 accumulation and fp16 output.
 *   ipu_stack_gemm_f16_gelu            as ipu_stack_gemm_f16, then the tanh
 *        GELU of each fp16 result element (bit-identical to
 *        ipu_stack_gemm_f16 followed by ipu_stack_gelu_tanh_approx_f16).  No
 *        reference symbol: build_package fuses a Gemm whose result feeds only
 *        one Gelu (graph.rs:315-331) into this launch.
 *   ipu_stack_gemm_f16_accumulate      out f16 [B,M,N]; left, right, addend
 *        f16; the ipu_stack_gemm_f16 scalars, then addend_batch_stride,
 *        addend_row_stride (elements; 0 broadcasts the addend over batches /
 *        rows): out = addend + A.B with the product rounded to fp16 first
 *        and the sum formed like ipu_stack_add_f16 (fp32 add, one rounding),
 *        so it is bit-identical to ipu_stack_gemm_f16 followed by that Add.
 *        The addend may be the output itself (the reference's accumulate
 *        mode, C += A.B: device/gemm_f16_amp.S:43-52, 290-363, used after
 *        the first K block by crates/ipu-codegen/src/low.rs:3483-3486), but
 *        the output must not overlap A or B.  build_package fuses a Gemm
 *        whose result only feeds an Add into this launch.
 *   ipu_stack_gemm_f16_split           out fp32 partials
 *        float[splits][batches][rows][columns]; inputs as ipu_stack_gemm_f16;
 *        scalars as ipu_stack_gemm_f16 plus splits: split z sums k in
 *        [z c, (z + 1) c), c = 64 * ceil(ceil(inner / splits) / 64), and
 *        ceil(inner / c) must equal splits.  Needs the 256 x 256 kernel's
 *        conditions (16-byte aligned operands; columns and inner, and rows
 *        when the left operand is transposed, multiples of 8), else
 *        IPUS_ERROR_UNAVAILABLE.  No reference symbol (the reference's
 *        split-K is the ParallelReduction plan, operator.rs:307-347):
 *        build_package plans it for few-tile, long-K GEMMs.
 *   ipu_stack_reduce_splits_f16        out f16; input the fp32 partials;
 *        splits, element_count (a multiple of 8), gelu (0/1): the sum over
 *        splits in order, rounded to fp16 once (GELU of that value when
 *        gelu = 1, as in ipu_stack_gemm_f16_gelu).
 *   ipu_stack_reduce_splits_accumulate_f16  out f16; partials, addend f16;
 *        splits, batches, rows, columns, addend_batch_stride,
 *        addend_row_stride: the split sum rounded to fp16, plus the addend
 *        as in ipu_stack_gemm_f16_accumulate (columns a multiple of 8).
 *   ipu_stack_gemm_f32                 as above in fp32
 *        (device/gemm_f32_64_amp.S:125-385).
 *   ipu_stack_flash_attention_online_f16  out (f32 or f16); query, key,
 *        value f16 [streams, rows, width]; matrices, query_rows, key_rows,
 *        query_dimension, value_dimension, scale_bits (0 = 1/sqrt(width)),
 *        causal, output_f16.  Shape fields follow AttentionKernelShape
 *        (kernel.rs:121-129); semantics device/flash_attention_online_f16.cpp:
 *        68-143 plus the causal limit of crates/ipu-tests/src/diagnostic.rs:741-745.
 *   ipu_stack_flash_attention_heads_f16  as above, then query_heads,
 *        key_heads, value_heads: operand stream s is head s % h of matrix
 *        s / h of an unsplit [streams / h, rows, h * width] tensor (h = 1:
 *        contiguous; streams % h == 0).  The zero-copy form of SplitHeads
 *        (operator.rs:213-279) feeding attention; build_package emits it.
 *   ipu_stack_gelu_tanh_approx_f16     out f16; input f16; element_count
 *        (kernel.rs:1251-1263; count must be even, kernel.rs:1400-1413).
 *   ipu_stack_reduce_sum_f16           out f16; initial, packed remotes f16;
 *        num_partials (= remote partial count), element_count
 *        (kernel.rs:1264-1274; partials >= 2 and count % 8 == 0,
 *        kernel.rs:1414-1423; semantics device/reduce_add_f16.S:54-70).
 *   ipu_stack_rearrange_row_major_f16  out f16; source f16 row-major;
 *        logical_rows, physical_rows, target_order (0 AmpLeft,
 *        1 AmpTransposedRight, 2 BlockMajor), logical_columns,
 *        physical_columns, row_block, column_block, matrices
 *        (kernel.rs:1340-1364; device/rearrange_f16.cpp:36-155).
 *   ipu_stack_unpack_amp_f16           out f16 row-major; source f16;
 *        matrices, logical_rows, physical_rows, logical_columns,
 *        physical_columns, source_order (0 AmpOutput, 1 AmpTransposedLeft)
 *        (kernel.rs:1319-1339; device/unpack_amp_f16.cpp:30-83).
 *   ipu_stack_transpose_f16            out f16 [B,N,M]; source f16 [B,M,N];
 *        matrices, rows, columns.  No reference symbol: the graph-level
 *        transpose of a row-major matrix (BlockMajorOrder::TransposedMatrix
 *        semantics, crates/ipu-codegen/src/storage.rs:390-401).
 *   ipu_stack_reduce_rows_f16          out f32 [rows]; source f16 logical
 *        [rows, columns]; rows, columns, source_order (3 row-major,
 *        2 block-major), row_block, column_block.  ReductionSum over the
 *        columns with fp32 accumulation (operator.rs:307-347).
 *   ipu_stack_fill_zero                out; no inputs; byte_count.  The
 *        plan's own FillZero step (arena values, fp32 partials); no reference
 *        symbol.
 *   ipu_stack_fill_zero_u64            out; no inputs; words_per_worker,
 *        remainder_workers: the reference's FillZero step as
 *        materialize_kernel_run emits it (FILL_ZERO_U64_SYMBOL,
 *        crates/ipu-target/src/emit.rs:38; scalars kernel.rs:1223-1229,
 *        1175-1176): zeroes 8 * (6 * words_per_worker + remainder_workers)
 *        bytes; remainder_workers must be < 6.
 *
 * Reference per-shape symbols.  The reference links one specialization per
 * operand shape and names it by that shape (KernelBuildPlan::from_program,
 * kernel.rs:321-328, 374-379, 506-515).  ipus_kernel_abi, ipus_launch and
 * ipus_validate_kernel_run accept those names; the suffix fixes the shape of
 * one launch of the generic kernel:
 *   ipu_stack_rearrange_row_major_to_amp_f16_o{T}_r{LR}_p{PR}_c{LC}_p{PC}
 *        out; source row-major; the reference's scalars logical_rows,
 *        physical_rows, target_order (= T), logical_columns,
 *        physical_columns (kernel.rs:1351-1361), one matrix.  The scalars'
 *        physical extents must equal the suffix, and the logical ones too
 *        unless the suffix holds 0 there (rearrangement_specialization,
 *        kernel.rs:1122-1146).  T = 2 is block-major {64, 16}, the one block
 *        shape the reference plans for this conversion (layout.rs:356-361).
 *        Replaces rearrange_amp_left_f16.S, rearrange_block_major_f16.S,
 *        rearrange_transposed_right_f16.S and rearrange_f16.cpp.
 *   ipu_stack_unpack_amp_to_row_major_f16_o{S}_r{LR}_p{PR}_c{LC}_p{PC}
 *        out row-major; source AMP-Output (S = 0) or AMP-TransposedLeft
 *        (S = 1); scalars matrices, logical_rows, physical_rows,
 *        logical_columns, physical_columns (kernel.rs:1327-1336), extents
 *        equal to the suffix (device/unpack_amp_f16.cpp:6-40).
 *   ipu_stack_flash_attention_online_f16_m{B}_q{Q}_k{K}_d{D}_v{V}_{scale:08x}
 *        out f32; query, key, value f16 row-major; no scalars
 *        (AttentionKernelShape, kernel.rs:121-129, 986-1040): non-causal,
 *        scale = the f32 with those bits.
 * Reference symbols that are not forwarded return IPUS_ERROR_TRANSLATED
 * (the tile GEMM codelets ipu_stack_gemm_{f16,f32}_{init,accumulate}_...,
 * kernel.rs:185-193, and the staged-attention codelets
 * ipu_stack_attention_{softmax,merge}_..., kernel.rs:546-640) or
 * IPUS_ERROR_UNAVAILABLE (symbols the reference itself marks Required:
 * fp8 GEMM and casts, ipu_stack_unsupported_*).
 *
 *   ipu_stack_cast_f32_f16, ipu_stack_cast_f16_f32   out; input;
 *        element_count (Cast, kernel.rs:1313-1318).
 *   ipu_stack_add_f16, ipu_stack_add_f32   out; left, right; element_count,
 *        left_broadcast_stride, right_broadcast_stride  (Add,
 *        kernel.rs:1275-1287): out[i] = left[i % L] + right[i % R] where
 *        L, R are the operand element counts given by the two strides
 *        (trailing-axis numpy broadcasting; the graph executor handles the
 *        general case).
 *
 * Roofline calibration (no counterpart in the reference; used by the bench
 * to report the clock the MFMA pipes sustain for a given operand pattern):
 *   ipus_calibrate_mfma_f16            out: u64 shader-clock cycles, u64
 *        100 MHz ticks, then blocks*256 floats; input: operand_count
 *        fragments of 8 fp16; operand_count, iterations, blocks.  Each
 *        wave issues 8*iterations v_mfma_f32_32x32x16_f16 on its fragments.
 *   ipus_calibrate_mfma_f16_16x16x32   the same with v_mfma_f32_16x16x32_f16
 *        (the form the GEMM and attention kernels issue), eight fragment
 *        pairs per lane so that consecutive MFMAs see different operands.
 *   ipus_calibrate_copy                out; input; byte_count (a multiple of
 *        16, both pointers 16-byte aligned): a plain copy with ordinary
 *        16-byte loads and stores, whose HBM traffic counters scale those of
 *        other kernels to bytes.
 */
#define IPUS_MAX_SCALARS 32

typedef struct ipus_kernel_abi_info {
  const char *symbol;
  int input_count;
  int scalar_count;
  const char *scalar_names[IPUS_MAX_SCALARS];
  int implemented; /* KernelAvailability::Implemented */
} ipus_kernel_abi_info;

int ipus_kernel_count(int *count);
int ipus_kernel_abi_at(int index, ipus_kernel_abi_info *info);
int ipus_kernel_abi(const char *symbol, ipus_kernel_abi_info *info);

/* validate_kernel_run (kernel.rs:1384-1435) without a device: the symbol
 * resolves (including the reference per-shape names above), pointer arity
 * and scalar count match its ABI, and the scalars meet its constraints
 * (even GELU count, reduce partials and count, FillZero remainder, per-shape
 * suffix agreement).  Returns 0 or the status ipus_launch would return for
 * the same call before touching the device. */
int ipus_validate_kernel_run(const char *symbol, int input_count, const uint32_t *scalars,
                             int scalar_count);

/* One ComputeStep{symbol, output_address, input_addresses, arguments}:
 * validates pointer arity and scalar constraints (validate_kernel_run,
 * kernel.rs:1384-1435) and enqueues on the context stream. */
int ipus_launch(ipus_context *context, const char *symbol, void *output,
                const void *const *inputs, int input_count, const uint32_t *scalars,
                int scalar_count);

/* ---- split-K fp16 GEMM that allocates nothing ----
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same computation as launching
 * ipu_stack_gemm_f16_split into a caller-allocated partials buffer and then
 * ipu_stack_reduce_splits_f16 (gelu 0/1) into `output`, with the partials in
 * a device array the library holds for each device from its first context
 * until the process ends.  Arguments are those two symbols' scalars; the
 * operands and output follow ipu_stack_gemm_f16.  The partials,
 * batches * rows * columns * splits fp32 values, must fit
 * IPUS_SPLIT_SCRATCH_BYTES (16 MiB: build_package's split plans, at most 64
 * split tiles of 256 x 256, all fit), else IPUS_ERROR_UNSUPPORTED_COUNT.
 * The call enqueues on the context's stream and calls no allocator.  Every
 * call on one device shares that device's array: calls that overlap on one
 * device (from different streams or threads) race. */
#define IPUS_SPLIT_SCRATCH_BYTES (16ull << 20)
int ipus_gemm_f16_split_noalloc(ipus_context *context, void *output, const void *left,
                                const void *right, uint32_t batches, uint32_t rows,
                                uint32_t columns, uint32_t inner, int transpose_left,
                                int transpose_right, uint64_t left_batch_stride,
                                uint64_t right_batch_stride, uint32_t splits, int gelu);

/* ---- synthetic inputs (host, deterministic, multithreaded) ----
 * value(seed, tensor, i) from SplitMix64(seed ^ (tensor << 48) ^ i):
 * distribution 0 = uniform [-1, 1) from the top 24 bits, 1 = normal (Box-Muller
 * on two draws), times `scale`; fp16 outputs are rounded to nearest even. */
int ipus_synth_f16(uint16_t *out, uint64_t count, uint64_t seed, uint32_t tensor,
                   int distribution, float scale);
int ipus_synth_f32(float *out, uint64_t count, uint64_t seed, uint32_t tensor,
                   int distribution, float scale);

#ifdef __cplusplus
}
#endif
#endif /* IPUS_H */

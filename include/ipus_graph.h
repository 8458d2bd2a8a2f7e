/*
 * libipus graph API: the ipu-codegen surface, build_package(ComputeGraph,
 * PackageConfig), lowered to a plan of GPU kernel launches.
 *
 * Reference interface replaced, per entry point:
 *   ComputeGraph (crates/ipu-codegen/src/graph.rs:209-515):
 *     ipus_graph_host_input      graph.rs:278-284   ComputeGraph::host_input
 *     ipus_graph_parameter       graph.rs:286-292   ComputeGraph::parameter
 *     ipus_graph_value_sequence  graph.rs:294-313   ComputeGraph::value_sequence
 *     ipus_graph_gemm            graph.rs:315-326   gemm / gemm_with_options
 *     ipus_graph_gelu            graph.rs:328-330   gelu
 *     ipus_graph_add             graph.rs:332-334   add (numpy broadcasting)
 *     ipus_graph_split_heads     graph.rs:336-343   split_heads
 *     ipus_graph_flash_attention graph.rs:345-362   flash_attention_with_options
 *     ipus_graph_repeat_begin/_end graph.rs:382-472 repeat (closure body)
 *     ipus_graph_set_outputs     graph.rs:474-479   set_outputs
 *     ipus_graph_value_shape     graph.rs:270-272   value_shape
 *   Graph-level extensions for the layout chain (no reference op: the
 *   reference inserts rearranges during mid lowering, mid.rs:3553-3642):
 *     ipus_graph_transpose, ipus_graph_rearrange, ipus_graph_reduce_rows
 *   build_package (crates/ipu-codegen/src/package.rs:532-538):
 *     ipus_build_package(graph, config) -> package (launch plan + bindings;
 *     CompiledPackage, package.rs:108-145)
 *   HostSession (crates/ipu-driver/src/lib.rs:1341-1600; invoke "run",
 *   crates/ipu-tests/src/main.rs:1523-1561):
 *     ipus_session_create / _write / _run / _read
 *
 * Errors: graph calls return IPUS_ERROR_GRAPH with the GraphError message
 * (graph.rs:221-245) in ipus_last_error(); build errors return
 * IPUS_ERROR_BUILD.
 */
#ifndef IPUS_GRAPH_H
#define IPUS_GRAPH_H

#include <stddef.h>
#include <stdint.h>

#include "ipus.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ipus_graph ipus_graph;
typedef uint32_t ipus_value;    /* ValueId */
typedef uint32_t ipus_sequence; /* ValueSequenceId */

#define IPUS_MAX_RANK 8

/* Precisions (crates/ipu-codegen/src/operator.rs:14-21). */
#define IPUS_PRECISION_F16 1
#define IPUS_PRECISION_F32 2

/* Physical orders of a stored tensor (ElementOrder, layout.rs:5-45).  The
 * first four are also the orders ipus_graph_rearrange produces; the others
 * occur only as declared input formats. */
#define IPUS_ORDER_AMP_LEFT 0
#define IPUS_ORDER_AMP_TRANSPOSED_RIGHT 1
#define IPUS_ORDER_BLOCK_MAJOR 2
#define IPUS_ORDER_ROW_MAJOR 3
#define IPUS_ORDER_AMP_OUTPUT 4
#define IPUS_ORDER_AMP_TRANSPOSED_LEFT 5
#define IPUS_ORDER_AMP_TRANSPOSED_OUTPUT 6
#define IPUS_ORDER_BLOCK_MAJOR_TRANSPOSED 7

int ipus_graph_create(ipus_graph **out);
int ipus_graph_destroy(ipus_graph *graph);

int ipus_graph_host_input(ipus_graph *graph, const char *name, const uint32_t *dims, int rank,
                          ipus_value *out);
int ipus_graph_parameter(ipus_graph *graph, const char *name, const uint32_t *dims, int rank,
                         ipus_value *out);
int ipus_graph_value_sequence(ipus_graph *graph, const char *name, const ipus_value *values,
                              int count, ipus_sequence *out);
int ipus_graph_gemm(ipus_graph *graph, ipus_value left, ipus_value right, int transpose_left,
                    int transpose_right, ipus_value *out);
int ipus_graph_gelu(ipus_graph *graph, ipus_value input, ipus_value *out);
int ipus_graph_add(ipus_graph *graph, ipus_value left, ipus_value right, ipus_value *out);
int ipus_graph_split_heads(ipus_graph *graph, ipus_value input, uint32_t heads, ipus_value *out);
/* has_scale = 0: AttentionScale::InverseSqrtQueryWidth; otherwise
 * AttentionScale::ValueBits(scale_bits) (must be finite and positive). */
int ipus_graph_flash_attention(ipus_graph *graph, ipus_value query, ipus_value key,
                               ipus_value value, int causal, int has_scale, uint32_t scale_bits,
                               ipus_value *out);
/* Extensions: logical transpose of the last two axes; a physical re-layout
 * (same logical tensor, stored in `order`); row sums over the last axis with
 * fp32 accumulation (result F32, shape without the last axis). */
int ipus_graph_transpose(ipus_graph *graph, ipus_value input, ipus_value *out);
int ipus_graph_rearrange(ipus_graph *graph, ipus_value input, int order, uint32_t row_block,
                         uint32_t column_block, ipus_value *out);
int ipus_graph_reduce_rows(ipus_graph *graph, ipus_value input, ipus_value *out);

/* Structured repeat.  Between begin and end, graph calls add operations to
 * the body region.  `arguments` receives carried, invariant then iterated
 * argument values (RepeatArguments, graph.rs:196-201). */
int ipus_graph_repeat_begin(ipus_graph *graph, uint32_t count, const ipus_value *carried,
                            int carried_count, const ipus_value *invariants, int invariant_count,
                            const ipus_sequence *iterated, int iterated_count,
                            ipus_value *arguments);
int ipus_graph_repeat_end(ipus_graph *graph, const ipus_value *yields, int yield_count,
                          ipus_value *results);
/* Discards the innermost open body (the closure returned an error). */
int ipus_graph_repeat_abort(ipus_graph *graph);

int ipus_graph_set_outputs(ipus_graph *graph, const ipus_value *values, int count);
int ipus_graph_value_shape(const ipus_graph *graph, ipus_value value, uint32_t *dims,
                           int capacity, int *rank);
int ipus_graph_operation_count(const ipus_graph *graph, int *count);

/* ---- package ---- */

/* One tiled axis of a tensor layout: AxisTiling (layout.rs:140-175).
 * `axis` counts from the start (from_end = 0) or, from 1, from the end
 * (from_end = 1), as TensorAxis::FromStart / FromEnd (layout.rs:115-131).
 * Zero-valued padding_groups, padding_multiple and shard_padding_multiple
 * take AxisTiling::new's defaults (1, block_size, 1); tile_stride 0 packs the
 * axis after the replicas and the preceding axes (axis_strides,
 * layout.rs:234-251). */
typedef struct ipus_axis_tiling {
  int from_end;
  uint32_t axis;
  uint32_t partitions;
  uint32_t padding_groups;
  uint32_t block_size;
  uint32_t padding_multiple;
  uint32_t shard_padding_multiple;
  int zero_padding; /* Padding::Zero (1) or Padding::Reject (0) */
  uint32_t tile_stride;
} ipus_axis_tiling;

#define IPUS_MAX_TILED_AXES 4

/* TensorFormat{precision, layout} (layout.rs:808-811) of a host-bound
 * tensor: the element order inside every shard (row_block / column_block for
 * the block-major orders) and the TensorTiling (layout.rs:205-210) that cuts
 * the tensor into tile_count shards.  The host bytes of such a tensor are
 * the shards' storage in logical tile order, each padded per its tiling, as
 * CompiledTensor::binding lays out the reference's binding file
 * (package.rs:2101-2137).  axis_count = 0 with tile_count = replicas = 1 is
 * one unsharded tensor in `order`.  AMP and block-major orders need F16. */
typedef struct ipus_tensor_format {
  int precision;
  int order;
  uint32_t row_block, column_block;
  uint32_t tile_count, replicas;
  int axis_count;
  ipus_axis_tiling axes[IPUS_MAX_TILED_AXES];
} ipus_tensor_format;

/* One entry of PipelineConfig's inputs (config.rs:310-320): with_input
 * (automatic = 0: the host writes `format`'s bytes and build_package plans
 * their conversion) or with_automatic_input (automatic = 1: only the
 * precision is fixed; the input is row-major). */
typedef struct ipus_input_format {
  ipus_value value;
  int automatic;
  ipus_tensor_format format;
} ipus_input_format;

typedef struct ipus_package_config {
  int compute_precision;    /* IPUS_PRECISION_F16 (default) or _F32 */
  int attention_output_f16; /* 0: F32 attention output (reference), 1: F16 */
  int input_format_count;   /* entries in input_formats (inputs not named are
                               row-major at the compute precision) */
  const ipus_input_format *input_formats;
} ipus_package_config;

typedef struct ipus_package ipus_package;

typedef struct ipus_tensor_info {
  const char *name;
  uint32_t value;
  int rank;
  uint32_t dims[IPUS_MAX_RANK];
  int precision;
  int order;
  uint32_t row_block, column_block;
  uint64_t bytes;      /* bytes the host writes or reads (all shards) */
  uint32_t shards;     /* tiles of a declared tiled format, else 1 */
} ipus_tensor_info;

int ipus_build_package(const ipus_graph *graph, const ipus_package_config *config,
                       ipus_package **out);
int ipus_package_destroy(ipus_package *package);
int ipus_package_input_count(const ipus_package *package, int *count);
int ipus_package_input_info(const ipus_package *package, int index, ipus_tensor_info *info);
int ipus_package_output_count(const ipus_package *package, int *count);
int ipus_package_output_info(const ipus_package *package, int index, ipus_tensor_info *info);
/* Launch plan inspection: one ComputeStep per entry. */
int ipus_package_step_count(const ipus_package *package, int *count);
int ipus_package_step(const ipus_package *package, int index, const char **symbol,
                      int *input_count, int *scalar_count, const uint32_t **scalars);
/* Bytes of the intermediate arena (lifetime-packed, replaces SRAM placement). */
int ipus_package_arena_bytes(const ipus_package *package, uint64_t *bytes);
/* Storage precision chosen for a graph value (CompiledPackage::precisions). */
int ipus_package_value_precision(const ipus_package *package, ipus_value value, int *precision);

/* ---- session: device buffers for one package ---- */
typedef struct ipus_session ipus_session;
/* The session borrows context and package: both must outlive it.  One
 * session is used from one thread at a time (HostSession's contract). */
int ipus_session_create(ipus_context *context, const ipus_package *package, ipus_session **out);
/* Releases the session even after a device error; returns the first error. */
int ipus_session_destroy(ipus_session *session);
/* Binding names: the graph input names; outputs are "output.<i>". */
int ipus_session_write(ipus_session *session, const char *name, const void *host, size_t bytes);
int ipus_session_read(ipus_session *session, const char *name, void *host, size_t bytes);
int ipus_session_tensor_pointer(ipus_session *session, const char *name, void **device_pointer);
/* Enqueues every step on the context stream (asynchronous). */
int ipus_session_run(ipus_session *session);
/* Records the package's launches on the context stream into a HIP graph;
 * every later ipus_session_run replays it with one hipGraphLaunch (the
 * buffers are the session's, so ipus_session_write between runs feeds the
 * replay).  The role of the reference's precompiled device program
 * (HostSession runs, crates/ipu-driver/src/lib.rs:1341-1600) for
 * launch-bound packages; no reference function of its own.  Every step is
 * a kernel (no memset nodes).  A second call is a no-op. */
int ipus_session_capture(ipus_session *session);

#ifdef __cplusplus
}
#endif
#endif /* IPUS_GRAPH_H */

// ComputeGraph, build_package and the session executor of libipus.
//
// The graph mirrors crates/ipu-codegen/src/graph.rs: structured SSA with
// globally unique value ids, shape inference at construction
// (graph.rs:662-777) and the same GraphError cases (graph.rs:221-245).
//
// build_package replaces the reference's mid/low lowering (mid.rs, low.rs),
// placement (place.rs) and emission (emit.rs) with a GPU plan:
//   1. precision and layout selection per value (row-major storage; fp16
//      compute by default; attention output F32 as in mid.rs:2064-2067;
//      Cast / Rearrange steps inserted at format boundaries, as ensure_format
//      does at mid.rs:3553-3642);
//   2. one ComputeStep{symbol, output, inputs, u32 scalars} per kernel launch,
//      the same record the reference materializes per tile
//      (kernel.rs:818-865), executed through the kernel ABI registry;
//   3. structured repeats unrolled into the step list with the iterated
//      values' buffers substituted per iteration (the role of RepeatPointer,
//      crates/ipu-target/src/program.rs:29-53);
//   4. lifetime-packed offsets for every intermediate value inside one arena
//      buffer (the role of SRAM placement, place.rs:75).
#include "../../include/ipus_graph.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "internal.h"
#include "kernels.h"
#include "tiling.h"

using namespace ipus;

namespace {

using Shape = std::vector<uint32_t>;

enum class OpKind {
  Gemm,
  Gelu,
  Add,
  SplitHeads,
  FlashAttention,
  Repeat,
  Transpose,
  Rearrange,
  ReduceRows
};

struct Region;

struct Operation {
  uint32_t id = 0;
  OpKind kind = OpKind::Gemm;
  std::vector<uint32_t> inputs;
  std::vector<uint32_t> results;
  // options
  bool transpose_left = false, transpose_right = false;
  uint32_t heads = 0;
  bool causal = false;
  bool has_scale = false;  // AttentionScale::ValueBits vs InverseSqrtQueryWidth
  uint32_t scale_bits = 0;
  int order = IPUS_ORDER_ROW_MAJOR;
  uint32_t row_block = 0, column_block = 0;
  // Repeat
  uint32_t count = 0;
  size_t carried = 0, invariants = 0;
  std::vector<uint32_t> iterated;  // sequence ids
  std::shared_ptr<Region> body;
};

struct Region {
  std::vector<uint32_t> arguments;
  std::vector<Operation> operations;
  std::vector<uint32_t> yields;
  std::set<uint32_t> values;  // values visible in this region
};

struct InputDecl {
  std::string name;
  bool parameter = false;
  uint32_t value = 0;
};

struct Sequence {
  uint32_t id;
  std::string name;
  std::vector<uint32_t> values;
};

struct OpenRepeat {
  uint32_t count;
  std::vector<uint32_t> carried_inputs, invariant_inputs, iterated;
  std::shared_ptr<Region> body;
};

int graph_error(const std::string& message) {
  return fail(IPUS_ERROR_GRAPH, "%s", message.c_str());
}

// graph.rs:755-777
bool broadcast(const Shape& left, const Shape& right, Shape* out, std::string* error) {
  const size_t rank = std::max(left.size(), right.size());
  out->assign(rank, 1);
  for (size_t i = 0; i < rank; ++i) {
    const uint32_t l = i + left.size() >= rank ? left[i + left.size() - rank] : 1;
    const uint32_t r = i + right.size() >= rank ? right[i + right.size() - rank] : 1;
    if (l != r && l != 1 && r != 1) {
      *error = "operation has invalid shapes: dimensions " + std::to_string(l) + " and " +
               std::to_string(r) + " cannot be broadcast";
      return false;
    }
    (*out)[i] = std::max(l, r);
  }
  return true;
}

uint64_t elements(const Shape& s) {
  uint64_t n = 1;
  for (uint32_t d : s) n *= d;
  return n;
}

// Product of every axis but the last `trailing` ones (the matrix or row
// count).  Computed from the axes themselves, so a zero-extent matrix axis
// leaves it well defined where elements / (rows * columns) would divide by 0.
uint64_t outer_count(const Shape& s, size_t trailing) {
  uint64_t n = 1;
  for (size_t i = 0; i + trailing < s.size(); ++i) n *= s[i];
  return n;
}

bool fits_u32(uint64_t v) { return v <= 0xffffffffull; }

}  // namespace

struct ipus_graph {
  std::vector<InputDecl> inputs;
  std::vector<Sequence> sequences;
  Region root;
  std::vector<uint32_t> outputs;
  std::map<uint32_t, Shape> shapes;
  uint32_t next_operation = 0, next_value = 0;
  std::vector<OpenRepeat> open;  // innermost last

  Region& current() { return open.empty() ? root : *open.back().body; }

  int validate(const std::vector<uint32_t>& values) {
    const Region& r = current();
    for (uint32_t v : values)
      if (!r.values.count(v))
        return graph_error("value ValueId(" + std::to_string(v) +
                           ") is not available in this operation list");
    return 0;
  }

  uint32_t new_value(const Shape& shape) {
    const uint32_t v = next_value++;
    shapes[v] = shape;
    current().values.insert(v);
    return v;
  }

  int infer(const Operation& op, Shape* out) {
    std::string error;
    auto in = [&](size_t i) -> const Shape& { return shapes[op.inputs[i]]; };
    switch (op.kind) {
      case OpKind::Gemm: {  // graph.rs:674-694
        const Shape &l = in(0), &r = in(1);
        if (l.size() < 2 || r.size() < 2)
          return graph_error("operation has invalid shapes: GEMM inputs must have rank at least two");
        const uint32_t rows = l[l.size() - 2 + (op.transpose_left ? 1 : 0)];
        const uint32_t linner = l[l.size() - 1 - (op.transpose_left ? 1 : 0)];
        const uint32_t rinner = r[r.size() - 2 + (op.transpose_right ? 1 : 0)];
        const uint32_t cols = r[r.size() - 1 - (op.transpose_right ? 1 : 0)];
        if (linner != rinner)
          return graph_error("operation has invalid shapes: GEMM inner dimensions do not match");
        Shape lb(l.begin(), l.end() - 2), rb(r.begin(), r.end() - 2);
        if (!broadcast(lb, rb, out, &error)) return graph_error(error);
        out->push_back(rows);
        out->push_back(cols);
        return 0;
      }
      case OpKind::Gelu:
        *out = in(0);
        return 0;
      case OpKind::Add:
        if (!broadcast(in(0), in(1), out, &error)) return graph_error(error);
        return 0;
      case OpKind::SplitHeads: {  // graph.rs:699-720
        const Shape& s = in(0);
        if (s.size() != 3 || op.heads == 0)
          return graph_error(
              "operation has invalid shapes: split_heads requires nonzero heads and [batch, rows, "
              "channels] input");
        if (s[2] % op.heads != 0)
          return graph_error(
              "operation has invalid shapes: split_heads channels must be divisible by heads");
        const uint64_t streams = (uint64_t)s[0] * op.heads;
        if (streams > 0xffffffffull)
          return graph_error("operation has invalid shapes: split_heads stream count overflow");
        *out = {(uint32_t)streams, s[1], s[2] / op.heads};
        return 0;
      }
      case OpKind::FlashAttention: {  // graph.rs:721-748
        const Shape &q = in(0), &k = in(1), &v = in(2);
        if (q.size() < 2 || k.size() < 2 || v.size() < 2)
          return graph_error(
              "operation has invalid shapes: FlashAttention inputs must have rank at least two");
        if (q.back() != k.back() || k[k.size() - 2] != v[v.size() - 2])
          return graph_error(
              "operation has invalid shapes: FlashAttention head or sequence dimensions do not "
              "match");
        if (op.has_scale) {
          float scale;
          memcpy(&scale, &op.scale_bits, 4);
          if (!std::isfinite(scale) || scale <= 0.0f)
            return graph_error(
                "operation has invalid shapes: attention scale must be finite and positive");
        }
        Shape qb(q.begin(), q.end() - 2), kb(k.begin(), k.end() - 2), vb(v.begin(), v.end() - 2);
        Shape kvb;
        if (!broadcast(kb, vb, &kvb, &error)) return graph_error(error);
        if (!broadcast(qb, kvb, out, &error)) return graph_error(error);
        out->push_back(q[q.size() - 2]);
        out->push_back(v.back());
        return 0;
      }
      case OpKind::Transpose: {
        const Shape& s = in(0);
        if (s.size() < 2)
          return graph_error("operation has invalid shapes: transpose requires rank at least two");
        *out = s;
        std::swap((*out)[s.size() - 1], (*out)[s.size() - 2]);
        return 0;
      }
      case OpKind::Rearrange: {
        const Shape& s = in(0);
        if (op.order != IPUS_ORDER_ROW_MAJOR && s.size() < 2)
          return graph_error("operation has invalid shapes: matrix storage requires rank at least two");
        *out = s;
        return 0;
      }
      case OpKind::ReduceRows: {
        const Shape& s = in(0);
        if (s.empty())
          return graph_error("operation has invalid shapes: reduce_rows requires rank at least one");
        *out = Shape(s.begin(), s.end() - 1);
        return 0;
      }
      case OpKind::Repeat:
        return graph_error(
            "operation has invalid shapes: repeat result shapes are defined by carried values");
    }
    return graph_error("unknown operation");
  }

  int add_op(Operation op, uint32_t* out) {
    if (int e = validate(op.inputs)) return e;
    Shape shape;
    if (int e = infer(op, &shape)) return e;
    op.id = next_operation++;
    const uint32_t v = new_value(shape);
    op.results = {v};
    current().operations.push_back(std::move(op));
    if (out) *out = v;
    return 0;
  }
};

namespace {

int check_graph(const ipus_graph* g) {
  if (!g) return fail(IPUS_ERROR_INVALID_ARGUMENT, "graph is null");
  return 0;
}

int add_input(ipus_graph* g, const char* name, const uint32_t* dims, int rank, bool parameter,
              ipus_value* out) {
  if (int e = check_graph(g)) return e;
  if (!name || !*name) return graph_error("graph name must not be empty");
  if (rank < 0 || rank > IPUS_MAX_RANK || (rank > 0 && !dims))
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "rank must be 0..%d", IPUS_MAX_RANK);
  if (!g->open.empty())
    return fail(IPUS_ERROR_GRAPH, "graph inputs must be declared outside repeat bodies");
  for (const auto& i : g->inputs)
    if (i.name == name) return fail(IPUS_ERROR_GRAPH, "graph input %s is declared twice", name);
  Shape shape(dims, dims + rank);
  const uint32_t v = g->new_value(shape);
  g->inputs.push_back({name, parameter, v});
  if (out) *out = v;
  return 0;
}

}  // namespace

extern "C" int ipus_graph_create(ipus_graph** out) {
  if (!out) return fail(IPUS_ERROR_INVALID_ARGUMENT, "out is null");
  *out = new ipus_graph();
  return 0;
}

extern "C" int ipus_graph_destroy(ipus_graph* g) {
  delete g;
  return 0;
}

extern "C" int ipus_graph_host_input(ipus_graph* g, const char* name, const uint32_t* dims,
                                     int rank, ipus_value* out) {
  return add_input(g, name, dims, rank, false, out);
}

extern "C" int ipus_graph_parameter(ipus_graph* g, const char* name, const uint32_t* dims,
                                    int rank, ipus_value* out) {
  return add_input(g, name, dims, rank, true, out);
}

extern "C" int ipus_graph_value_sequence(ipus_graph* g, const char* name, const ipus_value* values,
                                         int count, ipus_sequence* out) {
  if (int e = check_graph(g)) return e;
  if (!name || !*name) return graph_error("graph name must not be empty");
  if (count < 0 || (count > 0 && !values)) return fail(IPUS_ERROR_INVALID_ARGUMENT, "bad values");
  std::vector<uint32_t> vs(values, values + count);
  if (int e = g->validate(vs)) return e;
  for (int i = 1; i < count; ++i)
    if (g->shapes[vs[(size_t)i]] != g->shapes[vs[0]])
      return graph_error("value sequence entry " + std::to_string(i) +
                         " has a different shape from its first entry");
  const uint32_t id = (uint32_t)g->sequences.size();
  g->sequences.push_back({id, name, vs});
  if (out) *out = id;
  return 0;
}

extern "C" int ipus_graph_gemm(ipus_graph* g, ipus_value l, ipus_value r, int tl, int tr,
                               ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::Gemm;
  op.inputs = {l, r};
  op.transpose_left = tl != 0;
  op.transpose_right = tr != 0;
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_gelu(ipus_graph* g, ipus_value in, ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::Gelu;
  op.inputs = {in};
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_add(ipus_graph* g, ipus_value l, ipus_value r, ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::Add;
  op.inputs = {l, r};
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_split_heads(ipus_graph* g, ipus_value in, uint32_t heads,
                                      ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::SplitHeads;
  op.inputs = {in};
  op.heads = heads;
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_flash_attention(ipus_graph* g, ipus_value q, ipus_value k, ipus_value v,
                                          int causal, int has_scale, uint32_t scale_bits,
                                          ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::FlashAttention;
  op.inputs = {q, k, v};
  op.causal = causal != 0;
  op.has_scale = has_scale != 0;
  op.scale_bits = scale_bits;
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_transpose(ipus_graph* g, ipus_value in, ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::Transpose;
  op.inputs = {in};
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_rearrange(ipus_graph* g, ipus_value in, int order, uint32_t row_block,
                                    uint32_t column_block, ipus_value* out) {
  if (int e = check_graph(g)) return e;
  if (order < IPUS_ORDER_AMP_LEFT || order > IPUS_ORDER_ROW_MAJOR)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "unknown order %d", order);
  if (order == IPUS_ORDER_BLOCK_MAJOR &&
      (row_block == 0 || column_block == 0 || row_block % 16 != 0))
    return fail(IPUS_ERROR_INVALID_ARGUMENT,
                "block-major storage needs nonzero blocks with row_block a multiple of 16");
  Operation op;
  op.kind = OpKind::Rearrange;
  op.inputs = {in};
  op.order = order;
  op.row_block = row_block;
  op.column_block = column_block;
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_reduce_rows(ipus_graph* g, ipus_value in, ipus_value* out) {
  if (int e = check_graph(g)) return e;
  Operation op;
  op.kind = OpKind::ReduceRows;
  op.inputs = {in};
  return g->add_op(std::move(op), out);
}

extern "C" int ipus_graph_repeat_begin(ipus_graph* g, uint32_t count, const ipus_value* carried,
                                       int carried_count, const ipus_value* invariants,
                                       int invariant_count, const ipus_sequence* iterated,
                                       int iterated_count, ipus_value* arguments) {
  if (int e = check_graph(g)) return e;
  if (carried_count < 0 || invariant_count < 0 || iterated_count < 0)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "negative counts");
  if (count == 0) return graph_error("repeat count must be nonzero");
  std::vector<uint32_t> c(carried, carried + carried_count);
  std::vector<uint32_t> inv(invariants, invariants + invariant_count);
  std::vector<uint32_t> it(iterated, iterated + iterated_count);
  if (int e = g->validate(c)) return e;
  if (int e = g->validate(inv)) return e;
  for (uint32_t s : it) {
    if (s >= g->sequences.size())
      return graph_error("value sequence ValueSequenceId(" + std::to_string(s) + ") does not exist");
    if (g->sequences[s].values.size() < count)
      return graph_error("value sequence ValueSequenceId(" + std::to_string(s) + ") has " +
                         std::to_string(g->sequences[s].values.size()) + " entries for " +
                         std::to_string(count) + " iterations");
  }
  std::vector<Shape> arg_shapes;
  for (uint32_t v : c) arg_shapes.push_back(g->shapes[v]);
  for (uint32_t v : inv) arg_shapes.push_back(g->shapes[v]);
  for (uint32_t s : it) arg_shapes.push_back(g->shapes[g->sequences[s].values[0]]);
  OpenRepeat rep;
  rep.count = count;
  rep.carried_inputs = c;
  rep.invariant_inputs = inv;
  rep.iterated = it;
  rep.body = std::make_shared<Region>();
  g->open.push_back(rep);
  for (size_t i = 0; i < arg_shapes.size(); ++i) {
    const uint32_t v = g->new_value(arg_shapes[i]);
    g->open.back().body->arguments.push_back(v);
    if (arguments) arguments[i] = v;
  }
  return 0;
}

extern "C" int ipus_graph_repeat_end(ipus_graph* g, const ipus_value* yields, int yield_count,
                                     ipus_value* results) {
  if (int e = check_graph(g)) return e;
  if (g->open.empty()) return fail(IPUS_ERROR_GRAPH, "no repeat body is open");
  std::vector<uint32_t> ys(yields, yields + (yield_count > 0 ? yield_count : 0));
  OpenRepeat& rep = g->open.back();
  // A failed repeat discards its body, as the Rust builder's error return
  // drops the region (graph.rs:440-452).
  auto abort_with = [&](int status) {
    g->open.pop_back();
    return status;
  };
  if (ys.size() != rep.carried_inputs.size())
    return abort_with(graph_error("repeat body yielded " + std::to_string(ys.size()) +
                                  " values for " + std::to_string(rep.carried_inputs.size()) +
                                  " carried values"));
  if (int e = g->validate(ys)) return abort_with(e);
  for (size_t i = 0; i < ys.size(); ++i)
    if (g->shapes[ys[i]] != g->shapes[rep.carried_inputs[i]])
      return abort_with(graph_error("repeat yield " + std::to_string(i) +
                                    " does not have the shape of carried value " +
                                    std::to_string(i)));
  OpenRepeat done = rep;
  done.body->yields = ys;
  g->open.pop_back();
  Operation op;
  op.kind = OpKind::Repeat;
  op.id = g->next_operation++;
  op.count = done.count;
  op.carried = done.carried_inputs.size();
  op.invariants = done.invariant_inputs.size();
  op.iterated = done.iterated;
  op.body = done.body;
  op.inputs = done.carried_inputs;
  op.inputs.insert(op.inputs.end(), done.invariant_inputs.begin(), done.invariant_inputs.end());
  for (size_t i = 0; i < ys.size(); ++i) {
    const uint32_t v = g->new_value(g->shapes[done.carried_inputs[i]]);
    op.results.push_back(v);
    if (results) results[i] = v;
  }
  g->current().operations.push_back(std::move(op));
  return 0;
}

extern "C" int ipus_graph_repeat_abort(ipus_graph* g) {
  if (int e = check_graph(g)) return e;
  if (g->open.empty()) return fail(IPUS_ERROR_GRAPH, "no repeat body is open");
  g->open.pop_back();
  return 0;
}

extern "C" int ipus_graph_set_outputs(ipus_graph* g, const ipus_value* values, int count) {
  if (int e = check_graph(g)) return e;
  if (!g->open.empty()) return fail(IPUS_ERROR_GRAPH, "a repeat body is still open");
  std::vector<uint32_t> vs(values, values + (count > 0 ? count : 0));
  if (int e = g->validate(vs)) return e;
  g->outputs = vs;
  return 0;
}

extern "C" int ipus_graph_value_shape(const ipus_graph* g, ipus_value v, uint32_t* dims,
                                      int capacity, int* rank) {
  if (int e = check_graph(g)) return e;
  auto it = g->shapes.find(v);
  if (it == g->shapes.end()) return fail(IPUS_ERROR_GRAPH, "unknown value %u", v);
  if (rank) *rank = (int)it->second.size();
  if (dims)
    for (int i = 0; i < capacity && i < (int)it->second.size(); ++i) dims[i] = it->second[(size_t)i];
  return 0;
}

extern "C" int ipus_graph_operation_count(const ipus_graph* g, int* count) {
  if (int e = check_graph(g)) return e;
  if (count) *count = (int)g->root.operations.size();
  return 0;
}

// ===========================================================================
// build_package
// ===========================================================================
namespace {

struct Storage {
  int buffer = -1;      // index into package buffers; -2 = arena
  uint64_t offset = 0;  // byte offset (arena offset for arena values)
  int precision = IPUS_PRECISION_F16;
  int order = IPUS_ORDER_ROW_MAJOR;
  uint32_t row_block = 0, column_block = 0;
  Shape shape;
  // A declared input format's host bytes (all shards, padding and replicas
  // included); 0 for a plain tensor of `shape`.
  uint64_t file_bytes = 0;
  uint32_t shards = 1;
  uint64_t bytes() const {
    if (file_bytes) return file_bytes;
    return elements(shape) * (precision == IPUS_PRECISION_F32 ? 4 : 2);
  }
};

// A plan-level value ("slot"): one materialized tensor.
struct Slot {
  Storage storage;
  int first_def = -1, last_use = -1;
  bool external = false;  // own buffer: input or output binding, or a constant
  // Bytes uploaded into the slot's buffer when a session is created (the
  // shard table of a declared input format).
  std::vector<uint8_t> constant;
};

struct Operand {
  int slot;
  uint64_t byte_offset;  // within the slot
};

struct Step {
  std::string symbol;
  Operand out;
  std::vector<Operand> ins;
  std::vector<uint32_t> scalars;
};

struct Binding {
  std::string name;
  uint32_t value;
  int slot;
};

}  // namespace

struct ipus_package {
  // deque: the planner keeps references to slots while appending new ones.
  std::deque<Slot> slots;
  std::vector<Step> steps;
  std::vector<Binding> inputs, outputs;
  std::map<uint32_t, int> precisions;
  uint64_t arena_bytes = 0;
};

namespace {

int build_error(const std::string& message) {
  return fail(IPUS_ERROR_BUILD, "%s", message.c_str());
}

// Split-K count for an fp16 GEMM on the 256 x 256 kernel: min(16, K / 1024,
// 64 / tiles), i.e. only for outputs of at most 32 tiles and K >= 6144, with
// every split keeping >= 1024 k and about 64 workgroups in all.  Below
// 32 tiles the unsplit launch runs the small-tile kernel, which beats the
// split up to K ~ 4-6k (measured, us, unsplit against split: 1024 x 1024 x
// 2048 17 / 31, 729 x 1152 x 4304 33 / 38, 512 x 512 x 4096 28 / 30) and
// loses beyond (1024 x 1024 x 8192 57 / 49, 256 x 1024 x 16384 103 / 37,
// 64 x 64 x 40000 151 / 51; 256 x 256 x 8192 33 / 32).  Returns 1 (no split)
// when the shape is outside the fast kernel's reach.
uint32_t gemm_splits(uint32_t M, uint32_t N, uint32_t K, uint64_t batches, bool tl, bool tr) {
  if (K < 6144 || K % 8 != 0 || N % 8 != 0 || (tl && M % 8 != 0)) return 1;
  const uint64_t a_span = tl ? (uint64_t)K * M * 2 : 256ull * K * 2;
  const uint64_t b_span = tr ? 256ull * K * 2 : (uint64_t)K * N * 2;
  if (a_span >= (1ull << 31) || b_span >= (1ull << 31)) return 1;
  const uint64_t tiles = (uint64_t)((M + 255) / 256) * ((N + 255) / 256) * batches;
  if (tiles == 0) return 1;  // empty output: nothing to split
  const uint64_t want = std::min<uint64_t>({16, K / 1024, 64 / tiles});
  if (want < 2) return 1;
  const uint32_t chunk = (uint32_t)gemm_f16_split_chunk(K, (uint32_t)want);
  return (K + chunk - 1) / chunk;  // every split owns some k
}

struct Builder {
  const ipus_graph& g;
  ipus_package_config cfg;
  ipus_package& pkg;
  std::map<uint32_t, int> env;  // graph value -> slot (current binding)

  int new_slot(const Shape& shape, int precision, int order = IPUS_ORDER_ROW_MAJOR,
               uint32_t rb = 0, uint32_t cb = 0) {
    Slot s;
    s.storage.shape = shape;
    s.storage.precision = precision;
    s.storage.order = order;
    s.storage.row_block = rb;
    s.storage.column_block = cb;
    pkg.slots.push_back(s);
    return (int)pkg.slots.size() - 1;
  }

  const Storage& st(int slot) const { return pkg.slots[(size_t)slot].storage; }

  void emit(const std::string& symbol, int out, std::vector<Operand> ins,
            std::vector<uint32_t> scalars, uint64_t out_offset = 0) {
    Step s;
    s.symbol = symbol;
    s.out = {out, out_offset};
    s.ins = std::move(ins);
    s.scalars = std::move(scalars);
    pkg.steps.push_back(std::move(s));
  }

  // An element-wise step over `count` elements as launches of at most
  // kChunkElements each (the count scalar is u32; values of 2^32 elements
  // and more fit in HBM).  Offsets advance by the elements already covered.
  static constexpr uint64_t kChunkElements = 1ull << 30;
  void emit_chunked(const std::string& symbol, int out, int in, uint64_t count,
                    uint64_t in_bytes, uint64_t out_bytes) {
    for (uint64_t done = 0; done < count; done += kChunkElements) {
      const uint64_t n = std::min(kChunkElements, count - done);
      emit(symbol, out, {{in, done * in_bytes}}, {(uint32_t)n}, done * out_bytes);
    }
  }

  // Returns a slot holding `slot`'s tensor as row-major with `precision`,
  // inserting Rearrange / Cast steps as needed (ensure_format, mid.rs:3553).
  int ensure(int slot, int precision) {
    int cur = slot;
    const Storage s = st(cur);
    if (s.order != IPUS_ORDER_ROW_MAJOR) {
      if (s.precision != IPUS_PRECISION_F16) return -1;
      const Shape& sh = s.shape;
      const uint32_t rows = sh[sh.size() - 2], cols = sh[sh.size() - 1];
      const uint64_t matrices = outer_count(sh, 2);
      if (!fits_u32(matrices)) return -1;
      const int out = new_slot(sh, s.precision);
      emit("ipu_stack_rearrange_to_row_major_f16", out, {{cur, 0}},
           {(uint32_t)s.order, s.row_block, s.column_block, (uint32_t)matrices, rows, cols});
      cur = out;
    }
    if (st(cur).precision != precision) {
      const int out = new_slot(st(cur).shape, precision);
      const uint64_t in_bytes = st(cur).precision == IPUS_PRECISION_F32 ? 4 : 2;
      const uint64_t out_bytes = precision == IPUS_PRECISION_F32 ? 4 : 2;
      emit_chunked(precision == IPUS_PRECISION_F16 ? "ipu_stack_cast_f32_f16"
                                                   : "ipu_stack_cast_f16_f32",
                   out, cur, elements(st(cur).shape), in_bytes, out_bytes);
      cur = out;
    }
    return cur;
  }

  int lower_ops(const std::vector<Operation>& ops) {
    for (const Operation& op : ops)
      if (int e = lower(op)) return e;
    return 0;
  }

  int lower(const Operation& op) {
    auto slot_of = [&](uint32_t v) { return env.at(v); };
    const int cp = cfg.compute_precision;
    switch (op.kind) {
      case OpKind::Gemm: {
        const int l = ensure(slot_of(op.inputs[0]), cp), r = ensure(slot_of(op.inputs[1]), cp);
        if (l < 0 || r < 0) return build_error("GEMM operand format is not convertible");
        const Shape &ls = st(l).shape, &rs = st(r).shape;
        const Shape& os = g.shapes.at(op.results[0]);
        const uint32_t M = os[os.size() - 2], N = os[os.size() - 1];
        const uint32_t K = ls[ls.size() - 1 - (op.transpose_left ? 1 : 0)];
        const int out = new_slot(os, cp);
        env[op.results[0]] = out;
        const uint64_t esz = cp == IPUS_PRECISION_F32 ? 4 : 2;
        const Shape lb(ls.begin(), ls.end() - 2), rb(rs.begin(), rs.end() - 2);
        const Shape ob(os.begin(), os.end() - 2);
        const uint64_t lm = (uint64_t)ls[ls.size() - 2] * ls[ls.size() - 1];
        const uint64_t rm = (uint64_t)rs[rs.size() - 2] * rs[rs.size() - 1];
        const uint64_t batches = elements(ob);
        const char* sym = cp == IPUS_PRECISION_F32 ? "ipu_stack_gemm_f32" : "ipu_stack_gemm_f16";
        const uint64_t lcount = elements(lb), rcount = elements(rb);
        // graph.rs broadcasts extents 0 and 1 to 1 (max), so an operand with
        // an empty batch axis can meet a non-empty result: there is no data
        // to read for it.
        if (batches > 0 && (lcount == 0 || rcount == 0))
          return build_error("GEMM operand with an empty batch axis broadcast to a non-empty result");
        // One launch when each operand is either fully batched or a single
        // matrix; otherwise one launch per output batch.
        // The batch strides are u32 scalars: a batched operand whose matrix
        // holds 2^32 elements or more takes the per-batch path below.
        const bool strides_fit = (lcount == 1 || fits_u32(lm)) && (rcount == 1 || fits_u32(rm));
        if ((lcount == batches || lcount == 1) && (rcount == batches || rcount == 1) &&
            batches <= 65535 && strides_fit) {
          if (cp == IPUS_PRECISION_F16) {
            const uint32_t splits = gemm_splits(M, N, K, batches, op.transpose_left,
                                                op.transpose_right);
            if (splits > 1) {
              // Few output tiles, long K: split K over more workgroups into
              // fp32 partials (an arena value), then sum and round once.
              const int parts = new_slot({splits * (uint32_t)batches, M, N}, IPUS_PRECISION_F32);
              emit("ipu_stack_gemm_f16_split", parts, {{l, 0}, {r, 0}},
                   {(uint32_t)batches, M, N, K, op.transpose_left ? 1u : 0u,
                    op.transpose_right ? 1u : 0u, (uint32_t)(lcount == 1 ? 0 : lm),
                    (uint32_t)(rcount == 1 ? 0 : rm), splits});
              // At most 32 output tiles of 256 x 256 (gemm_splits), so the
              // element count fits its u32 scalar.
              emit("ipu_stack_reduce_splits_f16", out, {{parts, 0}},
                   {splits, (uint32_t)(batches * M * N), 0u});
              return 0;
            }
          }
          emit(sym, out, {{l, 0}, {r, 0}},
               {(uint32_t)batches, M, N, K, op.transpose_left ? 1u : 0u,
                op.transpose_right ? 1u : 0u, (uint32_t)(lcount == 1 ? 0 : lm),
                (uint32_t)(rcount == 1 ? 0 : rm)});
        } else {
          for (uint64_t b = 0; b < batches; ++b) {
            // Decode b over ob and map into each operand's broadcast batch.
            uint64_t rem = b, lo = 0, ro = 0, lstride = 1, rstride = 1;
            for (int ax = (int)ob.size() - 1; ax >= 0; --ax) {
              const uint64_t c = rem % ob[(size_t)ax];
              rem /= ob[(size_t)ax];
              const int la = ax - (int)(ob.size() - lb.size());
              const int ra = ax - (int)(ob.size() - rb.size());
              if (la >= 0) {
                if (lb[(size_t)la] != 1) lo += c * lstride;
                lstride *= lb[(size_t)la];
              }
              if (ra >= 0) {
                if (rb[(size_t)ra] != 1) ro += c * rstride;
                rstride *= rb[(size_t)ra];
              }
            }
            emit(sym, out, {{l, lo * lm * esz}, {r, ro * rm * esz}},
                 {1u, M, N, K, op.transpose_left ? 1u : 0u, op.transpose_right ? 1u : 0u, 0u, 0u},
                 b * (uint64_t)M * N * esz);
          }
        }
        return 0;
      }
      case OpKind::Gelu: {
        const int in = ensure(slot_of(op.inputs[0]), IPUS_PRECISION_F16);
        if (in < 0) return build_error("GELU operand format is not convertible");
        const Shape& s = st(in).shape;
        const int out = new_slot(s, IPUS_PRECISION_F16);
        env[op.results[0]] = out;
        const uint64_t n = elements(s);
        // The reference ABI needs whole half pairs (kernel.rs:1400-1413):
        // the even prefix goes through it (in launches of at most 2^30
        // elements), an odd last element through a one-element tail launch
        // of the same kernel body.
        emit_chunked("ipu_stack_gelu_tanh_approx_f16", out, in, n - n % 2, 2, 2);
        if (n % 2 == 1) emit("ipus_gelu_f16", out, {{in, (n - 1) * 2}}, {1u}, (n - 1) * 2);
        return 0;
      }
      case OpKind::Add: {
        const int l = ensure(slot_of(op.inputs[0]), cp), r = ensure(slot_of(op.inputs[1]), cp);
        if (l < 0 || r < 0) return build_error("Add operand format is not convertible");
        const Shape& os = g.shapes.at(op.results[0]);
        const int out = new_slot(os, cp);
        env[op.results[0]] = out;
        if (os.size() > 6) return build_error("Add supports rank <= 6");
        if (elements(os) > 0 && (elements(st(l).shape) == 0 || elements(st(r).shape) == 0))
          return build_error("Add operand with an empty axis broadcast to a non-empty result");
        std::vector<uint32_t> sc;
        sc.push_back((uint32_t)os.size());
        for (size_t i = 0; i < 6; ++i) sc.push_back(i < os.size() ? os[i] : 1);
        for (int which = 0; which < 2; ++which) {
          const Shape& s = st(which == 0 ? l : r).shape;
          std::vector<uint32_t> strides(6, 0);
          uint64_t stride = 1;
          for (int ax = (int)os.size() - 1; ax >= 0; --ax) {
            const int sa = ax - (int)(os.size() - s.size());
            if (sa >= 0) {
              if (s[(size_t)sa] != 1) {
                if (!fits_u32(stride)) return build_error("Add operand strides exceed u32");
                strides[(size_t)ax] = (uint32_t)stride;
              }
              stride *= s[(size_t)sa];
            }
          }
          sc.insert(sc.end(), strides.begin(), strides.end());
        }
        emit(cp == IPUS_PRECISION_F32 ? "ipu_stack_add_broadcast_f32" : "ipu_stack_add_broadcast_f16",
             out, {{l, 0}, {r, 0}}, sc);
        return 0;
      }
      case OpKind::SplitHeads: {
        const int in0 = slot_of(op.inputs[0]);
        const int in = ensure(in0, st(in0).precision);
        if (in < 0) return build_error("SplitHeads operand format is not convertible");
        const Shape& s = st(in).shape;
        const int out = new_slot(g.shapes.at(op.results[0]), st(in).precision);
        env[op.results[0]] = out;
        emit("ipu_stack_split_heads", out, {{in, 0}},
             {s[0], s[1], op.heads, s[2] / op.heads,
              st(in).precision == IPUS_PRECISION_F32 ? 4u : 2u});
        return 0;
      }
      case OpKind::FlashAttention: {
        int q = ensure(slot_of(op.inputs[0]), IPUS_PRECISION_F16);
        int k = ensure(slot_of(op.inputs[1]), IPUS_PRECISION_F16);
        int v = ensure(slot_of(op.inputs[2]), IPUS_PRECISION_F16);
        if (q < 0 || k < 0 || v < 0) return build_error("attention operand format is not convertible");
        const Shape &qs = st(q).shape, &ks = st(k).shape, &vs = st(v).shape;
        const Shape& os = g.shapes.at(op.results[0]);
        const uint64_t qstreams = outer_count(qs, 2), kstreams = outer_count(ks, 2);
        const uint64_t vstreams = outer_count(vs, 2), ostreams = outer_count(os, 2);
        if (qstreams != ostreams || kstreams != ostreams || vstreams != ostreams)
          return build_error("attention batch broadcasting is not supported by the GPU plan");
        if (!fits_u32(ostreams)) return build_error("attention stream count exceeds u32");
        const int prec = cfg.attention_output_f16 ? IPUS_PRECISION_F16 : IPUS_PRECISION_F32;
        const int out = new_slot(os, prec);
        env[op.results[0]] = out;
        emit("ipu_stack_flash_attention_online_f16", out, {{q, 0}, {k, 0}, {v, 0}},
             {(uint32_t)ostreams, qs[qs.size() - 2], ks[ks.size() - 2], qs.back(), vs.back(),
              op.scale_bits, op.causal ? 1u : 0u, cfg.attention_output_f16 ? 1u : 0u});
        return 0;
      }
      case OpKind::Transpose: {
        const int in = ensure(slot_of(op.inputs[0]), IPUS_PRECISION_F16);
        if (in < 0) return build_error("transpose operand format is not convertible");
        const Shape& s = st(in).shape;
        const uint32_t rows = s[s.size() - 2], cols = s[s.size() - 1];
        const int out = new_slot(g.shapes.at(op.results[0]), IPUS_PRECISION_F16);
        env[op.results[0]] = out;
        const uint64_t matrices = outer_count(s, 2);
        if (!fits_u32(matrices)) return build_error("transpose matrix count exceeds u32");
        emit("ipu_stack_transpose_f16", out, {{in, 0}}, {(uint32_t)matrices, rows, cols});
        return 0;
      }
      case OpKind::Rearrange: {
        int in = slot_of(op.inputs[0]);
        if (op.order == IPUS_ORDER_ROW_MAJOR) {
          in = ensure(in, st(in).precision);
          env[op.results[0]] = in;  // already row-major: alias
          return 0;
        }
        in = ensure(in, IPUS_PRECISION_F16);
        if (in < 0) return build_error("rearrange operand format is not convertible");
        const Shape& s = st(in).shape;
        const uint32_t rows = s[s.size() - 2], cols = s[s.size() - 1];
        const uint64_t matrices64 = outer_count(s, 2);
        if (!fits_u32(matrices64)) return build_error("rearrange matrix count exceeds u32");
        const uint32_t matrices = (uint32_t)matrices64;
        // Storage constraints (storage.rs:314-425): no padding at the graph
        // level, so the logical extents must fit the order's blocks.
        if (op.order == IPUS_ORDER_AMP_LEFT && cols % 16 != 0)
          return build_error("AMP-Left storage needs columns divisible by 16");
        if (op.order == IPUS_ORDER_AMP_TRANSPOSED_RIGHT && (rows % 16 != 0 || cols % 16 != 0))
          return build_error("AMP-TransposedRight storage needs rows and columns divisible by 16");
        if (op.order == IPUS_ORDER_BLOCK_MAJOR && (rows % op.row_block != 0 || cols % op.column_block != 0))
          return build_error("block-major storage needs rows and columns divisible by its blocks");
        const int out = new_slot(s, IPUS_PRECISION_F16, op.order, op.row_block, op.column_block);
        env[op.results[0]] = out;
        emit("ipu_stack_rearrange_row_major_f16", out, {{in, 0}},
             {rows, rows, (uint32_t)op.order, cols, cols, op.row_block, op.column_block, matrices});
        return 0;
      }
      case OpKind::ReduceRows: {
        int in = slot_of(op.inputs[0]);
        const Storage& s0 = st(in);
        if (!(s0.order == IPUS_ORDER_BLOCK_MAJOR && s0.precision == IPUS_PRECISION_F16 &&
              s0.shape.size() == 2))
          in = ensure(in, IPUS_PRECISION_F16);
        if (in < 0) return build_error("reduce_rows operand format is not convertible");
        const Storage& s = st(in);
        const uint64_t cols = s.shape.back();
        const uint64_t rows = outer_count(s.shape, 1);
        if (!fits_u32(rows)) return build_error("reduce_rows row count exceeds u32");
        const int out = new_slot(g.shapes.at(op.results[0]), IPUS_PRECISION_F32);
        env[op.results[0]] = out;
        emit("ipu_stack_reduce_rows_f16", out, {{in, 0}},
             {(uint32_t)rows, (uint32_t)cols, (uint32_t)s.order, s.row_block, s.column_block});
        return 0;
      }
      case OpKind::Repeat: {
        std::vector<int> carried;
        for (size_t i = 0; i < op.carried; ++i) carried.push_back(slot_of(op.inputs[i]));
        std::vector<int> inv;
        for (size_t i = 0; i < op.invariants; ++i) inv.push_back(slot_of(op.inputs[op.carried + i]));
        const Region& body = *op.body;
        for (uint32_t it = 0; it < op.count; ++it) {
          size_t a = 0;
          for (int c : carried) env[body.arguments[a++]] = c;
          for (int c : inv) env[body.arguments[a++]] = c;
          for (uint32_t seq : op.iterated)
            env[body.arguments[a++]] = slot_of(g.sequences[seq].values[it]);
          if (int e = lower_ops(body.operations)) return e;
          for (size_t y = 0; y < carried.size(); ++y) carried[y] = slot_of(body.yields[y]);
        }
        for (size_t y = 0; y < carried.size(); ++y) env[op.results[y]] = carried[y];
        return 0;
      }
    }
    return build_error("unknown operation");
  }
};

// A Gemm whose whole fp16 result is read only by a Gelu of all of it
// becomes one launch with GELU in the GEMM epilogue: the epilogue rounds
// each product to fp16 and applies the GELU kernel's function to that
// value, so the result is bit-identical and one 2-byte-per-element write
// and read of the intermediate disappear.
void fuse_gemm_gelu(ipus_package& pkg) {
  std::vector<int> reads(pkg.slots.size(), 0), writes(pkg.slots.size(), 0);
  for (const Step& s : pkg.steps) {
    ++writes[(size_t)s.out.slot];
    for (const Operand& o : s.ins) ++reads[(size_t)o.slot];
  }
  std::vector<Step> steps;
  for (size_t i = 0; i < pkg.steps.size(); ++i) {
    const Step& s = pkg.steps[i];
    // The split-K reduction (the last step of a split GEMM) fuses the same
    // way: it rounds each sum to fp16 before GELU.
    const bool split_reduce = s.symbol == "ipu_stack_reduce_splits_f16" && s.scalars[2] == 0;
    if (i + 1 < pkg.steps.size() && (s.symbol == "ipu_stack_gemm_f16" || split_reduce) &&
        s.out.byte_offset == 0) {
      const Step& n = pkg.steps[i + 1];
      const int mid = s.out.slot;
      const Slot& ms = pkg.slots[(size_t)mid];
      if (n.symbol == "ipu_stack_gelu_tanh_approx_f16" && n.ins.size() == 1 &&
          n.ins[0].slot == mid && n.ins[0].byte_offset == 0 && n.out.byte_offset == 0 &&
          !ms.external && writes[(size_t)mid] == 1 && reads[(size_t)mid] == 1 &&
          n.scalars[0] == elements(ms.storage.shape)) {
        Step f = s;
        if (split_reduce)
          f.scalars[2] = 1;
        else
          f.symbol = "ipu_stack_gemm_f16_gelu";
        f.out = n.out;
        steps.push_back(std::move(f));
        ++i;
        continue;
      }
    }
    steps.push_back(s);
  }
  pkg.steps = std::move(steps);
}

// An fp16 Gemm whose whole result is read only by the Add that follows it
// (the residual x + x . W of graph.rs:12-33 and of Repeat bodies, or a bias)
// becomes one ipu_stack_gemm_f16_accumulate launch: the epilogue rounds the
// product to fp16 and adds the other operand like the Add kernel does, so
// the result is bit-identical, and the product's write and read disappear.
// The other operand must broadcast only as whole rows or whole matrices
// (column stride 1; batch axes collapsing to one stride).  A split-K GEMM
// fuses into its reduction (ipu_stack_reduce_splits_accumulate_f16).
void fuse_gemm_add(ipus_package& pkg) {
  std::vector<int> reads(pkg.slots.size(), 0), writes(pkg.slots.size(), 0);
  for (const Step& s : pkg.steps) {
    ++writes[(size_t)s.out.slot];
    for (const Operand& o : s.ins) ++reads[(size_t)o.slot];
  }
  std::vector<Step> steps;
  for (size_t i = 0; i < pkg.steps.size(); ++i) {
    const Step& s = pkg.steps[i];
    const bool gemm = s.symbol == "ipu_stack_gemm_f16";
    const bool split_reduce = s.symbol == "ipu_stack_reduce_splits_f16" && s.scalars[2] == 0;
    if (i + 1 >= pkg.steps.size() || !(gemm || split_reduce) || s.out.byte_offset != 0) {
      steps.push_back(s);
      continue;
    }
    const Step& n = pkg.steps[i + 1];
    const int mid = s.out.slot;
    const Slot& ms = pkg.slots[(size_t)mid];
    if (n.symbol != "ipu_stack_add_broadcast_f16" || n.ins.size() != 2 || ms.external ||
        writes[(size_t)mid] != 1 || reads[(size_t)mid] != 1 ||
        (n.ins[0].slot == mid) == (n.ins[1].slot == mid)) {
      steps.push_back(s);
      continue;
    }
    // add_broadcast scalars: rank, shape[6], left strides[6], right strides[6]
    const int which = n.ins[0].slot == mid ? 0 : 1;
    const Operand product = n.ins[(size_t)which], addend = n.ins[(size_t)(1 - which)];
    const uint32_t rank = n.scalars[0];
    auto shape = [&](uint32_t ax) { return n.scalars[1 + ax]; };
    auto stride = [&](int op, uint32_t ax) { return n.scalars[7 + 6 * (size_t)op + ax]; };
    bool ok = rank >= 2 && product.byte_offset == 0;
    // The product covers the Add's whole output densely (strides of size-1
    // axes are 0 in the lowering).
    uint64_t dense = 1;
    for (int ax = (int)rank - 1; ok && ax >= 0; --ax) {
      const uint32_t want = shape((uint32_t)ax) == 1 ? 0 : (uint32_t)dense;
      ok = stride(which, (uint32_t)ax) == want;
      dense *= shape((uint32_t)ax);
    }
    if (!ok || dense != elements(ms.storage.shape)) {
      steps.push_back(s);
      continue;
    }
    const uint32_t M = shape(rank - 2), N = shape(rank - 1), other = (uint32_t)(1 - which);
    ok = N == 1 || stride(other, rank - 1) == 1;
    const uint32_t row_stride = M == 1 ? 0 : stride(other, rank - 2);
    // Batch axes collapse to one stride: the innermost non-1 axis sets it,
    // each outer one must be that stride times the batches inside it.
    int64_t batch_stride = -1;
    uint64_t inner = 1;
    for (int ax = (int)rank - 3; ok && ax >= 0; --ax) {
      const uint32_t extent = shape((uint32_t)ax);
      if (extent != 1) {
        const uint64_t st = stride(other, (uint32_t)ax);
        if (batch_stride < 0) {
          ok = st % inner == 0;
          batch_stride = (int64_t)(st / inner);
        } else {
          ok = st == (uint64_t)batch_stride * inner;
        }
      }
      inner *= extent;
    }
    const uint64_t batches = dense / ((uint64_t)M * N);
    if (batch_stride < 0) batch_stride = 0;
    if (ok && gemm) ok = s.scalars[0] == batches && s.scalars[1] == M && s.scalars[2] == N;
    // The split reduction loads the addend as 16-byte chunks.
    if (ok && split_reduce)
      ok = N % 8 == 0 && row_stride % 8 == 0 && batch_stride % 8 == 0 &&
           addend.byte_offset % 16 == 0 && fits_u32(batches);
    if (!ok || !fits_u32((uint64_t)batch_stride)) {
      steps.push_back(s);
      continue;
    }
    Step f = s;
    if (gemm) {
      f.symbol = "ipu_stack_gemm_f16_accumulate";
      f.ins.push_back(addend);
      f.scalars.push_back((uint32_t)batch_stride);
      f.scalars.push_back(row_stride);
    } else {
      f.symbol = "ipu_stack_reduce_splits_accumulate_f16";
      f.ins.push_back(addend);
      f.scalars = {s.scalars[0], (uint32_t)batches, M, N, (uint32_t)batch_stride, row_stride};
    }
    f.out = n.out;
    steps.push_back(std::move(f));
    ++i;
  }
  pkg.steps = std::move(steps);
}

bool is_attention(const std::string& symbol) {
  return symbol == "ipu_stack_flash_attention_online_f16" ||
         symbol == "ipu_stack_flash_attention_heads_f16";
}

// A SplitHeads (operator.rs:213-279) whose fp16 result is read only as a
// Q, K or V operand of attention launches becomes a strided view: the
// attention reads head s % h of the unsplit [batch, rows, h * width]
// tensor directly (ipu_stack_flash_attention_heads_f16), and the copy and
// its buffer disappear.
void elide_split_heads(ipus_package& pkg) {
  std::vector<int> writes(pkg.slots.size(), 0), reads(pkg.slots.size(), 0);
  std::vector<bool> other_reader(pkg.slots.size(), false);
  for (const Step& s : pkg.steps) {
    ++writes[(size_t)s.out.slot];
    for (const Operand& o : s.ins) {
      ++reads[(size_t)o.slot];
      if (!is_attention(s.symbol) || o.byte_offset != 0) other_reader[(size_t)o.slot] = true;
    }
  }
  std::map<int, std::pair<Operand, uint32_t>> view;  // split result -> (unsplit operand, heads)
  std::vector<Step> steps;
  for (const Step& s : pkg.steps) {
    // split_heads scalars: batch, rows, heads, head width, element bytes
    if (s.symbol == "ipu_stack_split_heads" && s.out.byte_offset == 0 && s.scalars.size() == 5 &&
        s.scalars[4] == 2) {
      const size_t o = (size_t)s.out.slot;
      if (!pkg.slots[o].external && writes[o] == 1 && reads[o] > 0 && !other_reader[o]) {
        view[s.out.slot] = {s.ins[0], s.scalars[2]};
        continue;
      }
    }
    steps.push_back(s);
  }
  for (Step& s : steps) {
    if (!is_attention(s.symbol)) continue;
    uint32_t heads[3] = {1, 1, 1};
    if (s.symbol == "ipu_stack_flash_attention_heads_f16")
      for (int k = 0; k < 3; ++k) heads[k] = s.scalars[8 + (size_t)k];
    bool changed = false;
    for (int k = 0; k < 3; ++k) {
      auto it = view.find(s.ins[(size_t)k].slot);
      if (it == view.end()) continue;
      s.ins[(size_t)k] = it->second.first;
      heads[k] = it->second.second;
      changed = true;
    }
    if (!changed) continue;
    s.symbol = "ipu_stack_flash_attention_heads_f16";
    s.scalars.resize(8);
    s.scalars.insert(s.scalars.end(), heads, heads + 3);
  }
  pkg.steps = std::move(steps);
}

// Lifetime-packed arena offsets for non-external slots.
uint64_t place(ipus_package& pkg) {
  for (size_t i = 0; i < pkg.steps.size(); ++i) {
    const Step& s = pkg.steps[i];
    auto touch = [&](int slot, bool def) {
      Slot& sl = pkg.slots[(size_t)slot];
      if (def && sl.first_def < 0) sl.first_def = (int)i;
      if (sl.first_def < 0) sl.first_def = (int)i;
      sl.last_use = std::max(sl.last_use, (int)i);
    };
    touch(s.out.slot, true);
    for (const Operand& o : s.ins) touch(o.slot, false);
  }
  struct Live {
    uint64_t offset, bytes;
    int end;
  };
  std::vector<Live> live;
  uint64_t arena = 0;
  std::vector<int> order;
  for (size_t i = 0; i < pkg.slots.size(); ++i)
    if (!pkg.slots[i].external && pkg.slots[i].first_def >= 0) order.push_back((int)i);
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    return pkg.slots[(size_t)a].first_def < pkg.slots[(size_t)b].first_def;
  });
  for (int idx : order) {
    Slot& s = pkg.slots[(size_t)idx];
    live.erase(std::remove_if(live.begin(), live.end(),
                              [&](const Live& l) { return l.end < s.first_def; }),
               live.end());
    std::sort(live.begin(), live.end(),
              [](const Live& a, const Live& b) { return a.offset < b.offset; });
    const uint64_t bytes = (s.storage.bytes() + 255) & ~uint64_t(255);
    uint64_t cursor = 0;
    for (const Live& l : live) {
      if (cursor + bytes <= l.offset) break;
      cursor = std::max(cursor, l.offset + l.bytes);
    }
    s.storage.buffer = -2;
    s.storage.offset = cursor;
    live.push_back({cursor, bytes, s.last_use});
    arena = std::max(arena, cursor + bytes);
  }
  return arena;
}

}  // namespace

extern "C" int ipus_build_package(const ipus_graph* g, const ipus_package_config* config,
                                  ipus_package** out) {
  if (!g || !out) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  if (!g->open.empty()) return build_error("graph has an open repeat body");
  ipus_package_config cfg = {IPUS_PRECISION_F16, 0, 0, nullptr};
  if (config) cfg = *config;
  if (cfg.compute_precision != IPUS_PRECISION_F16 && cfg.compute_precision != IPUS_PRECISION_F32)
    return build_error("compute precision must be F16 or F32");
  if (cfg.input_format_count < 0 || (cfg.input_format_count > 0 && !cfg.input_formats))
    return build_error("input formats: bad count or null array");
  // PipelineConfig inputs (config.rs:310-320): one entry per named input.
  std::map<uint32_t, const ipus_input_format*> formats;
  for (int i = 0; i < cfg.input_format_count; ++i) {
    const ipus_input_format& f = cfg.input_formats[i];
    bool is_input = false;
    for (const auto& in : g->inputs) is_input = is_input || in.value == f.value;
    if (!is_input)
      return build_error("input format names value " + std::to_string(f.value) +
                         ", which is not a graph input");
    if (f.format.precision != IPUS_PRECISION_F16 && f.format.precision != IPUS_PRECISION_F32)
      return build_error("input format precision must be F16 or F32");
    formats[f.value] = &f;  // a later entry replaces an earlier one, as with_input does
  }
  auto pkg = std::make_unique<ipus_package>();
  Builder b{*g, cfg, *pkg, {}};
  for (const auto& in : g->inputs) {
    const Shape& shape = g->shapes.at(in.value);
    auto fit = formats.find(in.value);
    const ipus_input_format* f = fit == formats.end() ? nullptr : fit->second;
    const int precision = f ? f->format.precision : cfg.compute_precision;
    const int slot = b.new_slot(shape, precision);
    pkg->slots[(size_t)slot].external = true;
    b.env[in.value] = slot;
    pkg->inputs.push_back({in.name, in.value, slot});
    if (!f || f->automatic) continue;
    // with_input: the host writes the format's shards; one unshard launch
    // turns them into the row-major tensor the rest of the plan reads.
    ipus::ResolvedFormat rf;
    std::string error;
    if (!ipus::resolve_format(shape, f->format, &rf, &error))
      return build_error("input " + in.name + ": " + error);
    if (ipus::format_is_row_major_identity(rf, f->format)) continue;
    const uint64_t esize = precision == IPUS_PRECISION_F32 ? 4 : 2;
    Storage& st = pkg->slots[(size_t)slot].storage;
    st.order = f->format.order;
    st.row_block = f->format.row_block;
    st.column_block = f->format.column_block;
    st.file_bytes = rf.file_elements * esize;
    st.shards = f->format.tile_count;
    uint32_t shard_count = 0;
    uint64_t max_elements = 0;
    const std::vector<uint32_t> table = ipus::shard_table(rf, &shard_count, &max_elements);
    if (shard_count > 65535) return build_error("input " + in.name + ": too many shards");
    if (st.file_bytes == 0 || shard_count == 0) continue;  // empty tensor: nothing to convert
    const int tslot = b.new_slot({(uint32_t)(table.size() * 2)}, IPUS_PRECISION_F16);
    Slot& ts = pkg->slots[(size_t)tslot];
    ts.external = true;
    ts.constant.resize(table.size() * 4);
    memcpy(ts.constant.data(), table.data(), ts.constant.size());
    const int unsharded = b.new_slot(shape, precision);
    b.emit("ipu_stack_unshard", unsharded, {{slot, 0}, {tslot, 0}},
           {shard_count, (uint32_t)shape.size(), (uint32_t)f->format.order, f->format.row_block,
            f->format.column_block, (uint32_t)esize,
            (uint32_t)std::min<uint64_t>(max_elements, 0xffffffffull)});
    b.env[in.value] = unsharded;
  }
  if (int e = b.lower_ops(g->root.operations)) return e;
  for (size_t i = 0; i < g->outputs.size(); ++i) {
    const uint32_t v = g->outputs[i];
    int slot = b.env.at(v);
    // Outputs get their own binding buffer: copy when the value is an input,
    // an earlier output, or otherwise not freshly produced.
    bool reuse = !pkg->slots[(size_t)slot].external;
    for (const auto& o : pkg->outputs)
      if (o.slot == slot) reuse = false;
    if (!reuse) {
      const Storage s = pkg->slots[(size_t)slot].storage;
      const int copy = b.new_slot(s.shape, s.precision, s.order, s.row_block, s.column_block);
      b.emit_chunked("ipu_stack_copy", copy, slot, s.bytes(), 1, 1);
      slot = copy;
    }
    pkg->slots[(size_t)slot].external = true;
    pkg->outputs.push_back({"output." + std::to_string(i), v, slot});
  }
  // Precision map (CompiledPackage::precisions) over every value bound to a slot.
  for (const auto& kv : b.env) pkg->precisions[kv.first] = pkg->slots[(size_t)kv.second].storage.precision;
  fuse_gemm_gelu(*pkg);
  fuse_gemm_add(*pkg);
  elide_split_heads(*pkg);
  pkg->arena_bytes = place(*pkg);
  *out = pkg.release();
  return 0;
}

extern "C" int ipus_package_destroy(ipus_package* p) {
  delete p;
  return 0;
}

namespace {
int tensor_info(const ipus_package* p, const Binding& b, ipus_tensor_info* info) {
  const Storage& s = p->slots[(size_t)b.slot].storage;
  memset(info, 0, sizeof(*info));
  info->name = b.name.c_str();
  info->value = b.value;
  info->rank = (int)s.shape.size();
  for (size_t i = 0; i < s.shape.size() && i < IPUS_MAX_RANK; ++i) info->dims[i] = s.shape[i];
  info->precision = s.precision;
  info->order = s.order;
  info->row_block = s.row_block;
  info->column_block = s.column_block;
  info->bytes = s.bytes();
  info->shards = s.shards;
  return 0;
}
}  // namespace

extern "C" int ipus_package_input_count(const ipus_package* p, int* count) {
  if (!p || !count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *count = (int)p->inputs.size();
  return 0;
}
extern "C" int ipus_package_input_info(const ipus_package* p, int i, ipus_tensor_info* info) {
  if (!p || !info || i < 0 || i >= (int)p->inputs.size())
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "bad input index");
  return tensor_info(p, p->inputs[(size_t)i], info);
}
extern "C" int ipus_package_output_count(const ipus_package* p, int* count) {
  if (!p || !count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *count = (int)p->outputs.size();
  return 0;
}
extern "C" int ipus_package_output_info(const ipus_package* p, int i, ipus_tensor_info* info) {
  if (!p || !info || i < 0 || i >= (int)p->outputs.size())
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "bad output index");
  return tensor_info(p, p->outputs[(size_t)i], info);
}
extern "C" int ipus_package_step_count(const ipus_package* p, int* count) {
  if (!p || !count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *count = (int)p->steps.size();
  return 0;
}
extern "C" int ipus_package_step(const ipus_package* p, int i, const char** symbol,
                                 int* input_count, int* scalar_count, const uint32_t** scalars) {
  if (!p || i < 0 || i >= (int)p->steps.size())
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "bad step index");
  const Step& s = p->steps[(size_t)i];
  if (symbol) *symbol = s.symbol.c_str();
  if (input_count) *input_count = (int)s.ins.size();
  if (scalar_count) *scalar_count = (int)s.scalars.size();
  if (scalars) *scalars = s.scalars.data();
  return 0;
}
extern "C" int ipus_package_arena_bytes(const ipus_package* p, uint64_t* bytes) {
  if (!p || !bytes) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *bytes = p->arena_bytes;
  return 0;
}
extern "C" int ipus_package_value_precision(const ipus_package* p, ipus_value v, int* precision) {
  if (!p || !precision) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  auto it = p->precisions.find(v);
  if (it == p->precisions.end()) return fail(IPUS_ERROR_INVALID_ARGUMENT, "value %u has no storage", v);
  *precision = it->second;
  return 0;
}

// ===========================================================================
// Session
// ===========================================================================
struct ipus_session {
  ipus_context* ctx = nullptr;
  const ipus_package* pkg = nullptr;
  std::vector<void*> slot_ptr;  // device pointer per slot
  std::vector<void*> owned;
  // After ipus_session_capture: the package's launches as one HIP graph.
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

extern "C" int ipus_session_create(ipus_context* ctx, const ipus_package* pkg, ipus_session** out) {
  if (!ctx || !pkg || !out) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  auto s = std::make_unique<ipus_session>();
  s->ctx = ctx;
  s->pkg = pkg;
  s->slot_ptr.assign(pkg->slots.size(), nullptr);
  void* arena = nullptr;
  if (pkg->arena_bytes) {
    if (int e = ipus_buffer_alloc(ctx, pkg->arena_bytes, &arena)) return e;
    s->owned.push_back(arena);
  }
  for (size_t i = 0; i < pkg->slots.size(); ++i) {
    const Slot& sl = pkg->slots[i];
    if (sl.external) {
      void* p = nullptr;
      int e = ipus_buffer_alloc(ctx, sl.storage.bytes(), &p);
      if (!e && !sl.constant.empty())
        e = ipus_buffer_upload(ctx, p, sl.constant.data(), sl.constant.size());
      if (e) {
        if (p) ipus_buffer_free(ctx, p);
        for (void* q : s->owned) ipus_buffer_free(ctx, q);
        return e;
      }
      s->owned.push_back(p);
      s->slot_ptr[i] = p;
    } else if (sl.storage.buffer == -2) {
      s->slot_ptr[i] = (uint8_t*)arena + sl.storage.offset;
    }
  }
  *out = s.release();
  return 0;
}

extern "C" int ipus_session_destroy(ipus_session* s) {
  if (!s) return 0;
  // The session is released even when the device reports an error; the
  // first error is returned.
  int status = use_device(s->ctx);
  if (int e = ipus_stream_sync(s->ctx); e && !status) status = e;
  if (s->exec) {
    const hipError_t e = hipGraphExecDestroy(s->exec);
    if (e != hipSuccess && !status) status = hip_fail(e, "hipGraphExecDestroy");
  }
  if (s->graph) {
    const hipError_t e = hipGraphDestroy(s->graph);
    if (e != hipSuccess && !status) status = hip_fail(e, "hipGraphDestroy");
  }
  for (void* p : s->owned)
    if (int e = ipus_buffer_free(s->ctx, p); e && !status) status = e;
  delete s;
  return status;
}

namespace {
int find_binding(ipus_session* s, const char* name, int* slot) {
  if (!s || !name) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  for (const auto& b : s->pkg->inputs)
    if (b.name == name) {
      *slot = b.slot;
      return 0;
    }
  for (const auto& b : s->pkg->outputs)
    if (b.name == name) {
      *slot = b.slot;
      return 0;
    }
  return fail(IPUS_ERROR_INVALID_ARGUMENT, "package has no binding named %s", name);
}
}  // namespace

extern "C" int ipus_session_write(ipus_session* s, const char* name, const void* host, size_t bytes) {
  int slot;
  if (int e = find_binding(s, name, &slot)) return e;
  const uint64_t need = s->pkg->slots[(size_t)slot].storage.bytes();
  if (bytes != need)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "binding %s holds %llu bytes, got %zu", name,
                (unsigned long long)need, bytes);
  return ipus_buffer_upload(s->ctx, s->slot_ptr[(size_t)slot], host, bytes);
}

extern "C" int ipus_session_read(ipus_session* s, const char* name, void* host, size_t bytes) {
  int slot;
  if (int e = find_binding(s, name, &slot)) return e;
  const uint64_t need = s->pkg->slots[(size_t)slot].storage.bytes();
  if (bytes != need)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "binding %s holds %llu bytes, got %zu", name,
                (unsigned long long)need, bytes);
  return ipus_buffer_download(s->ctx, host, s->slot_ptr[(size_t)slot], bytes);
}

extern "C" int ipus_session_tensor_pointer(ipus_session* s, const char* name, void** ptr) {
  int slot;
  if (int e = find_binding(s, name, &slot)) return e;
  if (!ptr) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *ptr = s->slot_ptr[(size_t)slot];
  return 0;
}

namespace {
// Enqueues every step of the package on the context stream.
int launch_steps(ipus_session* s) {
  std::vector<const void*> ins;
  for (const Step& st : s->pkg->steps) {
    ins.clear();
    for (const Operand& o : st.ins) ins.push_back((const uint8_t*)s->slot_ptr[(size_t)o.slot] + o.byte_offset);
    void* outp = (uint8_t*)s->slot_ptr[(size_t)st.out.slot] + st.out.byte_offset;
    if (int e = ipus_launch(s->ctx, st.symbol.c_str(), outp, ins.data(), (int)ins.size(),
                            st.scalars.data(), (int)st.scalars.size()))
      return e;
  }
  return 0;
}
}  // namespace

extern "C" int ipus_session_run(ipus_session* s) {
  if (!s) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null session");
  if (int status = use_device(s->ctx)) return status;
  if (s->exec) {
    const hipError_t e = hipGraphLaunch(s->exec, s->ctx->stream);
    return e == hipSuccess ? 0 : hip_fail(e, "hipGraphLaunch");
  }
  return launch_steps(s);
}

extern "C" int ipus_session_capture(ipus_session* s) {
  if (!s) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null session");
  if (s->exec || s->pkg->steps.empty()) return 0;
  if (int status = use_device(s->ctx)) return status;
  hipStream_t stream = s->ctx->stream;
  hipError_t e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
  const int status = launch_steps(s);
  hipGraph_t graph = nullptr;
  e = hipStreamEndCapture(stream, &graph);  // always ends the capture
  if (status != 0) {
    if (graph) (void)hipGraphDestroy(graph);
    return status;
  }
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_fail(e, "hipGraphInstantiate");
  }
  s->graph = graph;
  s->exec = exec;
  return 0;
}

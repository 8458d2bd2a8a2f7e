// Shard geometry of a declared input format: the reference's TensorTiling
// resolution (crates/ipu-codegen/src/layout.rs:1002-1135 resolve,
// 1267-1300 shard_extents, 1427-1504 resolve_axis_bounds, 1506-1570 tile
// mapping) restated for the host side of build_package, plus the table the
// unshard kernel reads.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/ipus_graph.h"

namespace ipus {

constexpr int kMaxShardRank = 8;

struct ShardExtent {
  uint32_t start = 0, logical_end = 0, physical_end = 0;
};

struct ResolvedShard {
  uint32_t tile = 0;
  std::vector<ShardExtent> extents;  // one per tensor axis
  uint64_t file_offset = 0;          // elements before this shard in the host bytes
  uint64_t physical_elements() const;
  uint64_t logical_elements() const;
};

struct ResolvedFormat {
  std::vector<uint32_t> shape;
  std::vector<ResolvedShard> shards;  // every tile, in logical tile order
  uint64_t file_elements = 0;         // all shards' storage, replicas included
};

// Resolves `format` for a tensor of `shape`; false with a LayoutError-style
// message when the layout does not apply to the shape.
bool resolve_format(const std::vector<uint32_t>& shape, const ipus_tensor_format& format,
                    ResolvedFormat* out, std::string* error);

// True when the host bytes already are the row-major tensor (no padding, no
// replicas, shards in row-major order of contiguous ranges).
bool format_is_row_major_identity(const ResolvedFormat& r, const ipus_tensor_format& format);

// Device table of the unshard kernel (u32 words): a 16-word header holding
// the tensor's dims (8 words) and 8 reserved words, then per distinct shard
// (one tile per distinct coordinate, empty shards skipped) kShardWords words:
// file element offset (lo, hi), start[8], logical width[8], physical
// width[8].
constexpr uint32_t kShardHeaderWords = 16;
constexpr uint32_t kShardWords = 2 + 3 * kMaxShardRank;
std::vector<uint32_t> shard_table(const ResolvedFormat& r, uint32_t* shard_count,
                                  uint64_t* max_shard_elements);

}  // namespace ipus

// TensorTiling resolution for declared input formats (see tiling.h).  The
// rules are the reference's, so a layout the reference accepts resolves to
// the same shards here:
//   * every tiled axis has nonzero partitions, padding groups, block size and
//     padding multiples; no axis is tiled twice (layout.rs:1029-1046);
//   * each padding group of the axis is padded up to the padding multiple
//     (Padding::Zero) or must divide (Padding::Reject), then must hold whole
//     blocks (layout.rs:1047-1081);
//   * tile_count = replicas x the product of partitions (layout.rs:1083-1088);
//   * tile strides: explicit or packed after the replicas (layout.rs:234-251),
//     and every axis coordinate tuple owned by exactly `replicas` tiles
//     (layout.rs:1506-1570);
//   * a partition owns a contiguous run of blocks, the first `long_shards`
//     one block more, padded to the shard padding multiple
//     (layout.rs:1427-1504).
#include "tiling.h"

#include <algorithm>
#include <map>

namespace ipus {

uint64_t ResolvedShard::physical_elements() const {
  uint64_t n = 1;
  for (const ShardExtent& e : extents) n *= (uint64_t)(e.physical_end - e.start);
  return n;
}

uint64_t ResolvedShard::logical_elements() const {
  uint64_t n = 1;
  for (const ShardExtent& e : extents) n *= (uint64_t)(e.logical_end - e.start);
  return n;
}

namespace {

struct Axis {
  ipus_axis_tiling t;  // defaults filled in
  uint32_t index = 0;  // resolved tensor axis
  uint32_t stride = 0; // tile stride
};

// resolve_axis_bounds (layout.rs:1427-1504): (start, logical_end,
// physical_end) of partition `coordinate`.
bool axis_bounds(const ipus_axis_tiling& t, uint32_t padded_extent, uint32_t logical_extent,
                 uint32_t coordinate, ShardExtent* out, std::string* error) {
  const uint32_t partitions = t.partitions, groups = t.padding_groups;
  if (groups == 0 || coordinate >= partitions || partitions % groups || padded_extent % groups ||
      logical_extent % groups) {
    *error = "invalid padding groups";
    return false;
  }
  const uint32_t per_group = partitions / groups;
  const uint32_t group = coordinate / per_group, in_group = coordinate % per_group;
  const uint32_t padded_group = padded_extent / groups, logical_group = logical_extent / groups;
  if (padded_group % t.block_size) {
    *error = "axis extent is not a multiple of its block size";
    return false;
  }
  const uint32_t blocks = padded_group / t.block_size;
  const uint32_t short_size = blocks / per_group, long_shards = blocks % per_group;
  const uint64_t start_blocks =
      (uint64_t)in_group * short_size + std::min(in_group, long_shards);
  const uint64_t shard_blocks = short_size + (in_group < long_shards ? 1 : 0);
  const uint64_t start_in_group = start_blocks * t.block_size;
  const uint64_t allocated = shard_blocks * t.block_size;
  const uint64_t remainder = allocated % t.shard_padding_multiple;
  if (remainder && !t.zero_padding) {
    *error = "shard extent is not a multiple of its shard padding multiple";
    return false;
  }
  const uint64_t physical_width = remainder ? allocated + t.shard_padding_multiple - remainder
                                            : allocated;
  const uint64_t base = (uint64_t)group * logical_group;
  const uint64_t start = base + start_in_group;
  const uint64_t logical_end =
      base + std::max<uint64_t>(std::min<uint64_t>(start_in_group + allocated, logical_group),
                                start_in_group);
  const uint64_t physical_end = start + physical_width;
  if (physical_end > 0xffffffffull) {
    *error = "axis extent overflow";
    return false;
  }
  *out = {(uint32_t)start, (uint32_t)logical_end, (uint32_t)physical_end};
  return true;
}

bool regular_mapping(const std::vector<Axis>& axes, uint32_t replicas) {
  std::vector<std::pair<uint32_t, uint32_t>> digits;
  for (const Axis& a : axes)
    if (a.t.partitions > 1) digits.push_back({a.stride, a.t.partitions});
  std::sort(digits.begin(), digits.end());
  if (digits.empty()) return true;
  const uint32_t base = digits[0].first;
  if (base == 0 || replicas % base) return false;
  uint64_t expected = base;
  for (const auto& d : digits) {
    if (d.first != expected) return false;
    expected *= d.second;
  }
  return true;
}

}  // namespace

bool resolve_format(const std::vector<uint32_t>& shape, const ipus_tensor_format& f,
                    ResolvedFormat* out, std::string* error) {
  const size_t rank = shape.size();
  if (rank == 0 || rank > (size_t)kMaxShardRank) {
    *error = "a declared format needs a tensor of rank 1 to 8";
    return false;
  }
  if (f.tile_count == 0 || f.replicas == 0) {
    *error = "empty tile group";
    return false;
  }
  if (f.axis_count < 0 || f.axis_count > IPUS_MAX_TILED_AXES) {
    *error = "too many tiled axes";
    return false;
  }
  std::vector<uint32_t> padded = shape;
  std::vector<Axis> axes;
  uint64_t used_tiles = f.replicas;
  for (int i = 0; i < f.axis_count; ++i) {
    Axis a;
    a.t = f.axes[i];
    if (a.t.padding_groups == 0) a.t.padding_groups = 1;
    if (a.t.padding_multiple == 0) a.t.padding_multiple = a.t.block_size;
    if (a.t.shard_padding_multiple == 0) a.t.shard_padding_multiple = 1;
    if (a.t.partitions == 0 || a.t.block_size == 0 || a.t.padding_multiple == 0) {
      *error = "empty axis tiling";
      return false;
    }
    used_tiles *= a.t.partitions;
    if (used_tiles > 0xffffull) {
      *error = "tile count overflow";
      return false;
    }
    if (a.t.from_end ? (a.t.axis == 0 || a.t.axis > rank) : a.t.axis >= rank) {
      *error = "tiled axis out of range";
      return false;
    }
    a.index = a.t.from_end ? (uint32_t)rank - a.t.axis : a.t.axis;
    for (const Axis& b : axes)
      if (b.index == a.index) {
        *error = "axis tiled twice";
        return false;
      }
    const uint32_t extent = padded[a.index], groups = a.t.padding_groups;
    if (a.t.partitions % groups || extent % groups) {
      *error = "invalid padding groups";
      return false;
    }
    const uint32_t group_extent = extent / groups;
    const uint32_t remainder = group_extent % a.t.padding_multiple;
    if (remainder && !a.t.zero_padding) {
      *error = "axis " + std::to_string(a.index) + " extent " + std::to_string(group_extent) +
               " is not a multiple of " + std::to_string(a.t.padding_multiple);
      return false;
    }
    if (remainder) {
      const uint64_t p = ((uint64_t)group_extent + a.t.padding_multiple - remainder) * groups;
      if (p > 0xffffffffull) {
        *error = "axis extent overflow";
        return false;
      }
      padded[a.index] = (uint32_t)p;
    }
    if ((padded[a.index] / groups) % a.t.block_size) {
      *error = "axis " + std::to_string(a.index) + " is not a multiple of its block size";
      return false;
    }
    axes.push_back(a);
  }
  if (used_tiles != f.tile_count) {
    *error = "tile count " + std::to_string(f.tile_count) + " does not match the tiling's " +
             std::to_string(used_tiles);
    return false;
  }
  // axis_strides (layout.rs:234-251).
  uint64_t packed = f.replicas;
  for (Axis& a : axes) {
    a.stride = a.t.tile_stride ? a.t.tile_stride : (uint32_t)packed;
    packed *= a.t.partitions;
  }
  if (!regular_mapping(axes, f.replicas)) {
    std::map<uint64_t, uint32_t> copies;
    for (uint32_t tile = 0; tile < f.tile_count; ++tile) {
      uint64_t c = 0;
      for (const Axis& a : axes) c = c * a.t.partitions + (tile / a.stride) % a.t.partitions;
      ++copies[c];
    }
    uint64_t coordinates = 1;
    for (const Axis& a : axes) coordinates *= a.t.partitions;
    bool ok = copies.size() == coordinates;
    for (const auto& kv : copies) ok = ok && kv.second == f.replicas;
    if (!ok) {
      *error = "tile strides do not map the tiles onto every coordinate";
      return false;
    }
  }
  out->shape = shape;
  out->shards.clear();
  uint64_t offset = 0;
  for (uint32_t tile = 0; tile < f.tile_count; ++tile) {
    ResolvedShard sh;
    sh.tile = tile;
    sh.extents.resize(rank);
    for (size_t ax = 0; ax < rank; ++ax) sh.extents[ax] = {0, shape[ax], padded[ax]};
    for (const Axis& a : axes) {
      const uint32_t coordinate = (tile / a.stride) % a.t.partitions;
      if (!axis_bounds(a.t, padded[a.index], shape[a.index], coordinate, &sh.extents[a.index],
                       error))
        return false;
    }
    sh.file_offset = offset;
    offset += sh.physical_elements();
    out->shards.push_back(std::move(sh));
  }
  out->file_elements = offset;
  // Per-shard storage constraints of the element order (storage.rs:300-426).
  const int order = f.order;
  if (order != IPUS_ORDER_ROW_MAJOR) {
    if (f.precision != IPUS_PRECISION_F16) {
      *error = "AMP and block-major input formats need F16";
      return false;
    }
    if (rank < 2) {
      *error = "AMP and block-major orders need a matrix";
      return false;
    }
    if (order == IPUS_ORDER_BLOCK_MAJOR || order == IPUS_ORDER_BLOCK_MAJOR_TRANSPOSED) {
      if (f.row_block == 0 || f.column_block == 0 || f.row_block % 16) {
        *error = "block-major orders need nonzero blocks with row_block a multiple of 16";
        return false;
      }
    }
    for (const ResolvedShard& sh : out->shards) {
      const uint32_t R = sh.extents[rank - 2].physical_end - sh.extents[rank - 2].start;
      const uint32_t C = sh.extents[rank - 1].physical_end - sh.extents[rank - 1].start;
      bool ok = true;
      switch (order) {
        case IPUS_ORDER_AMP_LEFT:
        case IPUS_ORDER_AMP_OUTPUT: ok = C % 16 == 0; break;
        case IPUS_ORDER_AMP_TRANSPOSED_LEFT:
        case IPUS_ORDER_AMP_TRANSPOSED_OUTPUT: ok = R % 16 == 0; break;
        case IPUS_ORDER_AMP_TRANSPOSED_RIGHT: ok = R % 16 == 0 && C % 16 == 0; break;
        case IPUS_ORDER_BLOCK_MAJOR: ok = R % f.row_block == 0 && C % f.column_block == 0; break;
        case IPUS_ORDER_BLOCK_MAJOR_TRANSPOSED:
          ok = C % f.row_block == 0 && R % f.column_block == 0;
          break;
        default:
          *error = "unknown element order";
          return false;
      }
      if (!ok) {
        *error = "a shard's matrix extents do not fit its element order's blocks";
        return false;
      }
    }
  }
  return true;
}

bool format_is_row_major_identity(const ResolvedFormat& r, const ipus_tensor_format& f) {
  if (f.order != IPUS_ORDER_ROW_MAJOR || f.replicas != 1) return false;
  // Shards in file order must be consecutive row-major ranges: every axis
  // but the first whole and unpadded, the first axis split in order.
  uint64_t expected_start = 0;
  for (const ResolvedShard& sh : r.shards) {
    for (size_t ax = 0; ax < r.shape.size(); ++ax) {
      const ShardExtent& e = sh.extents[ax];
      if (e.physical_end != e.logical_end) return false;
      if (ax > 0 && (e.start != 0 || e.logical_end != r.shape[ax])) return false;
    }
    if (sh.extents[0].start != expected_start) return false;
    expected_start = sh.extents[0].logical_end;
  }
  return expected_start == r.shape[0];
}

std::vector<uint32_t> shard_table(const ResolvedFormat& r, uint32_t* shard_count,
                                  uint64_t* max_shard_elements) {
  const size_t rank = r.shape.size();
  std::vector<uint32_t> t(kShardHeaderWords, 0);
  for (size_t ax = 0; ax < rank; ++ax) t[ax] = r.shape[ax];
  std::map<std::vector<uint32_t>, bool> seen;  // one tile per distinct region (replicas)
  *shard_count = 0;
  *max_shard_elements = 0;
  for (const ResolvedShard& sh : r.shards) {
    if (sh.logical_elements() == 0) continue;
    std::vector<uint32_t> key;
    for (const ShardExtent& e : sh.extents) key.push_back(e.start);
    if (seen.count(key)) continue;
    seen[key] = true;
    t.push_back((uint32_t)(sh.file_offset & 0xffffffffu));
    t.push_back((uint32_t)(sh.file_offset >> 32));
    for (int ax = 0; ax < kMaxShardRank; ++ax)
      t.push_back(ax < (int)rank ? sh.extents[(size_t)ax].start : 0);
    for (int ax = 0; ax < kMaxShardRank; ++ax)
      t.push_back(ax < (int)rank ? sh.extents[(size_t)ax].logical_end -
                                       sh.extents[(size_t)ax].start
                                 : 1);
    for (int ax = 0; ax < kMaxShardRank; ++ax)
      t.push_back(ax < (int)rank ? sh.extents[(size_t)ax].physical_end -
                                       sh.extents[(size_t)ax].start
                                 : 1);
    ++*shard_count;
    *max_shard_elements = std::max(*max_shard_elements, sh.logical_elements());
  }
  return t;
}

}  // namespace ipus

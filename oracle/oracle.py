"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or as the timed CPU baseline.
Product code (ipu-stack_amd/) never imports it.  Every function restates the
reference semantics cited in oracle/oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "liboracle.so")

F8, F16, F32 = 0, 1, 2
AMP_LEFT, AMP_TRANSPOSED_LEFT, AMP_TRANSPOSED_RIGHT, AMP_OUTPUT, AMP_TRANSPOSED_OUTPUT = range(5)

_lib = None


def build() -> None:
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            build()
        _lib = ctypes.CDLL(LIBRARY)
        u32, u64, i64, P = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p
        i32 = ctypes.c_int
        sigs = {
            "or_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "or_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "or_f32_to_f16_array": (None, [P, P, ctypes.c_size_t]),
            "or_f16_to_f32_array": (None, [P, P, ctypes.c_size_t]),
            "or_amp_matrix_index": (i64, [i32, i32, u32, u32, u32, u32]),
            "or_amp_matrix_coordinates": (
                i32, [i32, i32, u32, u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]),
            "or_right_matrix_index": (i64, [i32, u32, u32, u32, u32]),
            "or_block_major_matrix_index": (i64, [i32, u32, u32, i32, u32, u32, u32, u32]),
            "or_block_major_matrix_coordinates": (
                i32, [i32, u32, u32, i32, u32, u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]),
            "or_rearrange_row_major_f16": (i32, [i32, u32, u32, u32, u32, u32, u32, u32, P, P]),
            "or_unpack_to_row_major_f16": (i32, [i32, u32, u32, u32, u32, u32, P, P]),
            "or_transpose_u16": (None, [u32, u32, u32, P, P]),
            "or_gemm_f32": (i32, [P, P, P, u32, u64, u64, u32, u32, u32, i32, i32, i32]),
            "or_gemm_f16": (i32, [P, P, P, u32, u64, u64, u32, u32, u32, i32, i32, i32]),
            "or_gemm_f16_rows": (i32, [P, P, P, u32, u32, u32, P, u32, i32]),
            "or_attention": (
                i32, [P, P, P, P, u32, u32, u32, u32, u32, i32, ctypes.c_float, i32, P, u32, i32]),
            "or_gelu_reference": (ctypes.c_float, [ctypes.c_float]),
            "or_gelu_f16": (None, [P, P, ctypes.c_size_t]),
            "or_add_f32": (i32, [P, P, i32, P, P, i32, P, P, ctypes.POINTER(i32)]),
            "or_split_heads": (i32, [P, u32, u32, u32, u32, P]),
            "or_reduce_sum_f16": (None, [P, P, u32, u32, P]),
            "or_reduce_rows_f16": (None, [P, u32, u32, P, i32]),
            "or_reduce_rows_block_major_f16": (i32, [P, u32, u32, u32, u32, P, i32]),
            "or_splitmix64": (u64, [u64]),
            "or_pack_shard": (i32, [i32, i32, u32, u32, i32, P, P, P, P, P, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def threads() -> int:
    return min(os.cpu_count() or 1, 16)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- fp16 ----
def f32_to_f16(values) -> np.ndarray:
    src = _c(values, np.float32).reshape(-1)
    out = np.empty(src.size, dtype=np.uint16)
    lib().or_f32_to_f16_array(src.ctypes.data, out.ctypes.data, src.size)
    return out.reshape(np.shape(values))


def f16_to_f32(bits) -> np.ndarray:
    src = _c(bits, np.uint16).reshape(-1)
    out = np.empty(src.size, dtype=np.float32)
    lib().or_f16_to_f32_array(src.ctypes.data, out.ctypes.data, src.size)
    return out.reshape(np.shape(bits))


# ---- index maps ----
def amp_matrix_index(role, precision, rows, columns, row, column) -> int:
    return lib().or_amp_matrix_index(role, precision, rows, columns, row, column)


def amp_matrix_coordinates(role, precision, rows, columns, linear):
    r, c = ctypes.c_uint32(), ctypes.c_uint32()
    status = lib().or_amp_matrix_coordinates(role, precision, rows, columns, linear,
                                             ctypes.byref(r), ctypes.byref(c))
    return None if status != 0 else (r.value, c.value)


def block_major_matrix_index(transposed, row_block, column_block, precision, rows, columns, row,
                             column) -> int:
    return lib().or_block_major_matrix_index(int(transposed), row_block, column_block, precision,
                                             rows, columns, row, column)


def block_major_matrix_coordinates(transposed, row_block, column_block, precision, rows, columns,
                                   linear):
    r, c = ctypes.c_uint32(), ctypes.c_uint32()
    status = lib().or_block_major_matrix_coordinates(int(transposed), row_block, column_block,
                                                     precision, rows, columns, linear,
                                                     ctypes.byref(r), ctypes.byref(c))
    return None if status != 0 else (r.value, c.value)


# ---- rearranges ----
def rearrange_row_major_f16(src, target_order, matrices, logical_rows, physical_rows,
                            logical_columns, physical_columns, row_block=64,
                            column_block=16) -> np.ndarray:
    s = _c(src, np.uint16).reshape(-1)
    out = np.full(matrices * physical_rows * physical_columns, 0xFFFF, dtype=np.uint16)
    status = lib().or_rearrange_row_major_f16(target_order, row_block, column_block, matrices,
                                              logical_rows, physical_rows, logical_columns,
                                              physical_columns, s.ctypes.data, out.ctypes.data)
    if status != 0:
        raise ValueError(f"oracle rearrange rejected arguments ({status})")
    return out


def unpack_to_row_major_f16(src, source_order, matrices, logical_rows, physical_rows,
                            logical_columns, physical_columns) -> np.ndarray:
    s = _c(src, np.uint16).reshape(-1)
    out = np.full(matrices * physical_rows * physical_columns, 0xFFFF, dtype=np.uint16)
    status = lib().or_unpack_to_row_major_f16(source_order, matrices, logical_rows, physical_rows,
                                              logical_columns, physical_columns, s.ctypes.data,
                                              out.ctypes.data)
    if status != 0:
        raise ValueError(f"oracle unpack rejected arguments ({status})")
    return out


def transpose_u16(src, matrices, rows, columns) -> np.ndarray:
    s = _c(src, np.uint16).reshape(-1)
    out = np.empty_like(s)
    lib().or_transpose_u16(matrices, rows, columns, s.ctypes.data, out.ctypes.data)
    return out


# ---- arithmetic ----
def gemm_f32(left, right, rows, columns, inner, transpose_left=False, transpose_right=False,
             batches=1, left_batch_stride=None, right_batch_stride=None, nthreads=None):
    l, r = _c(left, np.float32).reshape(-1), _c(right, np.float32).reshape(-1)
    out = np.empty(batches * rows * columns, dtype=np.float32)
    lbs = rows * inner if left_batch_stride is None else left_batch_stride
    rbs = inner * columns if right_batch_stride is None else right_batch_stride
    lib().or_gemm_f32(l.ctypes.data, r.ctypes.data, out.ctypes.data, batches, lbs, rbs, rows,
                      columns, inner, int(transpose_left), int(transpose_right),
                      nthreads or threads())
    return out


def gemm_f16(left, right, rows, columns, inner, transpose_left=False, transpose_right=False,
             batches=1, left_batch_stride=None, right_batch_stride=None, nthreads=None):
    l, r = _c(left, np.uint16).reshape(-1), _c(right, np.uint16).reshape(-1)
    out = np.empty(batches * rows * columns, dtype=np.uint16)
    lbs = rows * inner if left_batch_stride is None else left_batch_stride
    rbs = inner * columns if right_batch_stride is None else right_batch_stride
    status = lib().or_gemm_f16(l.ctypes.data, r.ctypes.data, out.ctypes.data, batches, lbs, rbs,
                               rows, columns, inner, int(transpose_left), int(transpose_right),
                               nthreads or threads())
    if status != 0:
        raise MemoryError("oracle gemm_f16 allocation failed")
    return out


def gemm_f16_rows(left, right, rows, columns, inner, row_list, nthreads=None):
    l, r = _c(left, np.uint16).reshape(-1), _c(right, np.uint16).reshape(-1)
    rl = _c(row_list, np.uint32)
    out = np.empty((rl.size, columns), dtype=np.float32)
    status = lib().or_gemm_f16_rows(l.ctypes.data, r.ctypes.data, out.ctypes.data, rows, columns,
                                    inner, rl.ctypes.data, rl.size, nthreads or threads())
    if status != 0:
        raise ValueError("oracle gemm_f16_rows rejected arguments")
    return out


def attention(query, key, value, streams, query_rows, key_rows, width, value_width, causal=False,
              scale=None, row_list=None, nthreads=None):
    q = _c(query, np.float32).reshape(-1)
    k = _c(key, np.float32).reshape(-1)
    v = _c(value, np.float32).reshape(-1)
    if row_list is None:
        n = streams * query_rows
        rl_ptr, rl_n = None, 0
    else:
        rl = _c(row_list, np.uint32)
        n, rl_ptr, rl_n = rl.size, rl.ctypes.data, rl.size
    out = np.empty((n, value_width), dtype=np.float32)
    status = lib().or_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data,
                                streams, query_rows, key_rows, width, value_width, int(causal),
                                float(scale or 0.0), int(scale is not None), rl_ptr, rl_n,
                                nthreads or threads())
    if status != 0:
        raise ValueError("oracle attention rejected arguments")
    return out


def gelu_reference(x: float) -> float:
    return lib().or_gelu_reference(float(x))


def gelu_f16(bits) -> np.ndarray:
    s = _c(bits, np.uint16).reshape(-1)
    out = np.empty_like(s)
    lib().or_gelu_f16(s.ctypes.data, out.ctypes.data, s.size)
    return out


def add_f32(left, right):
    l, r = _c(left, np.float32), _c(right, np.float32)
    ls = (ctypes.c_uint32 * max(1, l.ndim))(*l.shape)
    rs = (ctypes.c_uint32 * max(1, r.ndim))(*r.shape)
    shape = np.broadcast_shapes(l.shape, r.shape)
    out = np.empty(shape, dtype=np.float32)
    os_ = (ctypes.c_uint32 * 16)()
    rank = ctypes.c_int(0)
    status = lib().or_add_f32(l.ctypes.data, ls, l.ndim, r.ctypes.data, rs, r.ndim,
                              out.ctypes.data, os_, ctypes.byref(rank))
    if status != 0:
        raise ValueError("shapes cannot be broadcast")
    return out


def split_heads(x, heads):
    x = _c(x, np.float32)
    b, r, w = x.shape
    out = np.empty((b * heads, r, w // heads), dtype=np.float32)
    if lib().or_split_heads(x.ctypes.data, b, r, w, heads, out.ctypes.data) != 0:
        raise ValueError("width not divisible by heads")
    return out


def reduce_sum_f16(initial, remote, remote_partials, count) -> np.ndarray:
    i, r = _c(initial, np.uint16).reshape(-1), _c(remote, np.uint16).reshape(-1)
    out = np.empty(count, dtype=np.uint16)
    lib().or_reduce_sum_f16(i.ctypes.data, r.ctypes.data, remote_partials, count, out.ctypes.data)
    return out


def reduce_rows_f16(src, rows, columns, nthreads=None) -> np.ndarray:
    s = _c(src, np.uint16).reshape(-1)
    out = np.empty(rows, dtype=np.float32)
    lib().or_reduce_rows_f16(s.ctypes.data, rows, columns, out.ctypes.data, nthreads or threads())
    return out


def reduce_rows_block_major_f16(src, row_block, column_block, rows, columns,
                                nthreads=None) -> np.ndarray:
    s = _c(src, np.uint16).reshape(-1)
    out = np.empty(rows, dtype=np.float32)
    if lib().or_reduce_rows_block_major_f16(s.ctypes.data, row_block, column_block, rows, columns,
                                            out.ctypes.data, nthreads or threads()) != 0:
        raise ValueError("bad block-major shape")
    return out


def splitmix64(state: int) -> int:
    return lib().or_splitmix64(state)


# ---- tiled host bindings (crates/ipu-codegen/src/layout.rs, storage.rs) ----
def _axis_defaults(a: dict) -> dict:
    """AxisTiling::new defaults (layout.rs:169-179) for missing fields."""
    d = dict(a)
    d.setdefault("padding_groups", 1)
    d.setdefault("padding_multiple", d["block_size"])
    d.setdefault("shard_padding_multiple", 1)
    d.setdefault("zero_padding", False)
    d.setdefault("tile_stride", None)
    return d


def _axis_bounds(a: dict, padded_extent: int, logical_extent: int, coordinate: int):
    """resolve_axis_bounds, layout.rs:1427-1504: (start, logical_end,
    physical_end) of partition `coordinate`."""
    partitions, groups = a["partitions"], a["padding_groups"]
    per_group = partitions // groups
    group, in_group = divmod(coordinate, per_group)
    padded_group = padded_extent // groups
    logical_group = logical_extent // groups
    if padded_group % a["block_size"]:
        raise ValueError("indivisible axis")
    blocks = padded_group // a["block_size"]
    short, long_shards = divmod(blocks, per_group)
    start_blocks = in_group * short + min(in_group, long_shards)
    shard_blocks = short + (1 if in_group < long_shards else 0)
    start_in_group = start_blocks * a["block_size"]
    allocated = shard_blocks * a["block_size"]
    rem = allocated % a["shard_padding_multiple"]
    if rem and not a["zero_padding"]:
        raise ValueError("indivisible shard")
    width = allocated + (a["shard_padding_multiple"] - rem if rem else 0)
    base = group * logical_group
    start = base + start_in_group
    logical_end = base + max(min(start_in_group + allocated, logical_group), start_in_group)
    return start, logical_end, start + width


def resolve_tiling(shape, tile_count: int, replicas: int, axes) -> list:
    """Per tile, in logical tile order, the (start, logical_end,
    physical_end) of every axis: ResolvedLayout::resolve and shard_extents
    (layout.rs:1002-1135, 1267-1300).  `axes` are dicts with AxisTiling's
    fields (`axis` as ("end", k) or ("start", k))."""
    rank = len(shape)
    padded = list(shape)
    resolved = []
    used = replicas
    for raw in axes:
        a = _axis_defaults(raw)
        kind, k = a["axis"]
        index = rank - k if kind == "end" else k
        if not (0 <= index < rank) or (kind == "end" and k == 0):
            raise ValueError("axis out of range")
        if any(r["index"] == index for r in resolved):
            raise ValueError("duplicate axis")
        used *= a["partitions"]
        extent = padded[index]
        if a["partitions"] % a["padding_groups"] or extent % a["padding_groups"]:
            raise ValueError("invalid padding groups")
        group_extent = extent // a["padding_groups"]
        rem = group_extent % a["padding_multiple"]
        if rem and not a["zero_padding"]:
            raise ValueError("indivisible axis")
        if rem:
            padded[index] = (group_extent + a["padding_multiple"] - rem) * a["padding_groups"]
        if (padded[index] // a["padding_groups"]) % a["block_size"]:
            raise ValueError("indivisible axis")
        a["index"] = index
        resolved.append(a)
    if used != tile_count:
        raise ValueError("tile count mismatch")
    packed = replicas
    for a in resolved:                       # axis_strides, layout.rs:234-251
        a["stride"] = a["tile_stride"] or packed
        packed *= a["partitions"]
    tiles = []
    for tile in range(tile_count):
        ext = [(0, shape[i], padded[i]) for i in range(rank)]
        for a in resolved:
            c = (tile // a["stride"]) % a["partitions"]
            ext[a["index"]] = _axis_bounds(a, padded[a["index"]], shape[a["index"]], c)
        tiles.append(ext)
    return tiles


ORDER_ROW_MAJOR, ORDER_AMP, ORDER_BLOCK_MAJOR = 0, 1, 2


def pack_tiled(logical, shape, kind: int, variant: int, tile_count: int, replicas: int, axes,
               row_block: int = 0, column_block: int = 0) -> np.ndarray:
    """The host bytes of a tiled binding (CompiledTensor::binding,
    package.rs:2101-2137): every tile's shard in logical tile order, each of
    its physical widths, the logical elements placed by storage.rs's
    physical_index and the padding zero.  kind 0 row-major (any dtype), 1 AMP
    (variant = AmpOrder role), 2 block-major (variant 1 = TransposedMatrix;
    fp16 only for kinds 1 and 2)."""
    x = np.ascontiguousarray(logical).reshape(shape)
    pieces = []
    for ext in resolve_tiling(list(shape), tile_count, replicas, axes):
        widths = [pe - st for st, _, pe in ext]
        shard = np.zeros(widths, dtype=x.dtype)
        if kind == ORDER_ROW_MAJOR:
            region = tuple(slice(st, le) for st, le, _ in ext)
            shard[tuple(slice(0, le - st) for st, le, _ in ext)] = x[region]
        else:
            if x.dtype != np.uint16:
                raise ValueError("AMP and block-major packing is fp16 only")
            rank = len(shape)
            arr = lambda v: (ctypes.c_uint32 * rank)(*v)  # noqa: E731
            flat = shard.reshape(-1)
            src = x.reshape(-1)
            status = lib().or_pack_shard(kind, variant, row_block, column_block, rank,
                                         arr(shape), arr([e[0] for e in ext]),
                                         arr([e[1] for e in ext]), arr([e[2] for e in ext]),
                                         src.ctypes.data, flat.ctypes.data)
            if status != 0:
                raise ValueError(f"oracle pack_shard rejected the shard ({status})")
        pieces.append(shard.reshape(-1))
    return np.concatenate(pieces) if pieces else np.zeros(0, dtype=x.dtype)

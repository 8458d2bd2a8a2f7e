"""ipu-stack for MI355X: Python binding of libipus (ctypes over the C ABI).

libipus.so (built in this directory by ``make``) holds the gfx950 kernels,
the kernel ABI registry, the ComputeGraph / build_package compiler and the
session executor; this module only marshals calls.  There is no CPU path:
every function that computes goes through libipus on a HIP device, and the
module raises if the library or the device is missing.

The API mirrors the reference's ipu-codegen surface
(crates/ipu-codegen/src/graph.rs:249-515, package.rs:532-538) in Python
spelling: ``ComputeGraph``, ``build_package(graph, config)``, plus the
kernel-level ``Context.launch`` that mirrors one ComputeStep
(crates/ipu-codegen/src/kernel.rs:818-865).
"""
from __future__ import annotations

import ctypes
import weakref
import os
import struct
from dataclasses import dataclass, field, replace
from typing import Callable, Iterable, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "libipus.so")

PRECISION_F16 = 1
PRECISION_F32 = 2
ORDER_AMP_LEFT = 0
ORDER_AMP_TRANSPOSED_RIGHT = 1
ORDER_BLOCK_MAJOR = 2
ORDER_ROW_MAJOR = 3
ORDER_AMP_OUTPUT = 4
ORDER_AMP_TRANSPOSED_LEFT = 5
ORDER_AMP_TRANSPOSED_OUTPUT = 6
ORDER_BLOCK_MAJOR_TRANSPOSED = 7
MAX_TILED_AXES = 4

OK = 0
ERROR_INVALID_ARGUMENT = -1
ERROR_POINTER_ARITY = -2
ERROR_UNAVAILABLE = -3
ERROR_UNSUPPORTED_COUNT = -4
ERROR_UNKNOWN_SYMBOL = -5
ERROR_GRAPH = -6
ERROR_BUILD = -7
ERROR_NO_DEVICE = -8
ERROR_OUT_OF_MEMORY = -9
ERROR_TRANSLATED = -10
ERROR_HIP_BASE = -1000

MAX_RANK = 8
MAX_SCALARS = 32


class IpusError(RuntimeError):
    """A libipus call failed; ``status`` is the negative IPUS_ERROR_* code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class GraphError(IpusError):
    """GraphError of crates/ipu-codegen/src/graph.rs:221-245."""


class PackageBuildError(IpusError):
    """PackageBuildError of crates/ipu-codegen/src/package.rs:48-78."""


class KernelAbiError(IpusError):
    """KernelAbiError of crates/ipu-codegen/src/kernel.rs:140-162."""


class _KernelAbiInfo(ctypes.Structure):
    _fields_ = [
        ("symbol", ctypes.c_char_p),
        ("input_count", ctypes.c_int),
        ("scalar_count", ctypes.c_int),
        ("scalar_names", ctypes.c_char_p * MAX_SCALARS),
        ("implemented", ctypes.c_int),
    ]


class _DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("arch", ctypes.c_char * 32),
        ("compute_units", ctypes.c_int),
        ("clock_khz", ctypes.c_int),
        ("memory_clock_khz", ctypes.c_int),
        ("memory_bus_width", ctypes.c_int),
        ("global_memory_bytes", ctypes.c_uint64),
        ("lds_bytes_per_block", ctypes.c_int),
    ]


class _TensorInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("value", ctypes.c_uint32),
        ("rank", ctypes.c_int),
        ("dims", ctypes.c_uint32 * MAX_RANK),
        ("precision", ctypes.c_int),
        ("order", ctypes.c_int),
        ("row_block", ctypes.c_uint32),
        ("column_block", ctypes.c_uint32),
        ("bytes", ctypes.c_uint64),
        ("shards", ctypes.c_uint32),
    ]


class _AxisTiling(ctypes.Structure):
    _fields_ = [("from_end", ctypes.c_int), ("axis", ctypes.c_uint32),
                ("partitions", ctypes.c_uint32), ("padding_groups", ctypes.c_uint32),
                ("block_size", ctypes.c_uint32), ("padding_multiple", ctypes.c_uint32),
                ("shard_padding_multiple", ctypes.c_uint32), ("zero_padding", ctypes.c_int),
                ("tile_stride", ctypes.c_uint32)]


class _TensorFormat(ctypes.Structure):
    _fields_ = [("precision", ctypes.c_int), ("order", ctypes.c_int),
                ("row_block", ctypes.c_uint32), ("column_block", ctypes.c_uint32),
                ("tile_count", ctypes.c_uint32), ("replicas", ctypes.c_uint32),
                ("axis_count", ctypes.c_int), ("axes", _AxisTiling * 4)]


class _InputFormat(ctypes.Structure):
    _fields_ = [("value", ctypes.c_uint32), ("automatic", ctypes.c_int),
                ("format", _TensorFormat)]


class _PackageConfig(ctypes.Structure):
    _fields_ = [("compute_precision", ctypes.c_int), ("attention_output_f16", ctypes.c_int),
                ("input_format_count", ctypes.c_int),
                ("input_formats", ctypes.POINTER(_InputFormat))]


_LIB: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_U32P = ctypes.POINTER(ctypes.c_uint32)
_SIGNATURES = {
    "ipus_last_error": (ctypes.c_char_p, []),
    "ipus_version": (ctypes.c_char_p, []),
    "ipus_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "ipus_context_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_P)]),
    "ipus_context_destroy": (ctypes.c_int, [_P]),
    "ipus_context_device_info": (ctypes.c_int, [_P, ctypes.POINTER(_DeviceInfo)]),
    "ipus_context_stream": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "ipus_buffer_alloc": (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.POINTER(_P)]),
    "ipus_buffer_free": (ctypes.c_int, [_P, _P]),
    "ipus_context_live_buffers": (
        ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "ipus_context_inject_launch_failure": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_int]),
    "ipus_gemm_f16_split_noalloc": (
        ctypes.c_int, [_P, _P, _P, _P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                       ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                       ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int]),
    "ipus_buffer_upload": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t]),
    "ipus_buffer_download": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t]),
    "ipus_buffer_copy": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t]),
    "ipus_buffer_memset": (ctypes.c_int, [_P, _P, ctypes.c_int, ctypes.c_size_t]),
    "ipus_stream_sync": (ctypes.c_int, [_P]),
    "ipus_event_create": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "ipus_event_destroy": (ctypes.c_int, [_P]),
    "ipus_event_record": (ctypes.c_int, [_P, _P]),
    "ipus_event_elapsed_ms": (ctypes.c_int, [_P, _P, ctypes.POINTER(ctypes.c_float)]),
    "ipus_kernel_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "ipus_kernel_abi_at": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_KernelAbiInfo)]),
    "ipus_kernel_abi": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_KernelAbiInfo)]),
    "ipus_validate_kernel_run": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, _U32P,
                                                ctypes.c_int]),
    "ipus_launch": (
        ctypes.c_int,
        [_P, ctypes.c_char_p, _P, ctypes.POINTER(_P), ctypes.c_int, _U32P, ctypes.c_int],
    ),
    "ipus_synth_f16": (
        ctypes.c_int,
        [_P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_float],
    ),
    "ipus_synth_f32": (
        ctypes.c_int,
        [_P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_float],
    ),
    "ipus_graph_create": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "ipus_graph_destroy": (ctypes.c_int, [_P]),
    "ipus_graph_host_input": (ctypes.c_int, [_P, ctypes.c_char_p, _U32P, ctypes.c_int, _U32P]),
    "ipus_graph_parameter": (ctypes.c_int, [_P, ctypes.c_char_p, _U32P, ctypes.c_int, _U32P]),
    "ipus_graph_value_sequence": (
        ctypes.c_int, [_P, ctypes.c_char_p, _U32P, ctypes.c_int, _U32P]),
    "ipus_graph_gemm": (
        ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, _U32P]),
    "ipus_graph_gelu": (ctypes.c_int, [_P, ctypes.c_uint32, _U32P]),
    "ipus_graph_add": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_uint32, _U32P]),
    "ipus_graph_split_heads": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_uint32, _U32P]),
    "ipus_graph_flash_attention": (
        ctypes.c_int,
        [_P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int,
         ctypes.c_uint32, _U32P],
    ),
    "ipus_graph_transpose": (ctypes.c_int, [_P, ctypes.c_uint32, _U32P]),
    "ipus_graph_rearrange": (
        ctypes.c_int,
        [_P, ctypes.c_uint32, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, _U32P],
    ),
    "ipus_graph_reduce_rows": (ctypes.c_int, [_P, ctypes.c_uint32, _U32P]),
    "ipus_graph_repeat_begin": (
        ctypes.c_int,
        [_P, ctypes.c_uint32, _U32P, ctypes.c_int, _U32P, ctypes.c_int, _U32P, ctypes.c_int,
         _U32P],
    ),
    "ipus_graph_repeat_end": (ctypes.c_int, [_P, _U32P, ctypes.c_int, _U32P]),
    "ipus_graph_repeat_abort": (ctypes.c_int, [_P]),
    "ipus_graph_set_outputs": (ctypes.c_int, [_P, _U32P, ctypes.c_int]),
    "ipus_graph_value_shape": (
        ctypes.c_int, [_P, ctypes.c_uint32, _U32P, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "ipus_graph_operation_count": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int)]),
    "ipus_build_package": (ctypes.c_int, [_P, ctypes.POINTER(_PackageConfig), ctypes.POINTER(_P)]),
    "ipus_package_destroy": (ctypes.c_int, [_P]),
    "ipus_package_input_count": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int)]),
    "ipus_package_input_info": (ctypes.c_int, [_P, ctypes.c_int, ctypes.POINTER(_TensorInfo)]),
    "ipus_package_output_count": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int)]),
    "ipus_package_output_info": (ctypes.c_int, [_P, ctypes.c_int, ctypes.POINTER(_TensorInfo)]),
    "ipus_package_step_count": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int)]),
    "ipus_package_step": (
        ctypes.c_int,
        [_P, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int),
         ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_U32P)],
    ),
    "ipus_package_arena_bytes": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "ipus_package_value_precision": (
        ctypes.c_int, [_P, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int)]),
    "ipus_session_create": (ctypes.c_int, [_P, _P, ctypes.POINTER(_P)]),
    "ipus_session_destroy": (ctypes.c_int, [_P]),
    "ipus_session_write": (ctypes.c_int, [_P, ctypes.c_char_p, _P, ctypes.c_size_t]),
    "ipus_session_read": (ctypes.c_int, [_P, ctypes.c_char_p, _P, ctypes.c_size_t]),
    "ipus_session_tensor_pointer": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_P)]),
    "ipus_session_run": (ctypes.c_int, [_P]),
    "ipus_session_capture": (ctypes.c_int, [_P]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Loads libipus.so (once) and declares every C signature.

    Raises FileNotFoundError when the library has not been built: there is
    no fallback implementation.
    """
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    path = path or LIBRARY_PATH
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `make -C {HERE}` (or __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path == LIBRARY_PATH:
        _LIB = lib
    return lib


def _lib() -> ctypes.CDLL:
    return _LIB if _LIB is not None else load_library()


def last_error() -> str:
    return (_lib().ipus_last_error() or b"").decode()


def _check(status: int, kind: type = IpusError) -> None:
    if status != 0:
        if status == ERROR_GRAPH:
            kind = GraphError
        elif status == ERROR_BUILD:
            kind = PackageBuildError
        elif status in (ERROR_POINTER_ARITY, ERROR_UNAVAILABLE, ERROR_UNSUPPORTED_COUNT,
                        ERROR_UNKNOWN_SYMBOL, ERROR_TRANSLATED):
            kind = KernelAbiError
        raise kind(status, last_error())


def _u32_array(values: Iterable[int]):
    values = [int(v) for v in values]
    return (ctypes.c_uint32 * max(1, len(values)))(*values), len(values)


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(_lib().ipus_device_count(ctypes.byref(n)))
    return n.value


# ---------------------------------------------------------------------------
# Kernel ABI registry
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class KernelAbi:
    symbol: str
    input_count: int
    scalar_names: tuple
    implemented: bool


def _abi_from(info: _KernelAbiInfo) -> KernelAbi:
    return KernelAbi(
        info.symbol.decode(), info.input_count,
        tuple(info.scalar_names[i].decode() for i in range(info.scalar_count)),
        bool(info.implemented))


def kernel_symbols() -> list[KernelAbi]:
    n = ctypes.c_int(0)
    _check(_lib().ipus_kernel_count(ctypes.byref(n)))
    out = []
    for i in range(n.value):
        info = _KernelAbiInfo()
        _check(_lib().ipus_kernel_abi_at(i, ctypes.byref(info)))
        out.append(_abi_from(info))
    return out


def kernel_abi(symbol: str) -> KernelAbi:
    info = _KernelAbiInfo()
    _check(_lib().ipus_kernel_abi(symbol.encode(), ctypes.byref(info)))
    return _abi_from(info)


def validate_kernel_run(symbol: str, input_count: int, scalars: Sequence[int]) -> None:
    """validate_kernel_run (crates/ipu-codegen/src/kernel.rs:1384-1435) on
    the host: raises KernelAbiError (or IpusError) with the status that
    ``Context.launch`` would return for the same step, before any device
    work."""
    arr, n = _u32_array(scalars)
    _check(_lib().ipus_validate_kernel_run(symbol.encode(), int(input_count), arr, n))


# ---------------------------------------------------------------------------
# Synthetic inputs
# ---------------------------------------------------------------------------
UNIFORM = 0
NORMAL = 1


def synth_f16(count: int, seed: int, tensor: int, distribution: int = UNIFORM,
              scale: float = 1.0) -> np.ndarray:
    """fp16 bit patterns (uint16) of value(seed, tensor, i), i < count."""
    out = np.empty(int(count), dtype=np.uint16)
    _check(_lib().ipus_synth_f16(out.ctypes.data, int(count), int(seed), int(tensor),
                                 int(distribution), float(scale)))
    return out


def synth_f32(count: int, seed: int, tensor: int, distribution: int = UNIFORM,
              scale: float = 1.0) -> np.ndarray:
    out = np.empty(int(count), dtype=np.float32)
    _check(_lib().ipus_synth_f32(out.ctypes.data, int(count), int(seed), int(tensor),
                                 int(distribution), float(scale)))
    return out


def _f32_bits(value: float) -> int:
    return struct.unpack("<I", struct.pack("<f", float(value)))[0]


def scale_bits(scale: float | None) -> int:
    """Kernel-level scale scalar: AttentionScale::ValueBits (graph.rs:147-165),
    0 = 1/sqrt(width) (a zero scale is never valid)."""
    return 0 if scale is None else _f32_bits(scale)


# ---------------------------------------------------------------------------
# Device context, buffers, launches
# ---------------------------------------------------------------------------
class DeviceBuffer:
    def __init__(self, context: "Context", ptr: int, nbytes: int):
        self.context = context
        self.ptr = ptr
        self.nbytes = nbytes

    def free(self) -> None:
        if self.ptr:
            ptr, self.ptr = self.ptr, 0
            self.context._buffers.discard(self)
            _check(_lib().ipus_buffer_free(self.context.handle, ptr))

    def download(self, dtype, shape=None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        self.context.download_into(self, out)
        return out.reshape(shape) if shape is not None else out


class Context:
    """One HIP device and stream (Runtime::open + HostSession roles)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(_lib().ipus_context_create(int(device), ctypes.byref(h)))
        self.handle = h.value
        self._buffers: set[DeviceBuffer] = set()  # live buffers, freed by close()
        self._sessions: "weakref.WeakSet[Session]" = weakref.WeakSet()  # closed by close()

    def close(self) -> None:
        """Closes the live sessions, frees the live buffers and destroys the
        context; every release runs even after an earlier one failed, and the
        first error is raised afterwards."""
        if self.handle:
            status = 0
            for session in list(self._sessions):
                rc = session._release()
                status = status or rc
            self._sessions.clear()
            handle, self.handle = self.handle, None
            for b in self._buffers:
                if b.ptr:
                    rc = _lib().ipus_buffer_free(handle, b.ptr)
                    status = status or rc
                    b.ptr = 0
            self._buffers.clear()
            rc = _lib().ipus_context_destroy(handle)
            status = status or rc
            _check(status)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_info(self) -> dict:
        info = _DeviceInfo()
        _check(_lib().ipus_context_device_info(self.handle, ctypes.byref(info)))
        return {
            "name": info.name.decode(), "arch": info.arch.decode(),
            "compute_units": info.compute_units, "clock_khz": info.clock_khz,
            "memory_clock_khz": info.memory_clock_khz,
            "memory_bus_width": info.memory_bus_width,
            "global_memory_bytes": info.global_memory_bytes,
            "lds_bytes_per_block": info.lds_bytes_per_block,
        }

    def live_buffers(self) -> tuple[int, int]:
        """(count, bytes) of the buffers allocated through this context and
        not yet freed, sessions' buffers included."""
        n, b = ctypes.c_uint64(), ctypes.c_uint64()
        _check(_lib().ipus_context_live_buffers(self.handle, ctypes.byref(n), ctypes.byref(b)))
        return n.value, b.value

    def inject_launch_failure(self, launches_before: int, status: int) -> None:
        """Test hook: the launch after `launches_before` more launches fails
        with `status` (< 0) without running; 0 cancels."""
        _check(_lib().ipus_context_inject_launch_failure(self.handle, int(launches_before),
                                                         int(status)))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = ctypes.c_void_p()
        _check(_lib().ipus_buffer_alloc(self.handle, int(nbytes), ctypes.byref(p)))
        buf = DeviceBuffer(self, p.value, int(nbytes))
        self._buffers.add(buf)
        return buf

    def upload(self, array: np.ndarray) -> DeviceBuffer:
        array = np.ascontiguousarray(array)
        buf = self.alloc(array.nbytes)
        _check(_lib().ipus_buffer_upload(self.handle, buf.ptr, array.ctypes.data, array.nbytes))
        return buf

    def write(self, buf: DeviceBuffer, array: np.ndarray) -> None:
        array = np.ascontiguousarray(array)
        if array.nbytes > buf.nbytes:
            raise ValueError("array larger than buffer")
        _check(_lib().ipus_buffer_upload(self.handle, buf.ptr, array.ctypes.data, array.nbytes))

    def download_into(self, buf: DeviceBuffer, out: np.ndarray) -> None:
        if not out.flags.c_contiguous or out.nbytes > buf.nbytes:
            raise ValueError("output must be contiguous and fit the buffer")
        _check(_lib().ipus_buffer_download(self.handle, out.ctypes.data, buf.ptr, out.nbytes))

    def memset(self, buf: DeviceBuffer, value: int = 0) -> None:
        _check(_lib().ipus_buffer_memset(self.handle, buf.ptr, int(value), buf.nbytes))

    def sync(self) -> None:
        _check(_lib().ipus_stream_sync(self.handle))

    def stream(self) -> int:
        s = ctypes.c_void_p()
        _check(_lib().ipus_context_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    def launch(self, symbol: str, out, inputs: Sequence, scalars: Sequence[int]) -> None:
        """One ComputeStep: symbol, output pointer, input pointers, u32 scalars."""
        ptrs = [x.ptr if isinstance(x, DeviceBuffer) else int(x) for x in inputs]
        in_arr = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
        sc, n = _u32_array(scalars)
        outp = out.ptr if isinstance(out, DeviceBuffer) else int(out)
        _check(_lib().ipus_launch(self.handle, symbol.encode(), outp, in_arr, len(ptrs), sc, n))

    def gemm_f16_split_noalloc(self, out, left, right, batches, rows, columns, inner,
                               transpose_left=False, transpose_right=False,
                               left_batch_stride=0, right_batch_stride=0, splits=2,
                               gelu=False) -> None:
        """Split-K fp16 GEMM whose partials use the library's per-device
        scratch array (ipus_gemm_f16_split_noalloc): no allocation."""
        ptr = lambda x: x.ptr if isinstance(x, DeviceBuffer) else int(x)  # noqa: E731
        _check(_lib().ipus_gemm_f16_split_noalloc(
            self.handle, ptr(out), ptr(left), ptr(right), int(batches), int(rows), int(columns),
            int(inner), int(bool(transpose_left)), int(bool(transpose_right)),
            int(left_batch_stride), int(right_batch_stride), int(splits), int(bool(gelu))))

    def timer(self) -> "Timer":
        return Timer(self)

    def event_series(self, count: int) -> "EventSeries":
        return EventSeries(self, count)


class Timer:
    """HIP events recorded on the context stream."""

    def __init__(self, context: Context):
        self.context = context
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        _check(_lib().ipus_event_create(context.handle, ctypes.byref(a)))
        _check(_lib().ipus_event_create(context.handle, ctypes.byref(b)))
        self.start_event, self.end_event = a.value, b.value

    def start(self) -> None:
        _check(_lib().ipus_event_record(self.context.handle, self.start_event))

    def stop(self) -> float:
        """Records the end event and returns the elapsed milliseconds."""
        _check(_lib().ipus_event_record(self.context.handle, self.end_event))
        ms = ctypes.c_float(0)
        _check(_lib().ipus_event_elapsed_ms(self.start_event, self.end_event, ctypes.byref(ms)))
        return ms.value

    def close(self) -> None:
        _lib().ipus_event_destroy(self.start_event)
        _lib().ipus_event_destroy(self.end_event)


class EventSeries:
    """`count` HIP events recorded on the context stream between launches:
    event i before launch i and event count - 1 after the last one, so
    durations()[i] is launch i's time on the stream (back-to-back launches)."""

    def __init__(self, context: Context, count: int):
        self.context = context
        self.events = []
        for _ in range(count):
            e = ctypes.c_void_p()
            _check(_lib().ipus_event_create(context.handle, ctypes.byref(e)))
            self.events.append(e.value)

    def record(self, i: int) -> None:
        _check(_lib().ipus_event_record(self.context.handle, self.events[i]))

    def durations(self) -> list:
        """Milliseconds between consecutive events (waits for the last)."""
        out = []
        ms = ctypes.c_float(0)
        for a, b in zip(self.events, self.events[1:]):
            _check(_lib().ipus_event_elapsed_ms(a, b, ctypes.byref(ms)))
            out.append(ms.value)
        return out

    def close(self) -> None:
        for e in self.events:
            _lib().ipus_event_destroy(e)
        self.events = []


# ---------------------------------------------------------------------------
# ComputeGraph (graph.rs) and build_package (package.rs)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class RepeatArguments:
    """graph.rs:196-201."""
    carried: list
    invariants: list
    iterated: list


class RegionBuilder:
    """Body builder handed to ``ComputeGraph.repeat`` (graph.rs:517-632)."""

    def __init__(self, graph: "ComputeGraph"):
        self._graph = graph

    def __getattr__(self, name):
        if name in ("gemm", "gemm_with_options", "gelu", "add", "split_heads", "flash_attention",
                    "flash_attention_with_options", "transpose", "rearrange", "reduce_rows",
                    "value_shape", "repeat"):
            return getattr(self._graph, name)
        raise AttributeError(name)


class ComputeGraph:
    """Structured-SSA graph (crates/ipu-codegen/src/graph.rs:203-515)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _check(_lib().ipus_graph_create(ctypes.byref(h)))
        self.handle = h.value

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                _lib().ipus_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    def _value(self, fn, *args) -> int:
        out = ctypes.c_uint32(0)
        _check(fn(self.handle, *args, ctypes.byref(out)))
        return out.value

    def host_input(self, name: str, shape: Sequence[int]) -> int:
        dims, n = _u32_array(shape)
        return self._value(_lib().ipus_graph_host_input, name.encode(), dims, n)

    def parameter(self, name: str, shape: Sequence[int]) -> int:
        dims, n = _u32_array(shape)
        return self._value(_lib().ipus_graph_parameter, name.encode(), dims, n)

    def value_sequence(self, name: str, values: Sequence[int]) -> int:
        vs, n = _u32_array(values)
        return self._value(_lib().ipus_graph_value_sequence, name.encode(), vs, n)

    def gemm(self, left: int, right: int) -> int:
        return self.gemm_with_options(left, right)

    def gemm_with_options(self, left: int, right: int, transpose_left: bool = False,
                          transpose_right: bool = False) -> int:
        return self._value(_lib().ipus_graph_gemm, left, right, int(transpose_left),
                           int(transpose_right))

    def gelu(self, value: int) -> int:
        return self._value(_lib().ipus_graph_gelu, value)

    def add(self, left: int, right: int) -> int:
        return self._value(_lib().ipus_graph_add, left, right)

    def split_heads(self, value: int, heads: int) -> int:
        return self._value(_lib().ipus_graph_split_heads, value, int(heads))

    def flash_attention(self, query: int, key: int, value: int) -> int:
        return self.flash_attention_with_options(query, key, value)

    def flash_attention_with_options(self, query: int, key: int, value: int,
                                     causal: bool = False, scale: float | None = None) -> int:
        return self._value(_lib().ipus_graph_flash_attention, query, key, value, int(causal),
                           int(scale is not None), 0 if scale is None else _f32_bits(scale))

    def transpose(self, value: int) -> int:
        return self._value(_lib().ipus_graph_transpose, value)

    def rearrange(self, value: int, order: int, row_block: int = 0,
                  column_block: int = 0) -> int:
        return self._value(_lib().ipus_graph_rearrange, value, int(order), int(row_block),
                           int(column_block))

    def reduce_rows(self, value: int) -> int:
        return self._value(_lib().ipus_graph_reduce_rows, value)

    def repeat(self, count: int, carried: Sequence[int], invariants: Sequence[int],
               iterated: Sequence[int], build: Callable) -> list:
        """graph.rs:382-472: ``build(body, arguments) -> yields``."""
        c, nc = _u32_array(carried)
        i, ni = _u32_array(invariants)
        s, ns = _u32_array(iterated)
        args = (ctypes.c_uint32 * max(1, nc + ni + ns))()
        _check(_lib().ipus_graph_repeat_begin(self.handle, int(count), c, nc, i, ni, s, ns, args))
        a = list(args)[: nc + ni + ns]
        arguments = RepeatArguments(a[:nc], a[nc:nc + ni], a[nc + ni:])
        try:
            yields = list(build(RegionBuilder(self), arguments))
        except Exception:
            # Drop the open body so the graph stays usable, then re-raise.
            _lib().ipus_graph_repeat_abort(self.handle)
            raise
        y, ny = _u32_array(yields)
        results = (ctypes.c_uint32 * max(1, ny))()
        _check(_lib().ipus_graph_repeat_end(self.handle, y, ny, results))
        return list(results)[:ny]

    def set_outputs(self, values: Sequence[int]) -> None:
        vs, n = _u32_array(values)
        _check(_lib().ipus_graph_set_outputs(self.handle, vs, n))

    def value_shape(self, value: int) -> tuple | None:
        dims = (ctypes.c_uint32 * MAX_RANK)()
        rank = ctypes.c_int(0)
        status = _lib().ipus_graph_value_shape(self.handle, value, dims, MAX_RANK,
                                               ctypes.byref(rank))
        if status != 0:
            return None
        return tuple(dims[i] for i in range(rank.value))

    def operation_count(self) -> int:
        n = ctypes.c_int(0)
        _check(_lib().ipus_graph_operation_count(self.handle, ctypes.byref(n)))
        return n.value


@dataclass
class PackageConfig:
    """GPU stand-in for PackageConfig (package.rs:89-94): compute precision
    of GEMM / Add and the attention output precision, plus PipelineConfig's
    per-input formats (config.rs:310-320): `with_input(value, format)` makes
    the host write that input in the given TensorFormat (shards in tile
    order, as the reference's binding file), `with_automatic_input(value,
    precision)` fixes only its precision."""
    compute_precision: str = "f16"
    attention_output_f16: bool = False
    inputs: dict = field(default_factory=dict)            # value -> TensorFormat
    automatic_inputs: dict = field(default_factory=dict)  # value -> precision

    def with_input(self, value: int, fmt: "TensorFormat") -> "PackageConfig":
        self.inputs[value] = fmt
        self.automatic_inputs.pop(value, None)
        return self

    def with_automatic_input(self, value: int, precision: int) -> "PackageConfig":
        self.automatic_inputs[value] = precision
        self.inputs.pop(value, None)
        return self


# ---------------------------------------------------------------------------
# Tensor formats of host-bound inputs (crates/ipu-codegen/src/layout.rs)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class TensorAxis:
    """TensorAxis::FromStart(i) / FromEnd(i) (layout.rs:115-131)."""
    index: int
    from_end: bool = True

    @staticmethod
    def from_start(i: int) -> "TensorAxis":
        return TensorAxis(i, False)

    @staticmethod
    def from_end_(i: int) -> "TensorAxis":
        return TensorAxis(i, True)


PADDING_REJECT, PADDING_ZERO = 0, 1


@dataclass(frozen=True)
class AxisTiling:
    """AxisTiling (layout.rs:140-197): AxisTiling(axis, partitions,
    block_size, padding) with the builder methods' fields."""
    axis: TensorAxis
    partitions: int
    block_size: int
    padding: int = PADDING_REJECT
    padding_groups: int = 1
    padding_multiple: int = 0            # 0: block_size (AxisTiling::new)
    shard_padding_multiple: int = 1
    tile_stride: int = 0                 # 0: packed after replicas and preceding axes

    def with_tile_stride(self, stride: int) -> "AxisTiling":
        return replace(self, tile_stride=stride)

    def with_padding_multiple(self, m: int) -> "AxisTiling":
        return replace(self, padding_multiple=m)

    def with_shard_padding_multiple(self, m: int) -> "AxisTiling":
        return replace(self, shard_padding_multiple=m)

    def with_padding_groups(self, g: int) -> "AxisTiling":
        return replace(self, padding_groups=g)


@dataclass(frozen=True)
class Layout:
    """Layout{order, tiling} (layout.rs:268-275) with the constructors the
    reference uses for host-bound inputs.  `order` is an ORDER_* code;
    row_block / column_block belong to the block-major orders."""
    order: int
    tile_count: int = 1
    replicas: int = 1
    axes: tuple = ()
    row_block: int = 0
    column_block: int = 0

    @staticmethod
    def row_major(tile_count: int = 1, axes=(), replicas: int = 1) -> "Layout":
        return Layout(ORDER_ROW_MAJOR, tile_count, replicas, tuple(axes))

    @staticmethod
    def row_sharded(tile_count: int) -> "Layout":            # layout.rs:297-299
        return Layout.row_major(tile_count, [AxisTiling(TensorAxis(2), tile_count, 1)])

    @staticmethod
    def head_sharded(tile_count: int) -> "Layout":           # layout.rs:301-303
        return Layout.row_major(tile_count, [AxisTiling(TensorAxis(3), tile_count, 1)])

    @staticmethod
    def _attention_tiling(heads: int, query_partitions: int) -> tuple:  # layout.rs:305-316
        return (AxisTiling(TensorAxis(2), query_partitions, 1).with_tile_stride(heads),
                AxisTiling(TensorAxis(3), heads, 1).with_tile_stride(1))

    @staticmethod
    def attention_query(heads: int, query_partitions: int) -> "Layout":  # layout.rs:318-332
        axes = Layout._attention_tiling(heads, query_partitions) + (
            AxisTiling(TensorAxis(1), 1, 16, PADDING_ZERO),)
        return Layout(ORDER_AMP_LEFT, heads * query_partitions, 1, axes)

    @staticmethod
    def attention_key(heads: int, key_partitions: int) -> "Layout":      # layout.rs:334-356
        axes = (AxisTiling(TensorAxis(3), heads, 1).with_tile_stride(1),
                AxisTiling(TensorAxis(2), key_partitions, 64, PADDING_ZERO).with_tile_stride(heads),
                AxisTiling(TensorAxis(1), 1, 16, PADDING_ZERO))
        return Layout(ORDER_AMP_TRANSPOSED_RIGHT, heads * key_partitions, 1, axes)

    @staticmethod
    def attention_block_major_key_value(heads: int, key_partitions: int) -> "Layout":
        return replace(Layout.attention_key(heads, key_partitions), order=ORDER_BLOCK_MAJOR,
                       row_block=64, column_block=16)                   # layout.rs:358-365

    @staticmethod
    def attention_output(heads: int, query_partitions: int) -> "Layout":  # layout.rs:367-375
        axes = Layout._attention_tiling(heads, query_partitions) + (
            AxisTiling(TensorAxis(1), 1, 16, PADDING_ZERO),)
        return Layout(ORDER_ROW_MAJOR, heads * query_partitions, 1, axes)

    @staticmethod
    def amp_left(inner: int, tile_count: int) -> "Layout":              # layout.rs:376-389
        return Layout(ORDER_AMP_LEFT, tile_count, 1,
                      (AxisTiling(TensorAxis(2), tile_count, 1),
                       AxisTiling(TensorAxis(1), 1, inner, PADDING_ZERO)))

    @staticmethod
    def amp_output(tile_count: int) -> "Layout":                        # layout.rs:402-418
        return Layout(ORDER_AMP_OUTPUT, tile_count, 1,
                      (AxisTiling(TensorAxis(2), tile_count, 1),
                       AxisTiling(TensorAxis(1), 1, 64, PADDING_ZERO)))

    @staticmethod
    def block_major_matrix(row_block: int, tile_count: int) -> "Layout":  # layout.rs:391-400
        return Layout.block_major_matrix_storage(row_block, 64, tile_count, 1, 1)

    @staticmethod
    def block_major_matrix_storage(inner_block: int, output_column_block: int,
                                   column_partitions: int, inner_partitions: int,
                                   copies: int) -> "Layout":              # layout.rs:552-590
        axes = (AxisTiling(TensorAxis(1), column_partitions, output_column_block,
                           PADDING_ZERO).with_tile_stride(1),
                AxisTiling(TensorAxis(2), inner_partitions, inner_block, PADDING_ZERO))
        return Layout(ORDER_BLOCK_MAJOR, column_partitions * inner_partitions * copies, copies,
                      axes, inner_block, 16)

    @staticmethod
    def transposed_block_major_matrix_storage(inner_block: int, output_column_block: int,
                                              column_partitions: int, inner_partitions: int,
                                              copies: int) -> "Layout":   # layout.rs:592-630
        axes = (AxisTiling(TensorAxis(2), column_partitions, output_column_block,
                           PADDING_ZERO).with_tile_stride(1),
                AxisTiling(TensorAxis(1), inner_partitions, inner_block, PADDING_ZERO))
        return Layout(ORDER_BLOCK_MAJOR_TRANSPOSED,
                      column_partitions * inner_partitions * copies, copies, axes, inner_block, 16)


@dataclass(frozen=True)
class TensorFormat:
    """TensorFormat{precision, layout} (layout.rs:808-811)."""
    precision: int
    layout: Layout

    def _c(self) -> _TensorFormat:
        L = self.layout
        if len(L.axes) > MAX_TILED_AXES:
            raise ValueError(f"at most {MAX_TILED_AXES} tiled axes")
        f = _TensorFormat(int(self.precision), int(L.order), int(L.row_block),
                          int(L.column_block), int(L.tile_count), int(L.replicas), len(L.axes))
        for i, a in enumerate(L.axes):
            f.axes[i] = _AxisTiling(int(a.axis.from_end), int(a.axis.index), int(a.partitions),
                                    int(a.padding_groups), int(a.block_size),
                                    int(a.padding_multiple), int(a.shard_padding_multiple),
                                    int(a.padding), int(a.tile_stride))
        return f


@dataclass(frozen=True)
class CompiledTensor:
    """Binding metadata (CompiledTensor, package.rs:131-145)."""
    name: str
    value: int
    shape: tuple
    precision: int
    order: int
    row_block: int
    column_block: int
    nbytes: int
    shards: int = 1

    @property
    def dtype(self):
        return np.float32 if self.precision == PRECISION_F32 else np.uint16


def _tensor(info: _TensorInfo) -> CompiledTensor:
    return CompiledTensor(info.name.decode(), info.value,
                          tuple(info.dims[i] for i in range(info.rank)), info.precision,
                          info.order, info.row_block, info.column_block, info.bytes,
                          info.shards)


class CompiledPackage:
    def __init__(self, handle: int):
        self.handle = handle
        lib = _lib()
        n = ctypes.c_int(0)
        _check(lib.ipus_package_input_count(handle, ctypes.byref(n)))
        self.inputs = []
        for i in range(n.value):
            info = _TensorInfo()
            _check(lib.ipus_package_input_info(handle, i, ctypes.byref(info)))
            self.inputs.append(_tensor(info))
        _check(lib.ipus_package_output_count(handle, ctypes.byref(n)))
        self.outputs = []
        for i in range(n.value):
            info = _TensorInfo()
            _check(lib.ipus_package_output_info(handle, i, ctypes.byref(info)))
            self.outputs.append(_tensor(info))
        _check(lib.ipus_package_step_count(handle, ctypes.byref(n)))
        self.steps = []
        for i in range(n.value):
            sym = ctypes.c_char_p()
            ni, ns = ctypes.c_int(0), ctypes.c_int(0)
            sc = _U32P()
            _check(lib.ipus_package_step(handle, i, ctypes.byref(sym), ctypes.byref(ni),
                                         ctypes.byref(ns), ctypes.byref(sc)))
            self.steps.append((sym.value.decode(), ni.value,
                               tuple(sc[k] for k in range(ns.value))))
        a = ctypes.c_uint64(0)
        _check(lib.ipus_package_arena_bytes(handle, ctypes.byref(a)))
        self.arena_bytes = a.value

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                _lib().ipus_package_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    def precision(self, value: int) -> int:
        p = ctypes.c_int(0)
        _check(_lib().ipus_package_value_precision(self.handle, value, ctypes.byref(p)))
        return p.value

    def session(self, context: Context) -> "Session":
        return Session(context, self)


def build_package(graph: ComputeGraph, config: PackageConfig | None = None) -> CompiledPackage:
    """package.rs:532-538 for the GPU plan."""
    config = config or PackageConfig()
    entries = [_InputFormat(int(v), 0, f._c()) for v, f in config.inputs.items()]
    for v, prec in config.automatic_inputs.items():
        fmt = _TensorFormat()
        fmt.precision = int(prec)
        fmt.order = ORDER_ROW_MAJOR
        fmt.tile_count = fmt.replicas = 1
        entries.append(_InputFormat(int(v), 1, fmt))
    arr = (_InputFormat * max(1, len(entries)))(*entries)
    c = _PackageConfig(PRECISION_F32 if config.compute_precision == "f32" else PRECISION_F16,
                       int(config.attention_output_f16), len(entries),
                       ctypes.cast(arr, ctypes.POINTER(_InputFormat)))
    h = ctypes.c_void_p()
    _check(_lib().ipus_build_package(graph.handle, ctypes.byref(c), ctypes.byref(h)))
    return CompiledPackage(h.value)


class Session:
    """Device buffers for one package (HostSession role)."""

    def __init__(self, context: Context, package: CompiledPackage):
        self.context = context
        self.package = package
        h = ctypes.c_void_p()
        _check(_lib().ipus_session_create(context.handle, package.handle, ctypes.byref(h)))
        self.handle = h.value
        self._meta = {t.name: t for t in package.inputs + package.outputs}
        context._sessions.add(self)

    def _release(self) -> int:
        """Destroys the C session once; returns its status (0 if already closed)."""
        if not self.handle:
            return 0
        handle, self.handle = self.handle, None
        self.context._sessions.discard(self)
        return _lib().ipus_session_destroy(handle)

    def close(self) -> None:
        _check(self._release())

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def write(self, name: str, array: np.ndarray) -> None:
        array = np.ascontiguousarray(array)
        _check(_lib().ipus_session_write(self.handle, name.encode(), array.ctypes.data,
                                         array.nbytes))

    def read(self, name: str) -> np.ndarray:
        meta = self._meta[name]
        out = np.empty(meta.shape, dtype=meta.dtype)
        _check(_lib().ipus_session_read(self.handle, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def pointer(self, name: str) -> int:
        p = ctypes.c_void_p()
        _check(_lib().ipus_session_tensor_pointer(self.handle, name.encode(), ctypes.byref(p)))
        return p.value

    def run(self) -> None:
        _check(_lib().ipus_session_run(self.handle))

    def capture(self) -> None:
        """Record the package's launches as a HIP graph; later runs replay it."""
        _check(_lib().ipus_session_capture(self.handle))

    def run_sync(self) -> None:
        self.run()
        self.context.sync()

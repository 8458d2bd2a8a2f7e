"""CPU checks of the C-ABI boundary: the library loads, exports every entry
point declared in include/*.h, its kernel registry mirrors the reference's
ABI table, and host-side errors surface as status codes (no GPU needed)."""
from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions() -> set[str]:
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(ipus_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol(ipus):
    lib = ctypes.CDLL(ipus.LIBRARY_PATH)
    declared = declared_functions()
    assert len(declared) > 50
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol(ipus):
    assert declared_functions() == set(ipus.EXPORTED_SYMBOLS)


def test_rust_binding_block_covers_every_declared_symbol():
    """The integration guide's Rust extern "C" block (what a Rust caller
    links against) declares every entry point of include/*.h and nothing
    else."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    rust = set(re.findall(r"pub fn (ipus_[a-z0-9_]+)\(", text))
    assert rust == declared_functions()


def test_version(ipus):
    assert "gfx950" in ipus._lib().ipus_version().decode()


# kernel.rs:1215-1382: symbol -> (pointer inputs, scalar names) for the kernels
# that have a reference counterpart.
REFERENCE_ABI = {
    "ipu_stack_gelu_tanh_approx_f16": (1, ("element_count",)),
    "ipu_stack_reduce_sum_f16": (2, ("num_partials", "element_count")),
    "ipu_stack_flash_attention_online_f16": (3, None),
    "ipu_stack_gemm_f16": (2, None),
    "ipu_stack_gemm_f32": (2, None),
    "ipu_stack_rearrange_row_major_f16": (1, None),
    "ipu_stack_unpack_amp_f16": (1, None),
    "ipu_stack_fill_zero": (0, None),
    "ipu_stack_add_f16": (2, ("element_count", "left_broadcast_stride", "right_broadcast_stride")),
    "ipu_stack_add_f32": (2, ("element_count", "left_broadcast_stride", "right_broadcast_stride")),
}


def test_kernel_registry_matches_reference_abi(ipus):
    table = {k.symbol: k for k in ipus.kernel_symbols()}
    for symbol, (inputs, scalars) in REFERENCE_ABI.items():
        assert symbol in table, symbol
        assert table[symbol].input_count == inputs
        if scalars is not None:
            assert table[symbol].scalar_names == scalars
        assert table[symbol].implemented
    # Rearrange scalars start with the reference's five (kernel.rs:1351-1361).
    assert table["ipu_stack_rearrange_row_major_f16"].scalar_names[:5] == (
        "logical_rows", "physical_rows", "target_order", "logical_columns", "physical_columns")
    # Unpack scalars start with the reference's five (kernel.rs:1327-1336).
    assert table["ipu_stack_unpack_amp_f16"].scalar_names[:5] == (
        "matrices", "logical_rows", "physical_rows", "logical_columns", "physical_columns")
    # Attention shape fields follow AttentionKernelShape (kernel.rs:121-129).
    assert table["ipu_stack_flash_attention_online_f16"].scalar_names[:6] == (
        "matrices", "query_rows", "key_rows", "query_dimension", "value_dimension", "scale_bits")


def test_unknown_symbol_abi(ipus):
    with pytest.raises(ipus.KernelAbiError) as e:
        ipus.kernel_abi("ipu_stack_no_such_kernel")
    assert e.value.status == ipus.ERROR_UNKNOWN_SYMBOL
    # the reference's own placeholder for a missing kernel is known, and
    # unavailable (kernel.rs:1252-1259)
    with pytest.raises(ipus.KernelAbiError) as e:
        ipus.kernel_abi("ipu_stack_unsupported_gelu")
    assert e.value.status == ipus.ERROR_UNAVAILABLE


def test_launch_without_context_is_rejected(ipus):
    lib = ipus._lib()
    status = lib.ipus_launch(None, b"ipu_stack_gemm_f16", None, None, 0, None, 0)
    assert status == ipus.ERROR_INVALID_ARGUMENT
    assert "context" in ipus.last_error()


def test_null_arguments_are_rejected(ipus):
    lib = ipus._lib()
    assert lib.ipus_device_count(None) == ipus.ERROR_INVALID_ARGUMENT
    assert lib.ipus_context_create(0, None) == ipus.ERROR_INVALID_ARGUMENT
    assert lib.ipus_buffer_alloc(None, 16, None) == ipus.ERROR_INVALID_ARGUMENT
    assert lib.ipus_stream_sync(None) == ipus.ERROR_INVALID_ARGUMENT


def test_synth_is_deterministic_and_matches_splitmix(ipus, oracle):
    a = ipus.synth_f16(4096, 99, 3, ipus.UNIFORM)
    b = ipus.synth_f16(4096, 99, 3, ipus.UNIFORM)
    assert (a == b).all()
    # uniform value i is 2 * (top 24 bits of SplitMix64(seed ^ tensor << 48 ^ i)) / 2^24 - 1
    import numpy as np
    for i in (0, 1, 17, 4095):
        z = oracle.splitmix64(99 ^ (3 << 48) ^ i)
        expect = np.float32(2.0 * ((z >> 40) / 16777216.0) - 1.0)
        assert a[i] == oracle.f32_to_f16(np.array([expect]))[0]
    n = ipus.synth_f32(1 << 16, 5, 1, ipus.NORMAL)
    assert abs(float(n.mean())) < 0.02 and abs(float(n.std()) - 1.0) < 0.02


def test_failure_injection_and_live_buffer_calls_validate_arguments(ipus):
    """The test hooks exist in the C ABI and reject a null context on the CPU
    (their GPU behaviour is covered by the package tests)."""
    lib = ipus._lib()
    assert lib.ipus_context_inject_launch_failure(None, 0, -1) == ipus.ERROR_INVALID_ARGUMENT
    n = ipus.ctypes.c_uint64()
    assert lib.ipus_context_live_buffers(None, ipus.ctypes.byref(n), ipus.ctypes.byref(n)) == \
        ipus.ERROR_INVALID_ARGUMENT

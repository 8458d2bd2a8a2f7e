"""Reference-shaped kernel calls against the C ABI's run validation (CPU).

Each case builds the (symbol, pointer count, scalars) of one reference
ComputeStep the way the reference computes them for a KernelRun:
symbols from KernelBuildPlan::from_program / tile_kernel_abi
(crates/ipu-codegen/src/kernel.rs:178-193, 321-328, 374-379, 506-517,
626-633, 1215-1382) and scalars from scalar_values (kernel.rs:1149-1193),
with the shard extents a lowering would give the run.  Every reference
kernel family appears once: it is either accepted by
ipus_validate_kernel_run (the host half of ipus_launch, run before any
device work) or refused with a status that says why
(IPUS_ERROR_TRANSLATED: translated per operator; IPUS_ERROR_UNAVAILABLE:
the reference has no device kernel for it either).  The GPU half, launching
the accepted per-shape symbols, is tests/test_gpu_reference_calls.py.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import pytest

F16, F32 = 2, 4  # Precision::bytes()


@dataclass
class Extent:
    """ShardExtent{start, logical_end, physical_end} of one view axis."""
    start: int
    logical_end: int
    physical_end: int


def ext(logical: int, physical: int | None = None) -> Extent:
    return Extent(0, logical, logical if physical is None else physical)


@dataclass
class Run:
    """The parts of a KernelRun that scalar_values reads."""
    output: list          # output view extents
    inputs: list          # per operand, its (single) view's extents
    output_bytes: int     # output precision bytes


def element_count(run: Run) -> int:
    """kernel.rs:1195-1201: product of the output's physical extents."""
    n = 1
    for e in run.output:
        n *= e.physical_end - e.start
    return n


def matrix_extent(extents, logical: bool, columns: bool) -> int:
    """kernel.rs:1087-1098 (output) / 1100-1112 (first input)."""
    e = extents[-1 if columns else -2]
    return (e.logical_end if logical else e.physical_end) - e.start


def matrix_count(run: Run) -> int:
    """kernel.rs:1108-1121: product of the first input's leading axes."""
    n = 1
    for e in run.inputs[0][:-2]:
        n *= e.physical_end - e.start
    return n


def scalar_values(run: Run, names, kernel: dict) -> list[int]:
    """kernel.rs:1149-1193 for the scalar names this ABI lists."""
    count = element_count(run)
    out = []
    for name in names:
        if name == "element_count":
            out.append(count)
        elif name == "num_partials":
            out.append(kernel["partials"] - 1)
        elif name == "words_per_worker":
            out.append(count * run.output_bytes // 8 // 6)
        elif name == "remainder_workers":
            out.append(count * run.output_bytes // 8 % 6)
        elif name == "logical_rows":
            out.append(matrix_extent(run.output, True, False))
        elif name == "physical_rows":
            out.append(matrix_extent(run.output, False, False))
        elif name == "matrices":
            out.append(matrix_count(run))
        elif name == "logical_columns":
            out.append(matrix_extent(run.output, True, True))
        elif name == "physical_columns":
            out.append(matrix_extent(run.output, False, True))
        elif name == "target_order":
            out.append(kernel["order"])
        else:
            # Add's broadcast strides have no arm in scalar_values: the
            # reference cannot materialize an Add step (KernelAvailability::
            # Required, kernel.rs:1275-1287); this ABI takes them as given.
            out.append(kernel[name])
    return out


def rearrangement_specialization(order, lr, pr, lc, pc):
    """kernel.rs:1123-1146."""
    if pr == 64 and lr < pr and order in (1, 2):
        return order, 0, pr, 0, pc
    return order, lr, pr, lc, pc


def rearrange_call(lr, pr, lc, pc, order):
    """Row-major -> AMP-Left (0) / AMP-TransposedRight (1) / block-major (2):
    symbol kernel.rs:374-379, scalars kernel.rs:1351-1361."""
    run = Run([ext(lr, pr), ext(lc, pc)], [[ext(lr, pr), ext(lc, pc)]], F16)
    o, a, b, c, d = rearrangement_specialization(order, lr, pr, lc, pc)
    symbol = f"ipu_stack_rearrange_row_major_to_amp_f16_o{o}_r{a}_p{b}_c{c}_p{d}"
    names = ("logical_rows", "physical_rows", "target_order", "logical_columns",
             "physical_columns")
    return symbol, 1, scalar_values(run, names, {"order": order})


def unpack_call(matrices, lr, pr, lc, pc, source):
    """AMP-Output (0) / AMP-TransposedLeft (1) -> row-major: the staging
    shard keeps the source's extents (low.rs:1150-1157); symbol from the
    input view (kernel.rs:321-328, 797-803), scalars kernel.rs:1327-1336."""
    view = [ext(matrices), ext(lr, pr), ext(lc, pc)]
    run = Run(view, [view], F16)
    symbol = f"ipu_stack_unpack_amp_to_row_major_f16_o{source}_r{lr}_p{pr}_c{lc}_p{pc}"
    names = ("matrices", "logical_rows", "physical_rows", "logical_columns", "physical_columns")
    return symbol, 1, scalar_values(run, names, {})


def attention_call(matrices, q, k, d, v, scale=None):
    """kernel.rs:506-517 suffix from attention_shape (986-1040), no scalars."""
    s = scale if scale is not None else 1.0 / (d ** 0.5)
    bits = struct.unpack("<I", struct.pack("<f", s))[0]
    return f"ipu_stack_flash_attention_online_f16_m{matrices}_q{q}_k{k}_d{d}_v{v}_{bits:08x}", 3, []


def gemm_call(prefix, mode, size, interleaved, k, c, small, large):
    """specialized_gemm_symbol (kernel.rs:178-193); no scalars for f16/f32."""
    suffix = "_interleaved" if interleaved else ""
    return (f"ipu_stack_gemm_{prefix}_{mode}_{size}_rows{suffix}_k{k}_c{c}_r{small}_r{large}",
            2, [])


def fill_zero_call(nbytes):
    run = Run([ext(nbytes // 4)], [], F32)  # e.g. an f32 shard of nbytes
    return "ipu_stack_fill_zero_u64", 0, scalar_values(
        run, ("words_per_worker", "remainder_workers"), {})


ACCEPTED = {
    "fill_zero_48": fill_zero_call(48),
    "fill_zero_4104": fill_zero_call(4104),
    "gelu": ("ipu_stack_gelu_tanh_approx_f16", 1,
             scalar_values(Run([ext(64), ext(64)], [[ext(64), ext(64)]], F16),
                           ("element_count",), {})),
    "reduce_sum": ("ipu_stack_reduce_sum_f16", 2,
                   scalar_values(Run([ext(1024)], [[ext(1024)], [ext(3072)]], F16),
                                 ("num_partials", "element_count"), {"partials": 4})),
    "cast_f16_f32": ("ipu_stack_cast_f16_f32", 1,
                     scalar_values(Run([ext(96)], [[ext(96)]], F32), ("element_count",), {})),
    "cast_f32_f16": ("ipu_stack_cast_f32_f16", 1,
                     scalar_values(Run([ext(96)], [[ext(96)]], F16), ("element_count",), {})),
    "add_f16": ("ipu_stack_add_f16", 2,
                scalar_values(Run([ext(4), ext(64)], [[ext(4), ext(64)], [ext(64)]], F16),
                              ("element_count", "left_broadcast_stride",
                               "right_broadcast_stride"),
                              {"left_broadcast_stride": 256, "right_broadcast_stride": 64})),
    "add_f32": ("ipu_stack_add_f32", 2,
                scalar_values(Run([ext(256)], [[ext(256)], [ext(256)]], F32),
                              ("element_count", "left_broadcast_stride",
                               "right_broadcast_stride"),
                              {"left_broadcast_stride": 256, "right_broadcast_stride": 256})),
    # the GEMM right operand's block-major conversion (64 x 16 blocks)
    "rearrange_block_major": rearrange_call(64, 64, 4096, 4096, 2),
    "rearrange_block_major_ragged": rearrange_call(40, 64, 100, 112, 2),
    "rearrange_amp_left": rearrange_call(729, 736, 1152, 1152, 0),
    "rearrange_amp_left_padded_columns": rearrange_call(19, 19, 72, 80, 0),
    "rearrange_transposed_right": rearrange_call(64, 64, 16, 16, 1),
    "rearrange_transposed_right_ragged": rearrange_call(50, 64, 32, 32, 1),
    "unpack_amp_output": unpack_call(1, 729, 736, 1152, 1152, 0),
    "unpack_amp_transposed_left": unpack_call(4, 30, 32, 40, 48, 1),
    "attention_smoke": attention_call(4, 17, 19, 72, 72),
    "attention_scaled": attention_call(128, 2048, 2048, 128, 128, scale=0.05),
}

REFUSED = {
    # tile GEMM codelets: translated to one operator-level launch
    "gemm_f16_init": (gemm_call("f16", "init", "small", False, 64, 64, 16, 32), "TRANSLATED"),
    "gemm_f16_accumulate": (gemm_call("f16", "accumulate", "large", False, 64, 64, 16, 32),
                            "TRANSLATED"),
    "gemm_f16_interleaved": (gemm_call("f16", "init", "large", True, 64, 128, 8, 8),
                             "TRANSLATED"),
    "gemm_f32_init": (gemm_call("f32", "init", "small", False, 64, 64, 32, 64), "TRANSLATED"),
    "gemm_f32_accumulate": (gemm_call("f32", "accumulate", "small", False, 64, 64, 32, 64),
                            "TRANSLATED"),
    # staged attention codelets (kernel.rs:626-633): one fused launch instead
    "attention_softmax": (("ipu_stack_attention_softmax_small_query_large_key_f16", 1, []),
                          "TRANSLATED"),
    "attention_merge": (("ipu_stack_attention_merge_large_query_f16", 2, [1, 0]), "TRANSLATED"),
    # KernelAvailability::Required in the reference as well
    "gemm_f8": (("ipu_stack_gemm_f8_init", 2, [3]), "UNAVAILABLE"),
    "cast_f8": (("ipu_stack_cast_f8_f16", 1, [64]), "UNAVAILABLE"),
    "cast_identity": (("ipu_stack_cast_identity", 1, [64]), "UNAVAILABLE"),
    "unsupported_gelu": (("ipu_stack_unsupported_gelu", 1, [64]), "UNAVAILABLE"),
    "generic_rearrange": (("ipu_stack_rearrange", 1, []), "UNAVAILABLE"),
}


@pytest.mark.parametrize("name", sorted(ACCEPTED))
def test_reference_call_is_accepted(ipus, name):
    symbol, inputs, scalars = ACCEPTED[name]
    ipus.validate_kernel_run(symbol, inputs, scalars)
    abi = ipus.kernel_abi(symbol)
    assert abi.symbol == symbol and abi.input_count == inputs
    assert len(abi.scalar_names) == len(scalars) and abi.implemented


@pytest.mark.parametrize("name", sorted(REFUSED))
def test_reference_call_is_listed_as_not_forwarded(ipus, name):
    (symbol, inputs, scalars), why = REFUSED[name]
    status = getattr(ipus, f"ERROR_{why}")
    with pytest.raises(ipus.KernelAbiError) as e:
        ipus.validate_kernel_run(symbol, inputs, scalars)
    assert e.value.status == status
    if why == "TRANSLATED":
        assert "translated" in e.value.message
    with pytest.raises(ipus.KernelAbiError):
        ipus.kernel_abi(symbol)


def test_reference_fill_zero_covers_every_byte():
    """words_per_worker and remainder_workers recombine to the byte count."""
    for nbytes in (8, 40, 48, 56, 4104, 1 << 20):
        _, _, (w, r) = fill_zero_call(nbytes)
        assert 8 * (6 * w + r) == nbytes and r < 6


def test_reference_calls_validation_rejects_what_validate_kernel_run_rejects(ipus):
    """validate_kernel_run's own refusals (kernel.rs:1384-1435) and the
    per-shape suffix agreement."""
    bad = [
        ("ipu_stack_gelu_tanh_approx_f16", 1, [63], ipus.ERROR_UNSUPPORTED_COUNT),
        ("ipu_stack_reduce_sum_f16", 2, [0, 64], ipus.ERROR_UNSUPPORTED_COUNT),   # 1 partial
        ("ipu_stack_reduce_sum_f16", 2, [3, 60], ipus.ERROR_UNSUPPORTED_COUNT),   # count % 8
        ("ipu_stack_gelu_tanh_approx_f16", 2, [64], ipus.ERROR_POINTER_ARITY),
        ("ipu_stack_fill_zero_u64", 0, [1, 6], ipus.ERROR_INVALID_ARGUMENT),
        # scalars that disagree with the suffix's shape
        ("ipu_stack_rearrange_row_major_to_amp_f16_o0_r64_p64_c64_p64", 1,
         [64, 64, 1, 64, 64], ipus.ERROR_INVALID_ARGUMENT),
        ("ipu_stack_rearrange_row_major_to_amp_f16_o2_r0_p64_c0_p128", 1,
         [40, 48, 2, 100, 128], ipus.ERROR_INVALID_ARGUMENT),
        ("ipu_stack_unpack_amp_to_row_major_f16_o1_r30_p32_c40_p48", 1,
         [4, 30, 32, 40, 40], ipus.ERROR_INVALID_ARGUMENT),
        ("ipu_stack_unpack_amp_to_row_major_f16_o2_r16_p16_c16_p16", 1,
         [1, 16, 16, 16, 16], ipus.ERROR_INVALID_ARGUMENT),
        # malformed suffixes
        ("ipu_stack_flash_attention_online_f16_m1_q2_k3_d4_v4_3DF1A952", 3, [],
         ipus.ERROR_UNKNOWN_SYMBOL),
        ("ipu_stack_flash_attention_online_f16_m1_q2_k3_d4_v4", 3, [], ipus.ERROR_UNKNOWN_SYMBOL),
        ("ipu_stack_rearrange_row_major_to_amp_f16_o0_r-1_p64_c64_p64", 1, [0, 64, 0, 64, 64],
         ipus.ERROR_UNKNOWN_SYMBOL),
        ("ipu_stack_unpack_amp_to_row_major_f16_o0_r99999999999_p16_c16_p16", 1,
         [1, 16, 16, 16, 16], ipus.ERROR_UNKNOWN_SYMBOL),
    ]
    for symbol, inputs, scalars, status in bad:
        with pytest.raises(ipus.IpusError) as e:
            ipus.validate_kernel_run(symbol, inputs, scalars)
        assert e.value.status == status, (symbol, e.value)


def test_every_reference_family_is_covered():
    """One case per tile_kernel_abi arm (kernel.rs:1223-1370) and per plan
    specialization (kernel.rs:221-640)."""
    families = {
        "fill_zero": "fill_zero_48", "gemm_f16": "gemm_f16_init", "gemm_f32": "gemm_f32_init",
        "gemm_f8": "gemm_f8", "gelu": "gelu", "reduce_sum": "reduce_sum", "add": "add_f16",
        "flash_attention": "attention_smoke", "attention_softmax": "attention_softmax",
        "attention_merge": "attention_merge", "cast": "cast_f16_f32",
        "unpack": "unpack_amp_output", "rearrange": "rearrange_block_major",
        "rearrange_generic": "generic_rearrange",
    }
    for case in families.values():
        assert case in ACCEPTED or case in REFUSED, case

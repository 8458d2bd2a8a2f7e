"""Register, scratch, occupancy and LDS budgets of the built gfx950 kernels.

The package Makefile keeps the compiler's resource-usage remarks of every
kernel source in ipu-stack_amd/_build/<file>.resources.  These tests read
them (no GPU needed) and hold the kernels to the budgets their designs rely
on: no scratch memory (an array indexed at run time, or a spill, puts it in
per-lane scratch and costs an order of magnitude), the two-workgroups-per-CU
occupancy the attention kernels overlap softmax and MFMAs with, and the
AGPR accumulators and LDS stages of the 256 x 256 GEMM."""
from __future__ import annotations

import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "ipu-stack_amd", "_build")
SOURCES = ("k_memory", "k_gemm_f16", "k_gemm_f32", "k_attention", "k_calibrate")
LINE = re.compile(r"remark:\s+(?P<key>[^:]+?):\s+(?P<value>\S+)\s+\[-Rpass-analysis")


def parse(text: str) -> dict[str, dict[str, str]]:
    """Kernel (mangled name) -> field -> value, from resource-usage remarks."""
    kernels: dict[str, dict[str, str]] = {}
    current = None
    for line in text.splitlines():
        m = LINE.search(line)
        if not m:
            continue
        key, value = m.group("key").strip(), m.group("value")
        if key == "Function Name":
            current = kernels.setdefault(value, {})
        elif current is not None:
            current[key] = value
    return kernels


def test_parse_reads_one_block_per_kernel():
    text = "\n".join([
        "k.hip:3:1: remark: Function Name: _Z3fooPf [-Rpass-analysis=kernel-resource-usage]",
        "k.hip:3:1: remark:     VGPRs: 12 [-Rpass-analysis=kernel-resource-usage]",
        "k.hip:3:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "k.hip:9:1: remark: Function Name: _Z3barPf [-Rpass-analysis=kernel-resource-usage]",
        "k.hip:9:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]",
        "k.hip:9:1: warning: not a remark line",
    ])
    got = parse(text)
    assert got == {"_Z3fooPf": {"VGPRs": "12", "ScratchSize [bytes/lane]": "0"},
                   "_Z3barPf": {"Occupancy [waves/SIMD]": "2"}}


@pytest.fixture(scope="module")
def kernels() -> dict[str, dict[str, str]]:
    files = {os.path.basename(p)[: -len(".resources")]: p
             for p in glob.glob(os.path.join(BUILD, "*.resources"))}
    if not all(s in files for s in SOURCES):
        pytest.skip("library not built by the package Makefile (no resource remarks)")
    out: dict[str, dict[str, str]] = {}
    for s in SOURCES:
        got = parse(open(files[s]).read())
        assert got, f"{s}.resources holds no kernel"
        out.update(got)
    return out


def matching(kernels, fragment: str) -> dict[str, dict[str, str]]:
    got = {k: v for k, v in kernels.items() if fragment in k}
    assert got, f"no kernel named like {fragment}"
    return got


def test_no_kernel_uses_scratch_memory(kernels):
    # Some instantiations of the 256 x 256 GEMM spill two or three values
    # across their K loop (stored before it, reloaded in the epilogue; no
    # scratch access inside the loop); nothing else may touch scratch.
    for name, f in kernels.items():
        limit = 16 if "gemm_f16_256_kernel" in name else 0
        assert int(f["ScratchSize [bytes/lane]"]) <= limit, (name, f)
        assert f.get("Dynamic Stack", "False") == "False", name


def test_attention_kernels_keep_two_waves_per_simd(kernels):
    # One wave's softmax runs beside the other's MFMAs only with two
    # workgroups (one wave of each) per SIMD.
    for name, f in matching(kernels, "attention_fwd_kernel").items():
        assert int(f["Occupancy [waves/SIMD]"]) >= 2, (name, f)
    for name, f in matching(kernels, "attention_wide_kernel").items():
        value_tile = int(re.search(r"attention_wide_kernelILj(\d+)ELj(\d+)E", name).group(2))
        assert int(f["Occupancy [waves/SIMD]"]) >= (1 if value_tile > 256 else 2), (name, f)


def test_gemm_f16_256_accumulators_and_stages(kernels):
    for name, f in matching(kernels, "gemm_f16_256_kernel").items():
        assert int(f["AGPRs"]) == 256, (name, f)        # 8 x 8 tiles of 4 fp32 per lane
        assert int(f["LDS Size [bytes/block]"]) == 131072, (name, f)  # two 64 KiB stages
        # At most a few values spilled around the K loop (never inside it).
        assert int(f["VGPRs Spill"]) <= 4, (name, f)


def test_memory_kernels_need_no_agprs_or_scratch(kernels):
    for name, f in kernels.items():
        if "gemm" in name or "attention" in name or "calibrate" in name:
            continue
        assert int(f["AGPRs"]) == 0, (name, f)
        assert int(f["VGPRs Spill"]) == 0 and int(f["SGPRs Spill"]) == 0, (name, f)

"""ProfileReport ingestion of rocprofv3 output and its queries (CPU only).

The query/calibration cases restate the scenarios and expected values of the
reference's own tests (crates/ipu-profile/src/lib.rs:792-1094); the
ingestion cases read rocprofv3 CSV files committed under tests/golden/ (a
kernel trace of the attention bench legs and FETCH_SIZE counters of the
traffic probe, both recorded on an MI355X) and check the report against the
CSV rows directly.
"""
from __future__ import annotations

import csv
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def prof(ipus):
    import ipu_stack_amd.profiling as profiling
    return profiling


def sample(prof, phase, kind, kernel, start, end):
    """Helper of the reference tests (lib.rs:766-790)."""
    return prof.CycleSample(
        prof.ProfileStep(local_index=phase, phase=phase, epoch=0, operation=f"operation {phase}",
                         kind=kind, kernel=kernel,
                         metadata=[prof.ProfileMetadata("block", str(phase))]),
        start % (1 << 32), end % (1 << 32))


def test_groups_parallel_samples_by_kernel(prof):
    C = prof.ProfileStepKind.COMPUTE
    report = prof.ProfileReport(1_000_000_000, [
        prof.TileProfile(2, [sample(prof, 0, C, "add", 100, 120)]),
        prof.TileProfile(3, [sample(prof, 1, C, "add", 100, 130)])])
    result = prof.query(report, prof.Query())
    assert len(result.groups) == 1
    assert result.groups[0].phase_cycles == 30
    assert result.groups[0].work_cycles == 50
    assert result.groups[0].average_active_tiles == 50.0 / 30.0
    assert result.profile_span_cycles == 30


def test_randomized_queries_crop_one_common_initial_entry_span(prof):
    rng = np.random.default_rng(0x7072_6f67_7261_6d)
    S, C = prof.ProfileStepKind.SYNCHRONIZATION, prof.ProfileStepKind.COMPUTE
    for case in range(64):
        tile_count = int(rng.integers(2, 33))
        starts = [int(x) for x in rng.integers(1_000, 10_001, tile_count)]
        latest = max(starts)
        boundary = latest + int(rng.integers(1, 2_001))
        work = int(rng.integers(1, 2_001))
        report = prof.ProfileReport(1_000_000_000, [
            prof.TileProfile(t, [sample(prof, 0, S, "", start, boundary),
                                 sample(prof, 1, C, "work", boundary, boundary + work)])
            for t, start in enumerate(starts)])
        aligned = prof.query(report, prof.Query(group_by=prof.GroupBy.KIND))
        shared = prof.query(report, prof.Query(shared_clock=True))
        retained = boundary - latest
        assert aligned.profile_span_cycles == retained + work, case
        assert shared.profile_span_cycles >= aligned.profile_span_cycles, case
        sync = next(g for g in aligned.groups if g.name == "synchronization")
        assert sync.first_offset == 0 and sync.maximum_cycles == retained, case
        compute = next(g for g in aligned.groups if g.name == "compute")
        assert compute.first_offset == retained, case


def test_phase_cycles_include_sequential_repeated_operations(prof):
    C = prof.ProfileStepKind.COMPUTE
    report = prof.ProfileReport(1_000_000_000, [
        prof.TileProfile(2, [sample(prof, 0, C, "gemm", 100, 110),
                             sample(prof, 0, C, "gemm", 110, 120)]),
        prof.TileProfile(3, [sample(prof, 0, C, "gemm", 100, 108),
                             sample(prof, 0, C, "gemm", 108, 116)])])
    result = prof.query(report, prof.Query())
    assert result.groups[0].phase_cycles == 20
    assert result.groups[0].work_cycles == 36
    assert result.groups[0].average_active_tiles == 1.8


def test_common_origin_does_not_turn_first_exchange_skew_into_later_skew(prof):
    E, C = prof.ProfileStepKind.EXCHANGE, prof.ProfileStepKind.COMPUTE
    report = prof.ProfileReport(1_000_000_000, [
        prof.TileProfile(2, [sample(prof, 0, E, "", 100, 150), sample(prof, 1, C, "gemm", 150, 160)]),
        prof.TileProfile(3, [sample(prof, 0, E, "", 120, 150), sample(prof, 1, C, "gemm", 150, 160)])])
    result = prof.query(report, prof.Query(kind=C, sample_limit=2, shared_clock=True))
    assert len(result.samples) == 2
    assert all(s.offset == 50 for s in result.samples)
    assert result.groups[0].phase_cycles == 10


def test_filters_by_normalized_time_and_metadata_across_counter_wrap(prof):
    E, C = prof.ProfileStepKind.EXCHANGE, prof.ProfileStepKind.COMPUTE
    report = prof.ProfileReport(1_500_000_000, [prof.TileProfile(9, [
        sample(prof, 0, E, "", (1 << 32) - 1 - 4, 5), sample(prof, 1, C, "add", 5, 15)])])
    q = prof.Query(at_offset=12, metadata=[prof.MetadataFilter("block", "1")], sample_limit=1)
    result = prof.query(report, q)
    assert result.matched_sample_count == 1
    assert result.samples[0].phase == 1
    assert result.samples[0].offset == 10


def test_groups_by_semantic_metadata_value(prof):
    C = prof.ProfileStepKind.COMPUTE
    report = prof.ProfileReport(1_000_000_000, [prof.TileProfile(1, [
        sample(prof, 0, C, "add", 0, 10), sample(prof, 1, C, "add", 10, 30)])])
    result = prof.query(report, prof.Query(group_by=prof.GroupBy.METADATA, metadata_key="block"))
    assert [g.name for g in result.groups] == ["1", "0"]


def test_calibration_normalizes_merged_invocations_and_excludes_graph_metadata(prof):
    C = prof.ProfileStepKind.COMPUTE
    first = sample(prof, 0, C, "gemm-f16", 10, 50)
    first.step.metadata += [prof.ProfileMetadata("kernelSpec", "Gemm"),
                            prof.ProfileMetadata("invocations", "2"),
                            prof.ProfileMetadata("reason", "OperatorKernel")]
    second = prof.CycleSample(first.step, 100, 160)
    db = prof.calibrate_profiles(
        [prof.ProfileReport(1_500_000_000, [prof.TileProfile(0, [first, second])])],
        "ipu21", "test-build")
    assert len(db.measurements) == 1
    m = db.measurements[0]
    assert (m.samples, m.minimum_cycles, m.maximum_cycles) == (2, 20, 30)
    assert "reason" not in m.dimensions and "invocations" not in m.dimensions
    with pytest.raises(ValueError):
        prof.calibrate_profiles([], "t", "b")


def test_percentile_and_union_definitions(prof):
    assert prof.percentile([], 50) == 0
    assert prof.percentile([1, 2, 3, 4], 50) == 2      # sorted[(n - 1) * p / 100]
    assert prof.percentile([1, 2, 3, 4], 95) == 3
    assert prof.union_length([(0, 10), (5, 20), (30, 31)]) == 21
    assert prof.union_length([]) == 0


# ---------------------------------------------------------------------------
# rocprofv3 ingestion
# ---------------------------------------------------------------------------
def _rows(name):
    with open(os.path.join(GOLDEN, name), newline="") as f:
        return list(csv.DictReader(f))


def test_kernel_trace_ingestion_matches_csv(prof):
    rows = _rows("rocprof_attention_kernel_trace.csv")
    report = prof.from_rocprof(os.path.join(GOLDEN, "rocprof_attention_kernel_trace.csv"))
    assert len(report.tiles) == 1 and report.clock_hz == 1_000_000_000
    samples = report.tiles[0].samples
    assert len(samples) == len(rows) == 24
    origin = min(int(r["Start_Timestamp"]) for r in rows)
    by_order = sorted(rows, key=lambda r: (int(r["Start_Timestamp"]), int(r["Dispatch_Id"])))
    for phase, (s, r) in enumerate(zip(samples, by_order)):
        assert s.step.phase == phase and s.step.local_index == phase
        assert s.step.kind is prof.ProfileStepKind.COMPUTE
        assert s.start_cycle == int(r["Start_Timestamp"]) - origin
        assert prof.duration(s) == int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        assert s.step.kernel == prof.kernel_symbol(r["Kernel_Name"])
        md = {m.name: m.value for m in s.step.metadata}
        assert md["ldsBytes"] == r["LDS_Block_Size"] and md["invocations"] == "1"
    # Group totals equal the CSV's per-kernel sums and maxima.
    result = prof.query(report, prof.Query(sort_by=prof.SortBy.NAME))
    names = sorted({prof.kernel_symbol(r["Kernel_Name"]) for r in rows})
    assert [g.name for g in result.groups] == names == [
        "attention_fwd_kernel<128, false, false>", "attention_fwd_kernel<128, true, false>"]
    for g in result.groups:
        d = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows
             if prof.kernel_symbol(r["Kernel_Name"]) == g.name]
        assert g.sample_count == len(d) == 12
        assert g.work_cycles == sum(d)
        assert g.maximum_cycles == max(d)
        assert g.p50_cycles == sorted(d)[(len(d) - 1) // 2]
        # dispatches on one queue do not overlap: the union is the work
        assert g.phase_cycles == g.work_cycles
    # A slower clock scales every interval.
    half = prof.from_rocprof(os.path.join(GOLDEN, "rocprof_attention_kernel_trace.csv"),
                             clock_hz=500_000_000)
    assert abs(prof.duration(half.tiles[0].samples[3]) * 2
               - prof.duration(samples[3])) <= 2


def test_counter_ingestion_and_calibration(prof):
    rows = _rows("rocprof_traffic_counter_collection.csv")
    report = prof.from_rocprof(counter_csv=os.path.join(GOLDEN, "rocprof_traffic_counter_collection.csv"))
    samples = report.tiles[0].samples
    assert len(samples) == len({r["Dispatch_Id"] for r in rows})
    fetch = {int(r["Dispatch_Id"]): float(r["Counter_Value"]) for r in rows}
    for s in samples:
        md = {m.name: m.value for m in s.step.metadata}
        assert float(md["counter.FETCH_SIZE"]) in fetch.values()
    gemm = prof.query(report, prof.Query(kernel="gemm_f16_256_kernel<false, false>", sample_limit=8))
    assert gemm.matched_sample_count == 3 and len(gemm.samples) == 3
    # Counters are measurements, not calibration dimensions: the three GEMM
    # dispatches form one measurement.
    db = prof.calibrate_profiles([report], "mi355x", "fixture")
    gm = [m for m in db.measurements if m.kernel == "gemm_f16_256_kernel<false, false>"]
    assert len(gm) == 1 and gm[0].samples == 3
    assert not any(k.startswith("counter.") for k in gm[0].dimensions)
    assert gm[0].dimensions["ldsBytes"] == "131072"


def test_operation_names_and_filters(prof):
    path = os.path.join(GOLDEN, "rocprof_attention_kernel_trace.csv")
    report = prof.from_rocprof(path, operations=["causal", "noncausal"],
                               kernel_filter=lambda k: k.startswith("attention_fwd_kernel"))
    ops = [s.step.operation for s in report.tiles[0].samples]
    assert ops[:4] == ["causal", "noncausal", "causal", "noncausal"]
    only = prof.query(report, prof.Query(operation_contains="non", group_by=prof.GroupBy.OPERATION))
    assert [g.name for g in only.groups] == ["noncausal"] and only.groups[0].sample_count == 12
    none = prof.from_rocprof(path, kernel_filter=lambda k: False)
    assert none.tiles == [] and prof.query(none).groups == []
    with pytest.raises(ValueError):
        prof.from_rocprof()


def test_json_round_trip(prof):
    report = prof.from_rocprof(os.path.join(GOLDEN, "rocprof_attention_kernel_trace.csv"))
    again = prof.ProfileReport.from_json(report.to_json())
    assert again == report
    assert prof.query(again) == prof.query(report)
    with pytest.raises(ValueError):
        prof.ProfileReport.from_json('{"schemaVersion": 99, "clockHz": 1, "tiles": []}')


def test_kernel_symbol(prof):
    assert prof.kernel_symbol(
        "void ipus::(anonymous namespace)::gemm_f16_256_kernel<false, false>(unsigned short*)"
    ) == "gemm_f16_256_kernel<false, false>"
    assert prof.kernel_symbol("ipus::(anonymous namespace)::copy_bytes_kernel(unsigned char*)") \
        == "copy_bytes_kernel"
    assert prof.kernel_symbol("__amd_rocclr_fillBufferAligned") == "__amd_rocclr_fillBufferAligned"
    assert prof.kernel_symbol("void ns::k<a::b<1>, 2>(int)") == "k<a::b<1>, 2>"

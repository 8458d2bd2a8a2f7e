"""Profiles of GPU runs in the reference's ProfileReport shape, and its queries.

The reference records, per IPU tile, the cycle interval of every program
step (``ProfileReport``/``TileProfile``/``CycleSample``/``ProfileStep``,
crates/ipu-package/src/lib.rs:26-85, 174-258; schemas/profile.capnp) and
answers grouped queries over them (``query``, ``calibrate_profiles``,
crates/ipu-profile/src/lib.rs:1-760).  Here the samples come from rocprofv3
instead of the IPU's cycle counters:

* one "tile" per hardware queue that dispatched kernels (a HIP stream; the
  library runs everything on its context stream, so a run is one tile per
  context);
* one Compute sample per kernel dispatch, its interval the dispatch's begin
  and end timestamps converted to cycles of ``clock_hz`` (default 1 GHz, so a
  cycle is a nanosecond) and kept, like the IPU counter, as a wrapping 32-bit
  value relative to the first dispatch;
* ``kernel`` is the kernel's symbol without its argument list, ``operation``
  the caller's name for the dispatch (by default the kernel), ``phase`` the
  dispatch's order, and ``metadata`` the launch shape (grid, workgroup, LDS,
  VGPRs) plus every counter collected for the dispatch (``counter.FETCH_SIZE``,
  ...; counters are not calibration dimensions).

``query`` and ``calibrate_profiles`` follow the reference's definitions
(cropping of the common initial entry span, interval unions for phase
cycles, percentiles ``sorted[(n - 1) * p / 100]``, sort orders and
tie-breaks), so the same samples give the same report.  IPU exchange-role
accounting has no GPU counterpart and is not carried over.
"""
from __future__ import annotations

import csv
import enum
import json
import math
import os
from dataclasses import asdict, dataclass, field
from typing import Iterable, Optional, Sequence

U32 = 1 << 32
COUNTER_PREFIX = "counter."  # metadata names of rocprofv3 counter values
SCHEMA_VERSION = 5  # crates/ipu-package/src/lib.rs (ProfileReport::write)


class ProfileStepKind(enum.Enum):
    """crates/ipu-package/src/lib.rs:26-31."""
    EXCHANGE = "exchange"
    COMPUTE = "compute"
    SYNCHRONIZATION = "synchronization"
    IDLE = "idle"


@dataclass
class ProfileMetadata:
    name: str
    value: str


@dataclass
class ProfileStep:
    """crates/ipu-package/src/lib.rs:75-85 (exchange fields omitted)."""
    local_index: int
    phase: int
    epoch: int
    operation: str
    kind: ProfileStepKind
    kernel: str
    metadata: list = field(default_factory=list)


@dataclass
class CycleSample:
    step: ProfileStep
    start_cycle: int  # 32-bit wrapping counter
    end_cycle: int


@dataclass
class TileProfile:
    physical_tile: int
    samples: list = field(default_factory=list)


@dataclass
class ProfileReport:
    clock_hz: int
    tiles: list = field(default_factory=list)

    # Serialization: the reference writes Cap'n Proto (schemas/profile.capnp);
    # this image has no Cap'n Proto, so the same fields go to JSON.
    def to_json(self) -> str:
        def step(s: ProfileStep):
            d = asdict(s)
            d["kind"] = s.kind.value
            return d
        return json.dumps({
            "schemaVersion": SCHEMA_VERSION,
            "clockHz": self.clock_hz,
            "tiles": [{"physicalTile": t.physical_tile,
                       "samples": [{"step": step(c.step), "startCycle": c.start_cycle,
                                    "endCycle": c.end_cycle} for c in t.samples]}
                      for t in self.tiles],
        })

    @staticmethod
    def from_json(text: str) -> "ProfileReport":
        root = json.loads(text)
        if not 1 <= root.get("schemaVersion", 0) <= SCHEMA_VERSION:
            raise ValueError(f"unsupported profile schema version {root.get('schemaVersion')}")
        tiles = []
        for t in root["tiles"]:
            samples = []
            for c in t["samples"]:
                s = dict(c["step"])
                s["kind"] = ProfileStepKind(s["kind"])
                s["metadata"] = [ProfileMetadata(**m) for m in s.get("metadata", [])]
                samples.append(CycleSample(ProfileStep(**s), c["startCycle"], c["endCycle"]))
            tiles.append(TileProfile(t["physicalTile"], samples))
        return ProfileReport(root["clockHz"], tiles)


# ---------------------------------------------------------------------------
# Ingestion of rocprofv3 CSV output
# ---------------------------------------------------------------------------
def kernel_symbol(name: str) -> str:
    """Kernel name without its argument list, return type or namespace
    prefix: ``void ipus::(anonymous namespace)::gemm<false>(...)`` ->
    ``gemm<false>``."""
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    name = name.replace("(anonymous namespace)::", "")
    depth = 0
    begin = 0
    end = len(name)
    i = 0
    while i < len(name):
        ch = name[i]
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif depth == 0 and ch == "(":
            end = i
            break
        elif depth == 0 and name.startswith("::", i):
            begin = i + 2
            i += 1
        i += 1
    return name[begin:end]


_LAUNCH_FIELDS = (("Grid_Size", "grid"), ("Grid_Size_X", "grid"), ("Workgroup_Size", "workgroup"),
                  ("Workgroup_Size_X", "workgroup"), ("LDS_Block_Size", "ldsBytes"),
                  ("VGPR_Count", "vgprs"), ("Accum_VGPR_Count", "agprs"),
                  ("SGPR_Count", "sgprs"), ("Scratch_Size", "scratchBytes"))


def _find(directory: str, suffix: str) -> Optional[str]:
    for root, _, files in os.walk(directory):
        for f in sorted(files):
            if f.endswith(suffix):
                return os.path.join(root, f)
    return None


def from_rocprof(kernel_trace_csv: Optional[str] = None, counter_csv: Optional[str] = None,
                 clock_hz: int = 1_000_000_000, operations: Optional[Sequence[str]] = None,
                 kernel_filter=None) -> ProfileReport:
    """Builds a ProfileReport from rocprofv3 ``--output-format csv`` files:
    ``*_kernel_trace.csv`` (``--kernel-trace``) and/or
    ``*_counter_collection.csv`` (``--pmc``).  Either may be a directory,
    which is searched for the file.  ``operations`` names dispatches in
    order (cycled), e.g. a CompiledPackage's step symbols repeated per run;
    ``kernel_filter(symbol) -> bool`` keeps a subset of the kernels."""
    if kernel_trace_csv and os.path.isdir(kernel_trace_csv):
        kernel_trace_csv = _find(kernel_trace_csv, "kernel_trace.csv")
    if counter_csv and os.path.isdir(counter_csv):
        counter_csv = _find(counter_csv, "counter_collection.csv")
    if not kernel_trace_csv and not counter_csv:
        raise ValueError("a kernel trace or a counter collection is required")

    dispatches = {}  # dispatch id -> record
    def record(row):
        did = int(row["Dispatch_Id"])
        d = dispatches.get(did)
        if d is None:
            d = dispatches[did] = {
                "id": did, "name": row["Kernel_Name"],
                "queue": (row.get("Agent_Id", ""), row.get("Queue_Id", "")),
                "start": int(row["Start_Timestamp"]), "end": int(row["End_Timestamp"]),
                "launch": {}, "counters": {}}
            for key, label in _LAUNCH_FIELDS:
                if row.get(key) not in (None, ""):
                    d["launch"][label] = row[key]
        return d

    if kernel_trace_csv:
        with open(kernel_trace_csv, newline="") as f:
            for row in csv.DictReader(f):
                if row.get("Kind", "KERNEL_DISPATCH") == "KERNEL_DISPATCH":
                    record(row)
    if counter_csv:
        with open(counter_csv, newline="") as f:
            for row in csv.DictReader(f):
                d = record(row)
                name = row["Counter_Name"]
                d["counters"][name] = d["counters"].get(name, 0.0) + float(row["Counter_Value"])

    ordered = sorted(dispatches.values(), key=lambda d: (d["start"], d["id"]))
    if kernel_filter is not None:
        ordered = [d for d in ordered if kernel_filter(kernel_symbol(d["name"]))]
    if not ordered:
        return ProfileReport(clock_hz, [])
    origin = ordered[0]["start"]
    queues = sorted({d["queue"] for d in ordered})
    tile_of = {q: i for i, q in enumerate(queues)}
    tiles = [TileProfile(i) for i in range(len(queues))]
    scale = clock_hz / 1e9
    for phase, d in enumerate(ordered):
        tile = tiles[tile_of[d["queue"]]]
        symbol = kernel_symbol(d["name"])
        metadata = [ProfileMetadata(k, str(v)) for k, v in d["launch"].items()]
        for k in sorted(d["counters"]):
            v = d["counters"][k]
            text = str(int(v)) if float(v).is_integer() else repr(v)
            metadata.append(ProfileMetadata(COUNTER_PREFIX + k, text))
        metadata.append(ProfileMetadata("invocations", "1"))
        op = operations[phase % len(operations)] if operations else symbol
        step = ProfileStep(local_index=len(tile.samples), phase=phase, epoch=0, operation=op,
                           kind=ProfileStepKind.COMPUTE, kernel=symbol, metadata=metadata)
        start = int(round((d["start"] - origin) * scale)) % U32
        end = int(round((d["end"] - origin) * scale)) % U32
        tile.samples.append(CycleSample(step, start, end))
    return ProfileReport(clock_hz, tiles)


# ---------------------------------------------------------------------------
# Queries (crates/ipu-profile/src/lib.rs)
# ---------------------------------------------------------------------------
class GroupBy(enum.Enum):
    KIND = "kind"
    KERNEL = "kernel"
    OPERATION = "operation"
    PHASE = "phase"
    TILE = "tile"
    METADATA = "metadata"


class SortBy(enum.Enum):
    PHASE_CYCLES = "phase-cycles"
    WORK_CYCLES = "work-cycles"
    MAXIMUM_CYCLES = "maximum-cycles"
    SAMPLES = "samples"
    NAME = "name"


@dataclass
class MetadataFilter:
    name: str
    value: Optional[str] = None


@dataclass
class Query:
    """crates/ipu-profile/src/lib.rs:93-109 (defaults: group by kernel, sort by
    phase cycles, crop the common initial entry span, no samples)."""
    group_by: GroupBy = GroupBy.KERNEL
    sort_by: SortBy = SortBy.PHASE_CYCLES
    kind: Optional[ProfileStepKind] = None
    kernel: Optional[str] = None
    operation_contains: Optional[str] = None
    tiles: frozenset = frozenset()
    phases: frozenset = frozenset()
    metadata: list = field(default_factory=list)
    metadata_key: Optional[str] = None
    at_offset: Optional[int] = None
    shared_clock: bool = False
    limit: Optional[int] = None
    sample_limit: int = 0


@dataclass
class GroupSummary:
    name: str
    dimensions: dict
    sample_count: int
    tile_count: int
    phase_count: int
    phase_cycles: int
    phase_ms: float
    work_cycles: int
    average_active_tiles: float
    mean_cycles: float
    p50_cycles: int
    p95_cycles: int
    maximum_cycles: int
    first_offset: int
    last_offset: int


@dataclass
class SampleRecord:
    physical_tile: int
    offset: int
    duration: int
    phase: int
    epoch: int
    kind: str
    operation: str
    kernel: str
    metadata: list


@dataclass
class QueryReport:
    clock_hz: int
    tile_count: int
    sample_count: int
    matched_sample_count: int
    profile_span_cycles: int
    profile_span_ms: float
    at_offset: Optional[int]
    groups: list
    samples: list


def _wrapsub(a: int, b: int) -> int:
    return (a - b) % U32


def duration(sample: CycleSample) -> int:
    return _wrapsub(sample.end_cycle, sample.start_cycle)


def percentile(sorted_values: Sequence[int], percentage: int) -> int:
    if not sorted_values:
        return 0
    return sorted_values[(len(sorted_values) - 1) * percentage // 100]


def union_length(intervals: Iterable[tuple]) -> int:
    spans = sorted(intervals)
    if not spans:
        return 0
    total = 0
    start, end = spans[0]
    for s, e in spans[1:]:
        if s <= end:
            end = max(end, e)
        else:
            total += end - start
            start, end = s, e
    return total + end - start


def cycles_to_ms(cycles: int, clock_hz: int) -> float:
    return 0.0 if clock_hz == 0 else cycles * 1000.0 / clock_hz


def cycle_origin(report: ProfileReport) -> int:
    """Common origin of the tiles' first samples on the wrapping counter: the
    earliest of them, measured as signed 32-bit deltas from the first."""
    firsts = [t.samples[0].start_cycle for t in report.tiles if t.samples]
    if not firsts:
        return 0
    reference = firsts[0]
    def signed(delta):
        return delta - U32 if delta >= 1 << 31 else delta
    minimum = min(signed(_wrapsub(s, reference)) for s in firsts)
    return (reference + minimum) % U32


def _initial_sample_entry_span(report: ProfileReport, base: int) -> int:
    return max((_wrapsub(t.samples[0].start_cycle, base) for t in report.tiles if t.samples),
               default=0)


def _matches(q: Query, tile: int, sample: CycleSample, offset: int, dur: int) -> bool:
    step = sample.step
    if q.kind is not None and q.kind != step.kind:
        return False
    if q.kernel is not None and step.kernel != q.kernel:
        return False
    if q.operation_contains is not None and q.operation_contains not in step.operation:
        return False
    if q.tiles and tile not in q.tiles:
        return False
    if q.phases and step.phase not in q.phases:
        return False
    if q.at_offset is not None and not (offset <= q.at_offset < offset + dur):
        return False
    return all(any(m.name == f.name and (f.value is None or m.value == f.value)
                   for m in step.metadata) for f in q.metadata)


def _group_key(q: Query, tile: int, sample: CycleSample):
    step = sample.step
    dims = {}
    if q.group_by is GroupBy.KIND:
        name = step.kind.value
    elif q.group_by is GroupBy.KERNEL:
        name = step.kernel or "(no kernel)"
    elif q.group_by is GroupBy.OPERATION:
        name = step.operation
    elif q.group_by is GroupBy.PHASE:
        dims = {"phase": str(step.phase), "epoch": str(step.epoch)}
        name = f"phase {step.phase}/{step.epoch}"
    elif q.group_by is GroupBy.TILE:
        dims = {"physicalTile": str(tile)}
        name = f"tile {tile}"
    else:
        key = q.metadata_key or ""
        value = next((m.value for m in step.metadata if m.name == key), "(missing)")
        dims = {"metadataKey": key, "metadataValue": value}
        name = value
    return name, dims


def _sort_key(sort_by: SortBy, g: GroupSummary):
    primary = {
        SortBy.PHASE_CYCLES: -g.phase_cycles,
        SortBy.WORK_CYCLES: -g.work_cycles,
        SortBy.MAXIMUM_CYCLES: -g.maximum_cycles,
        SortBy.SAMPLES: -g.sample_count,
    }.get(sort_by)
    if sort_by is SortBy.NAME:
        return (g.name, g.first_offset, g.name)
    return (primary, g.first_offset, g.name)


def query(report: ProfileReport, q: Query = Query()) -> QueryReport:
    """Grouped summary of the samples matching ``q``
    (crates/ipu-profile/src/lib.rs:416-560)."""
    sample_count = sum(len(t.samples) for t in report.tiles)
    base = cycle_origin(report)
    crop = 0 if q.shared_clock else _initial_sample_entry_span(report, base)
    span = max((max(0, _wrapsub(s.start_cycle, base) + duration(s) - crop)
                for t in report.tiles for s in t.samples), default=0)
    groups = {}
    candidates = []
    matched = 0
    for t in report.tiles:
        for s in t.samples:
            raw_offset = _wrapsub(s.start_cycle, base)
            raw_end = raw_offset + duration(s)
            offset = max(0, raw_offset - crop)
            end = max(0, raw_end - crop)
            dur = min(end - offset, U32 - 1)
            if dur == 0 or not _matches(q, t.physical_tile, s, offset, dur):
                continue
            matched += 1
            name, dims = _group_key(q, t.physical_tile, s)
            acc = groups.get(name)
            if acc is None:
                acc = groups[name] = {"dims": dims, "durations": [], "tiles": set(),
                                      "phases": set(), "intervals": [], "work": 0,
                                      "first": offset, "last": 0}
            acc["durations"].append(dur)
            acc["tiles"].add(t.physical_tile)
            acc["phases"].add((s.step.phase, s.step.epoch))
            acc["intervals"].append((offset, offset + dur))
            acc["work"] += dur
            acc["first"] = min(acc["first"], offset)
            acc["last"] = max(acc["last"], offset + dur)
            if q.sample_limit > 0:
                candidates.append((t.physical_tile, offset, dur, s))
    summaries = []
    for name, acc in groups.items():
        durations = sorted(acc["durations"])
        phase_cycles = union_length(acc["intervals"])
        summaries.append(GroupSummary(
            name=name, dimensions=acc["dims"], sample_count=len(durations),
            tile_count=len(acc["tiles"]), phase_count=len(acc["phases"]),
            phase_cycles=phase_cycles, phase_ms=cycles_to_ms(phase_cycles, report.clock_hz),
            work_cycles=acc["work"],
            average_active_tiles=acc["work"] / phase_cycles if phase_cycles else 0.0,
            mean_cycles=acc["work"] / len(durations) if durations else 0.0,
            p50_cycles=percentile(durations, 50), p95_cycles=percentile(durations, 95),
            maximum_cycles=durations[-1] if durations else 0,
            first_offset=acc["first"], last_offset=acc["last"]))
    summaries.sort(key=lambda g: _sort_key(q.sort_by, g))
    if q.limit is not None:
        summaries = summaries[:q.limit]
    candidates.sort(key=lambda c: (-c[2], c[0], c[1]))
    samples = [SampleRecord(tile, offset, dur, s.step.phase, s.step.epoch, s.step.kind.value,
                            s.step.operation, s.step.kernel,
                            [ProfileMetadata(m.name, m.value) for m in s.step.metadata])
               for tile, offset, dur, s in candidates[:q.sample_limit]]
    return QueryReport(report.clock_hz, len(report.tiles), sample_count, matched, span,
                       cycles_to_ms(span, report.clock_hz), q.at_offset, summaries, samples)


# ---------------------------------------------------------------------------
# Calibration database (crates/ipu-profile/src/lib.rs:207-273)
# ---------------------------------------------------------------------------
@dataclass
class CalibrationMeasurement:
    kernel: str
    dimensions: dict
    samples: int
    minimum_cycles: int
    median_cycles: int
    p95_cycles: int
    maximum_cycles: int


@dataclass
class CalibrationDatabase:
    schema_version: int
    target: str
    build_id: str
    clock_hz: int
    measurements: list


_GRAPH_METADATA = ("reason", "value", "invocations")


def _is_dimension(name: str) -> bool:
    # Hardware counters are measurements of a dispatch, not part of its key.
    return name not in _GRAPH_METADATA and not name.startswith(COUNTER_PREFIX)


def calibrate_profiles(reports: Sequence[ProfileReport], target: str,
                       build_id: str) -> CalibrationDatabase:
    """Per (kernel, metadata) cycle statistics of the Compute samples; a sample
    that merges ``invocations`` calls counts ceil(duration / invocations)."""
    if not reports:
        raise ValueError("at least one profile is required")
    clock_hz = reports[0].clock_hz
    if any(r.clock_hz != clock_hz for r in reports):
        raise ValueError("profile clock frequencies differ")
    groups = {}
    for r in reports:
        for t in r.tiles:
            for s in t.samples:
                if s.step.kind is not ProfileStepKind.COMPUTE or not s.step.kernel:
                    continue
                inv = 1
                for m in s.step.metadata:
                    if m.name == "invocations":
                        try:
                            inv = max(1, int(m.value))
                        except ValueError:
                            inv = 1
                        break
                dims = tuple(sorted((m.name, m.value) for m in s.step.metadata
                                    if _is_dimension(m.name)))
                groups.setdefault((s.step.kernel, dims), []).append(
                    math.ceil(duration(s) / inv))
    measurements = []
    for (kernel, dims), cycles in sorted(groups.items()):
        cycles.sort()
        measurements.append(CalibrationMeasurement(
            kernel, dict(dims), len(cycles), cycles[0], percentile(cycles, 50),
            percentile(cycles, 95), cycles[-1]))
    return CalibrationDatabase(1, target, build_id, clock_hz, measurements)

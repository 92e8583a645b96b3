"""Per-op GPU timings of a program: the budget table a step is made of, and a Chrome-trace file for Perfetto
(``monolith/trace.py:20-105``: ``OpTiming``, ``op_timings``, ``budget``, ``format_budget``, ``write_chrome_trace``).

``runs`` is ``Engine.profile(k)``: per step, a ``(start_ms, end_ms)`` pair per dispatch from HIP events. Consecutive
ops of one name that carry ``meta["t_range"]`` (predicated per-T variants: one runs, the others return at once)
count as one op: their durations add up and their bytes count once.
"""

from __future__ import annotations

import json
from collections import defaultdict
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

from .program import Program


@dataclass
class OpTiming:
    index: int
    name: str
    kernel: str
    kind: str
    ms_min: float
    ms_median: float
    bytes: int

    @property
    def gbps(self) -> Optional[float]:
        if not self.bytes or self.ms_min <= 0:
            return None
        return self.bytes / (self.ms_min * 1e6)


def _groups(program: Program):
    ops, i = program.ops, 0
    while i < len(ops):
        j = i + 1
        if ops[i].meta.get("t_range") is not None:
            while j < len(ops) and ops[j].name == ops[i].name and ops[j].meta.get("t_range") is not None:
                j += 1
        yield i, j
        i = j


def op_timings(program: Program, runs: Sequence[Sequence[Tuple[float, float]]]) -> List[OpTiming]:
    out = []
    for i, j in _groups(program):
        per_run = []
        for run in runs:
            spans = [e - s for s, e in run[i:j] if s >= 0]
            if spans:
                per_run.append(sum(max(0.0, d) for d in spans))
        if not per_run:
            continue
        per_run.sort()
        op = program.ops[i]
        kind = str(op.meta.get("kind", op.name.split(":")[0]))
        out.append(OpTiming(i, op.name, op.kernel.split("|")[0], kind, per_run[0], per_run[len(per_run) // 2],
                            int(op.meta.get("bytes", 0))))
    return out


def budget(timings: Sequence[OpTiming]) -> List[Tuple[str, int, float, int]]:
    """Per kind: (kind, ops, summed minimum ms, summed bytes), the most time first."""
    acc: Dict[str, list] = defaultdict(lambda: [0, 0.0, 0])
    for t in timings:
        acc[t.kind][0] += 1
        acc[t.kind][1] += t.ms_min
        acc[t.kind][2] += t.bytes
    return sorted(((k, n, ms, b) for k, (n, ms, b) in acc.items()), key=lambda r: -r[2])


def format_budget(timings: Sequence[OpTiming], nominal_gbps: Optional[float] = None) -> str:
    total = sum(t.ms_min for t in timings) or 1e-12
    rows = [f"{'op kind':18s} {'n':>4s} {'ms (min)':>9s} {'share':>6s} {'GB streamed':>12s} {'GB/s':>7s}"]
    for kind, n, ms, nbytes in budget(timings):
        rate = f"{nbytes / (ms * 1e6):7.1f}" if nbytes and ms > 0 else "      -"
        rows.append(f"{kind:18s} {n:4d} {ms:9.3f} {100 * ms / total:5.1f}% {nbytes / 1e9:12.3f} {rate}")
    streamed = sum(t.bytes for t in timings)
    tail = ""
    if nominal_gbps and streamed:
        tail = f"; bandwidth bound of the streamed bytes at {nominal_gbps:.0f} GB/s: {streamed / nominal_gbps / 1e6:.2f} ms"
    rows.append(f"{'total':18s} {len(timings):4d} {sum(t.ms_min for t in timings):9.3f} "
                f"(sum of per-op minima; launch gaps excluded){tail}")
    return "\n".join(rows)


def write_chrome_trace(path: str, program: Program, runs: Sequence[Sequence[Tuple[float, float]]]) -> None:
    """Complete events ("X") in µs, one row per step laid end to end."""
    events, base = [], 0.0
    for step, run in enumerate(runs):
        for i, (s, e) in enumerate(run):
            if s < 0:
                continue
            op = program.ops[i]
            events.append({"name": op.name, "cat": str(op.meta.get("kind", "")), "ph": "X", "ts": (base + s) * 1e3,
                           "dur": max(0.0, e - s) * 1e3, "pid": 1, "tid": 1,
                           "args": {"kernel": op.kernel, "step": step, **op.meta}})
        base += max((e for _, e in run), default=0.0) + 0.05
    with open(path, "w") as f:
        json.dump({"traceEvents": events, "displayTimeUnit": "ms"}, f)

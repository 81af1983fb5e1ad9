"""Named-section timing with HIP events.

Mirrors the interface of the reference's AttentionTimingCollector
(sinkattention/timing.py:12-100) that SinkRuntimeState.time_section hands out: the
section(name) context manager, summarize(), reset() and is_enabled.  Enabled by
SINK_ATTN_ENABLE_TIMING (or WAN_ATTN_ENABLE_TIMING) set to 1/true/yes/on.

Also the two summary helpers the Wan inference CLI imports
(wanx/runtime/inference.py:23): extract_attention_time_ms and
aggregate_timing_summaries (sinkattention/timing.py:103-169).
"""
from __future__ import annotations

import os
import time
from collections import defaultdict
from contextlib import contextmanager
from typing import Dict, Iterable, List, Optional, Tuple

import torch


def _env_enabled() -> bool:
    raw = os.environ.get("SINK_ATTN_ENABLE_TIMING", os.environ.get("WAN_ATTN_ENABLE_TIMING", "0"))
    return raw.strip().lower() in {"1", "true", "yes", "on"}


class AttentionTimingCollector:
    def __init__(self, *, label: str, enabled: Optional[bool] = None):
        self.label = label
        self.enabled = _env_enabled() if enabled is None else bool(enabled)
        self._events: List[Tuple[str, object, object]] = []
        self._host: List[Tuple[str, float]] = []

    @property
    def is_enabled(self) -> bool:
        return self.enabled

    def reset(self) -> None:
        self._events.clear()
        self._host.clear()

    @contextmanager
    def section(self, name: str):
        if not self.enabled:
            yield
            return
        if torch.cuda.is_available():
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            try:
                yield
            finally:
                end.record()
                self._events.append((name, start, end))
            return
        t0 = time.perf_counter()
        try:
            yield
        finally:
            self._host.append((name, (time.perf_counter() - t0) * 1e3))

    def summarize(self) -> dict:
        if not self.enabled:
            return {"enabled": False, "label": self.label, "num_records": 0, "by_section": {},
                    "total_ms": 0.0}
        if self._events:
            torch.cuda.synchronize()
        tot: Dict[str, float] = defaultdict(float)
        cnt: Dict[str, int] = defaultdict(int)
        for name, s, e in self._events:
            tot[name] += float(s.elapsed_time(e))
            cnt[name] += 1
        for name, ms in self._host:
            tot[name] += ms
            cnt[name] += 1
        names = sorted(tot, key=lambda n: (-tot[n], n))
        return {
            "enabled": True,
            "label": self.label,
            "num_records": int(sum(cnt.values())),
            "by_section": {n: {"total_ms": tot[n], "mean_ms": tot[n] / max(cnt[n], 1),
                               "count": cnt[n]} for n in names},
            "total_ms": float(sum(tot.values())),
        }


def extract_attention_time_ms(
    summary: Optional[dict],
    *,
    preferred_sections: Iterable[str] = ("inner_total",),
) -> Optional[float]:
    """Attention time of one summarize() result (sinkattention/timing.py:103-123).

    None for a missing or disabled summary; else the total of the first preferred section
    that has one, else the summary's own total (None when that is absent).
    """
    if not summary or not summary.get("enabled", False):
        return None
    sections = summary.get("by_section") or {}
    for name in preferred_sections:
        entry = sections.get(name)
        if entry is not None and entry.get("total_ms") is not None:
            return float(entry["total_ms"])
    total = summary.get("total_ms")
    return None if total is None else float(total)


def aggregate_timing_summaries(summaries: Iterable[Optional[dict]]) -> Optional[dict]:
    """Mean / max / sum over several summarize() results (sinkattention/timing.py:126-169).

    Disabled or empty summaries are skipped; None when none is left.  Per-section statistics
    are keyed by str(section name) in sorted order; the totals skip entries without total_ms.
    """
    kept = [s for s in summaries if s and s.get("enabled", False)]
    if not kept:
        return None
    per_section: Dict[str, List[float]] = defaultdict(list)
    totals: List[float] = []
    for s in kept:
        if s.get("total_ms") is not None:
            totals.append(float(s["total_ms"]))
        for name, entry in (s.get("by_section") or {}).items():
            if entry.get("total_ms") is not None:
                per_section[str(name)].append(float(entry["total_ms"]))
    names = sorted(n for n in per_section if per_section[n])
    return {
        "count": len(kept),
        "labels": sorted({str(s.get("label", "")) for s in kept if s.get("label")}),
        "mean_total_ms": sum(totals) / len(totals) if totals else None,
        "max_total_ms": max(totals) if totals else None,
        "mean_by_section_ms": {n: sum(per_section[n]) / len(per_section[n]) for n in names},
        "max_by_section_ms": {n: max(per_section[n]) for n in names},
        "total_by_section_ms": {n: float(sum(per_section[n])) for n in names},
    }

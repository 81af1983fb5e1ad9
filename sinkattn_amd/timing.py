"""Named-section timing with HIP events.

Mirrors the interface of the reference's AttentionTimingCollector
(sinkattention/timing.py:12-100) that SinkRuntimeState.time_section hands out: the
section(name) context manager, summarize(), reset() and is_enabled.  Enabled by
SINK_ATTN_ENABLE_TIMING (or WAN_ATTN_ENABLE_TIMING) set to 1/true/yes/on.
"""
from __future__ import annotations

import os
import time
from collections import defaultdict
from contextlib import contextmanager
from typing import Dict, List, Optional, Tuple

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

"""GPU-side timing of library launches with stream events.

Each span records an event before and after its launches on the stream the
launches go to (the caller's current stream), so the measured interval is
the launches' device time when the stream is busy (back-to-back enqueue).
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Dict, List, Tuple

import torch


class KernelTimer:
    def __init__(self, enabled: bool = True):
        self.enabled = enabled
        self.spans: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event, int]]] = {}

    @contextmanager
    def span(self, name: str, nbytes: int = 0):
        if not self.enabled:
            yield
            return
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        try:
            yield
        finally:
            e1.record(stream)
            self.spans.setdefault(name, []).append((e0, e1, int(nbytes)))

    def reset(self) -> None:
        self.spans = {}

    def summary(self) -> Dict[str, Dict[str, float]]:
        """Per span name: launches, total / mean device ms, bytes per launch, GB/s."""
        torch.cuda.synchronize()
        out = {}
        for name, recs in self.spans.items():
            ms = [a.elapsed_time(b) for a, b, _ in recs]
            nbytes = sum(n for _, _, n in recs)
            tot = sum(ms)
            out[name] = {
                "launches": len(recs),
                "total_ms": tot,
                "mean_ms": tot / len(recs),
                "bytes_per_launch": nbytes / len(recs),
                "GBps": (nbytes / (tot * 1e-3) / 1e9) if tot > 0 else 0.0,
            }
        return out

"""GPU-side timing of library launches with stream events.

A span times the launches made inside it with an event pair on the stream
they go to (the caller's current stream). When the span is given the tables
it launches through, the library records the pair itself as its first kernel
starts and its last kernel ends (dz_table_time_next, hipExtLaunchKernel), so
the interval is the kernels' device time even when the stream was idle and
the host's launch work would otherwise fall inside it. Without tables, or
while the stream is being captured into a graph, the span records the pair
before and after its launches.
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Dict, List, Sequence, Tuple

import torch


class KernelTimer:
    def __init__(self, enabled: bool = True, kernel_events: bool = True):
        self.enabled = enabled
        self.kernel_events = kernel_events
        self.spans: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event, int]]] = {}

    @contextmanager
    def span(self, name: str, nbytes: int = 0, tables: Sequence = ()):
        """tables: the library tables the span's launches go through, in launch
        order (each makes one launching call inside the span)."""
        if not self.enabled:
            yield
            return
        stream = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        by_kernel = bool(tables) and self.kernel_events and not torch.cuda.is_current_stream_capturing()
        if by_kernel:
            # both events exist now (recorded once); the launches record them again
            e1.record(stream)
            first, last = tables[0], tables[-1]
            if first is last:
                first.time_next(e0, e1)
            else:
                first.time_next(e0, None)
                last.time_next(None, e1)
        try:
            yield
        finally:
            if not by_kernel:
                e1.record(stream)
            self.spans.setdefault(name, []).append((e0, e1, int(nbytes)))

    def reset(self) -> None:
        self.spans = {}

    def summary(self) -> Dict[str, Dict[str, float]]:
        """Per span name: launches, total / mean / median / min / max device ms,
        bytes per launch, GB/s (from the total)."""
        torch.cuda.synchronize()
        out = {}
        for name, recs in self.spans.items():
            ms = [a.elapsed_time(b) for a, b, _ in recs]
            nbytes = sum(n for _, _, n in recs)
            tot = sum(ms)
            srt = sorted(ms)
            mid = len(srt) // 2
            out[name] = {
                "launches": len(recs),
                "total_ms": tot,
                "mean_ms": tot / len(recs),
                "median_ms": srt[mid] if len(srt) % 2 else 0.5 * (srt[mid - 1] + srt[mid]),
                "min_ms": srt[0],
                "max_ms": srt[-1],
                "bytes_per_launch": nbytes / len(recs),
                "GBps": (nbytes / (tot * 1e-3) / 1e9) if tot > 0 else 0.0,
            }
        return out

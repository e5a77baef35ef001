"""Low-perturbation GPU timing of attention phases (dfsattn/utils/timing.py:24-218).

Events are recorded on the current stream without synchronising; durations
are resolved when ``rows`` / ``dump_csv`` is called after the run.
"""
from __future__ import annotations

import csv
import os
import time
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Union

import torch


@dataclass
class _EventPair:
    phase: str
    step_idx: int
    layer_idx: int
    start: Union[torch.cuda.Event, float]
    end: Union[torch.cuda.Event, float]


class AttentionTimingRecorder:
    def __init__(self, enabled: bool = False) -> None:
        self.enabled = enabled
        self._records: List[_EventPair] = []
        self._metric_records: Dict[str, List[float]] = {}

    def reset(self, enabled: bool) -> None:
        self.enabled = enabled
        self._records.clear()
        self._metric_records.clear()

    def record_metrics(self, metrics: Dict[str, float]) -> None:
        if not self.enabled:
            return
        for name, value in metrics.items():
            self._metric_records.setdefault(name, []).append(float(value))

    def start(self, device: torch.device):
        if not self.enabled:
            return None
        if device.type == "cuda":
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            return ev
        return time.perf_counter()

    def stop(self, start, phase: str, step_idx: int, layer_idx: int, device: torch.device) -> None:
        if not self.enabled or start is None:
            return
        if device.type == "cuda":
            end = torch.cuda.Event(enable_timing=True)
            end.record()
        else:
            end = time.perf_counter()
        self._records.append(_EventPair(phase, int(step_idx), int(layer_idx), start, end))

    def rows(self) -> List[Dict[str, Any]]:
        if any(isinstance(r.end, torch.cuda.Event) for r in self._records):
            torch.cuda.synchronize()
        out = []
        for r in self._records:
            if isinstance(r.start, torch.cuda.Event):
                ms = r.start.elapsed_time(r.end)
            else:
                ms = (r.end - r.start) * 1e3
            out.append({"phase": r.phase, "step_idx": r.step_idx, "layer_idx": r.layer_idx, "elapsed_ms": ms})
        return out

    def dump_csv(self, output_path: str, extra_totals: Optional[Dict[str, float]] = None
                 ) -> Dict[str, Dict[str, float]]:
        """One aggregate row per phase: ``top_k_selection`` (sum of
        ``topk_mask`` events) and ``attention_execution``, plus extra totals."""
        totals: Dict[str, float] = {"top_k_selection": 0.0, "attention_execution": 0.0}
        calls: Dict[str, float] = {p: 0.0 for p in totals}
        aliases = {"topk_mask": "top_k_selection", "attention_execution": "attention_execution"}
        for row in self.rows():
            phase = aliases.get(row["phase"])
            if phase is None:
                continue
            totals[phase] += float(row["elapsed_ms"])
            calls[phase] += 1.0
        for phase, ms in (extra_totals or {}).items():
            totals[phase] = float(ms)
            calls[phase] = 1.0
        os.makedirs(os.path.dirname(output_path) or ".", exist_ok=True)
        with open(output_path, "w", newline="") as fh:
            wr = csv.DictWriter(fh, fieldnames=["phase", "total_ms", "calls", "mean_ms"])
            wr.writeheader()
            for phase, total in totals.items():
                n = calls.get(phase, 0.0)
                wr.writerow({"phase": phase, "total_ms": total, "calls": int(n),
                             "mean_ms": total / n if n else 0.0})
        return {p: {"calls": calls.get(p, 0.0), "total_ms": t, "mean_ms": t / calls[p] if calls.get(p) else 0.0}
                for p, t in totals.items()}

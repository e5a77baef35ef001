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

    # Phases of the reference's CSV besides the two this build records: its
    # research executors time these sub-phases (timing.py:113-138). They are
    # written with zero calls so the file has the same rows.
    DETAILED_PHASES = (
        "flashinfer_qkv_permute", "flashinfer_fine_score", "flashinfer_fine_topk", "flashinfer_core_score",
        "flashinfer_core_select", "flashinfer_occupancy", "flashinfer_partition", "flashinfer_residual_select",
        "flashinfer_peak_score", "flashinfer_promotion", "flashinfer_residual_compact", "flashinfer_plan",
        "flashinfer_core_csr_expand", "flashinfer_core_run", "flashinfer_residual_micro_run",
        "flashinfer_residual_rode_plan", "flashinfer_residual_rode_fp32", "flashinfer_residual_rode_sddmm",
        "flashinfer_residual_rode_softmax", "flashinfer_residual_rode_spmm", "flashinfer_residual_rode_run",
        "flashinfer_density_accounting", "flashinfer_lse_merge", "flashinfer_output_unpermute",
    )
    METRIC_FIELDS = ("residual_count_mean", "residual_count_p50", "residual_count_p95", "residual_count_max",
                     "residual_count_nonempty_ratio", "fine_top_k", "occupancy_threshold", "occupancy_mean")

    def dump_csv(self, output_path: str, extra_totals: Optional[Dict[str, float]] = None
                 ) -> Dict[str, Dict[str, float]]:
        """One aggregate row per phase (timing.py:97-218): ``top_k_selection``
        (sum of ``topk_mask`` events), ``attention_execution``, the detailed
        phases, any ``extra_totals``, then a ``residual_route_stats`` row when
        metrics were recorded. Columns: phase, total_ms, calls, mean_ms and
        the metric fields."""
        totals: Dict[str, float] = {"top_k_selection": 0.0, "attention_execution": 0.0}
        totals.update({p: 0.0 for p in self.DETAILED_PHASES})
        calls: Dict[str, float] = {p: 0.0 for p in totals}
        aliases = {"topk_mask": "top_k_selection", "attention_execution": "attention_execution"}
        for row in self.rows():
            raw = row["phase"]
            phase = aliases.get(raw)
            if phase is None and (raw in self.DETAILED_PHASES or raw.startswith("flashinfer_residual_bucket_le")):
                phase = raw
                totals.setdefault(phase, 0.0)
                calls.setdefault(phase, 0.0)
            if phase is None:
                continue
            totals[phase] += float(row["elapsed_ms"])
            calls[phase] += 1.0
        for phase, ms in (extra_totals or {}).items():
            totals[phase] = float(ms)
            calls[phase] = 1.0
        os.makedirs(os.path.dirname(output_path) or ".", exist_ok=True)
        with open(output_path, "w", newline="") as fh:
            wr = csv.DictWriter(fh, fieldnames=["phase", "total_ms", "calls", "mean_ms", *self.METRIC_FIELDS])
            wr.writeheader()
            for phase, total in totals.items():
                n = calls.get(phase, 0.0)
                wr.writerow({"phase": phase, "total_ms": total, "calls": int(n),
                             "mean_ms": total / n if n else 0.0})
            metrics = {name: self._metric_records.get(name, []) for name in self.METRIC_FIELDS}
            n_metric = max((len(v) for v in metrics.values()), default=0)
            if n_metric:
                wr.writerow({"phase": "residual_route_stats", "total_ms": "", "calls": n_metric, "mean_ms": "",
                             **{k: sum(v) / len(v) if v else float("nan") for k, v in metrics.items()}})
        return {p: {"calls": calls.get(p, 0.0), "total_ms": t, "mean_ms": t / calls[p] if calls.get(p) else 0.0}
                for p, t in totals.items()}

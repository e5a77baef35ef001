"""Low-perturbation timing of attention phases, written out in the CSV form of
dfsattn/utils/timing.py:97-218 (the same rows and columns).

A measurement is a pair of marks taken around a phase. On a GPU device a mark
is a HIP event recorded on the current stream, so taking it never waits for
the device; on other devices it is a ``perf_counter`` reading. Marks are kept
unresolved in one ledger per phase and turned into milliseconds together, with
a single device synchronisation, the first time a summary is asked for after
new GPU marks were added.
"""
from __future__ import annotations

import csv
import os
import time
from typing import Dict, List, Optional, Tuple

import torch

Mark = object  # a torch.cuda.Event or a perf_counter() float


def _take_mark(device: torch.device) -> Mark:
    if device.type == "cuda":
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev
    return time.perf_counter()


def _span_ms(first: Mark, last: Mark) -> float:
    if isinstance(first, torch.cuda.Event):
        return float(first.elapsed_time(last))
    return (float(last) - float(first)) * 1e3


class _Ledger:
    """The spans of one phase: unresolved mark pairs plus settled durations
    (each with the step and layer it was recorded for)."""

    __slots__ = ("open_pairs", "settled")

    def __init__(self) -> None:
        self.open_pairs: List[Tuple[Mark, Mark, int, int]] = []
        self.settled: List[Tuple[float, int, int]] = []

    def needs_device(self) -> bool:
        return any(isinstance(a, torch.cuda.Event) for a, _, _, _ in self.open_pairs)

    def settle(self) -> None:
        self.settled.extend((_span_ms(a, b), s, l) for a, b, s, l in self.open_pairs)
        self.open_pairs = []

    def total_ms(self) -> float:
        return sum(ms for ms, _, _ in self.settled)


class AttentionTimingRecorder:
    """Per-phase timing of DFS calls; disabled recorders take no marks."""

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
    # Recorded phase name -> CSV row it is summed into.
    _CSV_ROW = {"topk_mask": "top_k_selection", "attention_execution": "attention_execution"}

    def __init__(self, enabled: bool = False) -> None:
        self.enabled = enabled
        self._ledgers: Dict[str, _Ledger] = {}
        self._metric_snapshots: List[Dict[str, float]] = []

    def reset(self, enabled: bool) -> None:
        """Drop everything recorded and switch recording on or off."""
        self.enabled = enabled
        self._ledgers = {}
        self._metric_snapshots = []

    def record_metrics(self, metrics: Dict[str, float]) -> None:
        """One snapshot of route statistics; the CSV reports each field's
        mean over the snapshots that carry it."""
        if self.enabled:
            self._metric_snapshots.append({k: float(v) for k, v in metrics.items()})

    def start(self, device: torch.device) -> Optional[Mark]:
        """Opening mark of a phase (None when disabled)."""
        return _take_mark(device) if self.enabled else None

    def stop(self, start: Optional[Mark], phase: str, step_idx: int, layer_idx: int, device: torch.device) -> None:
        """Closes the span opened by ``start`` and files it under ``phase``."""
        if not self.enabled or start is None:
            return
        ledger = self._ledgers.setdefault(phase, _Ledger())
        ledger.open_pairs.append((start, _take_mark(device), int(step_idx), int(layer_idx)))

    def _settle(self) -> None:
        if any(ledger.needs_device() for ledger in self._ledgers.values()):
            torch.cuda.synchronize()
        for ledger in self._ledgers.values():
            ledger.settle()

    def rows(self) -> List[Dict[str, object]]:
        """Every settled span as {phase, step_idx, layer_idx, elapsed_ms}."""
        self._settle()
        return [{"phase": phase, "step_idx": s, "layer_idx": l, "elapsed_ms": ms}
                for phase, ledger in self._ledgers.items() for ms, s, l in ledger.settled]

    def _csv_row_of(self, phase: str) -> Optional[str]:
        if phase in self._CSV_ROW:
            return self._CSV_ROW[phase]
        if phase in self.DETAILED_PHASES or phase.startswith("flashinfer_residual_bucket_le"):
            return phase
        return None  # recorded for rows() only, as the reference's own extra phases

    def dump_csv(self, output_path: str, extra_totals: Optional[Dict[str, float]] = None
                 ) -> Dict[str, Dict[str, float]]:
        """Writes the reference's timing CSV (timing.py:97-218): rows
        ``top_k_selection`` (the ``topk_mask`` spans), ``attention_execution``,
        every detailed phase (zero calls when not recorded), then any bucket
        phases seen, each ``extra_totals`` entry as one call, and a
        ``residual_route_stats`` row when metrics were recorded. Columns:
        phase, total_ms, calls, mean_ms and the metric fields. Returns
        {row: {calls, total_ms, mean_ms}}."""
        self._settle()
        order = ["top_k_selection", "attention_execution", *self.DETAILED_PHASES]
        acc: Dict[str, List[float]] = {row: [0.0, 0.0] for row in order}  # row -> [total_ms, calls]
        for phase, ledger in self._ledgers.items():
            row = self._csv_row_of(phase)
            if row is None:
                continue
            slot = acc.setdefault(row, [0.0, 0.0])
            slot[0] += ledger.total_ms()
            slot[1] += len(ledger.settled)
        for row, ms in (extra_totals or {}).items():
            acc[row] = [float(ms), 1.0]
        summary = {row: {"calls": n, "total_ms": t, "mean_ms": t / n if n else 0.0} for row, (t, n) in acc.items()}

        header = ["phase", "total_ms", "calls", "mean_ms", *self.METRIC_FIELDS]
        lines = [{"phase": row, "total_ms": s["total_ms"], "calls": int(s["calls"]), "mean_ms": s["mean_ms"]}
                 for row, s in summary.items()]
        per_field = {f: [snap[f] for snap in self._metric_snapshots if f in snap] for f in self.METRIC_FIELDS}
        n_stats = max(len(v) for v in per_field.values())
        if n_stats:
            lines.append({"phase": "residual_route_stats", "total_ms": "", "calls": n_stats, "mean_ms": "",
                          **{f: sum(v) / len(v) if v else float("nan") for f, v in per_field.items()}})
        os.makedirs(os.path.dirname(output_path) or ".", exist_ok=True)
        with open(output_path, "w", newline="") as fh:
            writer = csv.DictWriter(fh, fieldnames=header)
            writer.writeheader()
            writer.writerows(lines)
        return summary

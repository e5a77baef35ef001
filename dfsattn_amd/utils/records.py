"""Density and sparsity record files of the DFS attention classes, in the
formats their drivers and analysis scripts read:

* Wan execution-tile records (attention_wan.py:604-661): a printed table and
  one CSV row per (step, layer);
* HunyuanVideo density records (attention_hyvideo.py:1511-1573): a printed
  table and a CSV of density plus route statistics per (step, layer);
* HunyuanVideo density summary (attention_hyvideo.py:1575-1691, written by
  hyvideo_t2v_inference.py:390-396): one row per prompt, appended to a CSV;
* HunyuanVideo sparsity records (attention_hyvideo.py:1693-1727).

Records are ``{step: {layer: value}}`` dicts; every writer visits them in
ascending (step, layer) order.
"""
from __future__ import annotations

import csv
import math
import os
from typing import Any, Dict, Iterator, List, Optional, Sequence, Tuple

Records = Dict[int, Dict[int, Any]]

EXECUTION_TILE_FIELDS = ("step_idx", "layer_idx", "execution_backend", "execution_tile_size", "q_tile_rows",
                         "k_tile_cols", "tile_k_mean", "tile_k_min", "tile_k_max", "tiles_executed", "tiles_dense",
                         "execution_tile_density")
# (title, width, record field, format) of the printed execution-tile table.
EXECUTION_TILE_TABLE = (("step_idx", 9, "step_idx", "d"), ("layer_idx", 10, "layer_idx", "d"),
                        ("backend", 10, "execution_backend", "s"), ("tile", 6, "execution_tile_size", "d"),
                        ("k(mean)", 9, "tile_k_mean", ".2f"), ("D_HW", 9, "execution_tile_density", ".4f"))
ROUTE_FIELDS = ("residual_count_mean", "residual_count_p50", "residual_count_p95", "residual_count_max",
                "residual_count_nonempty_ratio")
DENSITY_METRIC_FIELDS = (*ROUTE_FIELDS, "fine_top_k", "occupancy_threshold", "occupancy_mean", "fine_top_ratio",
                         "occupancy_histogram")
SPARSITY_FIELDS = ("p_mass", "fine_top_p", "token_top_k", "token_top_ratio", "residual_candidate_blocks",
                   "block_density", "realized_block_sparsity", "residual_token_interactions",
                   "residual_micro_tiles", "promoted_macro_tiles", *ROUTE_FIELDS, "fine_top_k", "fine_top_ratio",
                   "occupancy_threshold", "occupancy_mean", "occupancy_histogram", "final_density",
                   "final_hybrid_sparsity")
DENSITY_DEFINITION = "final_selected_qk / all_qk; mean_over_sparse_steps_of_mean_over_recorded_layers"
HISTOGRAM_BINS = 49
RULE = "=" * 48


def ordered(records: Records) -> Iterator[Tuple[int, int, Any]]:
    """(step, layer, value) in ascending step, then layer."""
    for step in sorted(records):
        for layer in sorted(records[step]):
            yield step, layer, records[step][layer]


def _mean(values: Sequence[float]) -> float:
    return sum(values) / len(values) if values else float("nan")


def step_means(density: Records) -> List[float]:
    """Mean over each step's recorded layers, for the steps that have any."""
    return [_mean(list(layers.values())) for _, layers in sorted(density.items()) if layers]


def _write_rows(path: str, header: Sequence[str], rows: Sequence[Dict[str, Any]]) -> None:
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    with open(path, "w", newline="") as fh:
        writer = csv.DictWriter(fh, fieldnames=list(header))
        writer.writeheader()
        writer.writerows(rows)


def execution_tile_report(records: Records) -> List[str]:
    """Printed lines of the Wan execution-tile records."""
    rows = [{"step_idx": s, "layer_idx": l, **rec} for s, l, rec in ordered(records)]
    cast = {"d": int, "s": str, ".2f": float, ".4f": float}
    head = " ".join(f"{title:>{width}}" for title, width, _, _ in EXECUTION_TILE_TABLE)
    body = [" ".join(f"{cast[fmt](row[key]):>{width}{'' if fmt == 's' else fmt}}"
                     for _, width, key, fmt in EXECUTION_TILE_TABLE) for row in rows]
    dens = {s: {l: float(rec["execution_tile_density"]) for l, rec in layers.items()}
            for s, layers in records.items()}
    overall = _mean([d for _, _, d in ordered(dens)])
    per_step = _mean(step_means(dens))
    return ["\n===== DFS Attention execution-tile records =====", head, "-" * len(head), *body,
            f"\nMean execution-tile density: {overall:.4f} ({overall * 100:.2f}%)",
            f"Mean per-step execution-tile density: {per_step:.4f} ({per_step * 100:.2f}%)", RULE]


def write_execution_tiles(path: str, records: Records) -> None:
    rows = [{f: ({"step_idx": s, "layer_idx": l, **rec}).get(f) for f in EXECUTION_TILE_FIELDS}
            for s, l, rec in ordered(records)]
    _write_rows(path, EXECUTION_TILE_FIELDS, rows)


def density_report(density: Records) -> List[str]:
    """Printed lines of the HunyuanVideo density records."""
    head = f"{'step_idx':>9} {'layer_idx':>10} {'density':>9} {'density%':>9}"
    body = [f"{s:>9} {l:>10} {d:>9.4f} {d * 100:>9.2f}" for s, l, d in ordered(density)]
    overall = _mean([d for _, _, d in ordered(density)])
    per_step = _mean(step_means(density))
    return ["\n===== DFS Attention actual density records =====", head, "-" * len(head), *body,
            f"\nMean density over all layers/steps: {overall:.4f} ({overall * 100:.2f}%)",
            f"Mean density per step (averaged over layers): {per_step:.4f} ({per_step * 100:.2f}%)", RULE]


def write_density(path: str, density: Records, sparsity: Records) -> None:
    """Density per (step, layer) with the route statistics recorded for it
    (NaN where none was)."""
    rows = []
    for s, l, d in ordered(density):
        extra = sparsity.get(s, {}).get(l, {})
        rows.append({"step_idx": s, "layer_idx": l, "density": d,
                     **{f: extra.get(f, float("nan")) for f in DENSITY_METRIC_FIELDS}})
    _write_rows(path, ("step_idx", "layer_idx", "density", *DENSITY_METRIC_FIELDS), rows)


def write_sparsity(path: str, sparsity: Records) -> None:
    rows = [{"step_idx": s, "layer_idx": l, **{f: rec.get(f, float("nan")) for f in SPARSITY_FIELDS}}
            for s, l, rec in ordered(sparsity)]
    _write_rows(path, ("step_idx", "layer_idx", *SPARSITY_FIELDS), rows)


def density_summary(density: Records, sparsity: Records, prompt_idx: Optional[int] = None,
                    prompt: Optional[str] = None) -> Dict[str, Any]:
    """One prompt's summary row: the mean over sparse steps of the mean over
    each step's recorded layers (the comparison value, under several names
    the analysis scripts read), the mean over all records, counts, and the
    mean of each finite route statistic; the occupancy histogram summed bin
    by bin when any record has one."""
    records = [d for _, _, d in ordered(density)]
    per_step = step_means(density)
    canonical = _mean(per_step)
    row: Dict[str, Any] = {
        "prompt_idx": "" if prompt_idx is None else prompt_idx,
        "prompt": "" if prompt is None else prompt,
        "density_definition": DENSITY_DEFINITION,
        "mean_final_density_sparse_steps_avg_over_layers": canonical,
        "mean_density_over_sparse_step_layer_records": _mean(records),
        "mean_density_per_sparse_step": canonical,
        "mean_density_per_step_averaged_over_layers": canonical,
        "num_sparse_step_layer_records": len(records),
        "num_sparse_steps": len(per_step),
        "num_layers_with_records": len({l for layers in density.values() for l in layers}),
    }
    stats = [rec for _, _, rec in ordered(sparsity)]
    for name in (*ROUTE_FIELDS, "fine_top_k", "fine_top_ratio", "occupancy_threshold", "occupancy_mean"):
        finite = [float(r[name]) for r in stats if name in r and math.isfinite(float(r[name]))]
        row[f"mean_{name}"] = _mean(finite)
    hists = [r["occupancy_histogram"] for r in stats if r.get("occupancy_histogram")]
    if hists:
        row["occupancy_histogram"] = tuple(sum(int(h[i]) for h in hists) for i in range(HISTOGRAM_BINS))
    return row


def append_summary(path: str, row: Dict[str, Any]) -> None:
    """Appends ``row`` to the summary CSV at ``path``. Earlier rows are kept:
    a file whose columns are a subset of the row's is rewritten under the
    row's header (missing cells empty); an old two-column ``metric,value``
    file becomes one row; any other header is refused with ValueError."""
    header = list(row)
    kept: List[Dict[str, Any]] = []
    if os.path.isfile(path) and os.path.getsize(path) > 0:
        with open(path, newline="") as fh:
            reader = csv.DictReader(fh)
            cols = reader.fieldnames or []
            if cols == ["metric", "value"]:
                old = {r["metric"]: r.get("value", "") for r in reader if r.get("metric")}
                kept.append({h: old.get(h, "") for h in header})
            elif set(cols) <= set(header):
                kept.extend({h: r.get(h, "") for h in header} for r in reader)
            else:
                raise ValueError(f"Unexpected density summary schema in {path}: {cols}")
    _write_rows(path, header, [*kept, row])

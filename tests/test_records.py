"""On-disk and record formats (CPU): block-mask export and heatmaps
(visualization.py:8-330), the timing CSV (timing.py:97-218) and the
execution-tile density records (attention_wan.py:576-661)."""
import csv
import os

import numpy as np
import pytest
import torch

from dfsattn_amd.utils import visualization as vis
from dfsattn_amd.utils.timing import AttentionTimingRecorder


def test_export_block_mask_layout(tmp_path):
    mask = torch.rand(3, 6, 6, generator=torch.Generator().manual_seed(0)) < 0.4
    npy, pngs = vis.export_block_mask(mask, str(tmp_path), 12, 3, head_indices=(0, 2), save_bool=True)
    layer = tmp_path / "step_012" / "layer_03"
    assert npy == str(layer / "block_mask.npy")
    saved = np.load(npy, allow_pickle=False)
    assert saved.dtype == np.bool_ and np.array_equal(saved, mask.numpy())
    assert pngs == [str(layer / "head_00_block_mask.png"), str(layer / "head_02_block_mask.png")]
    assert all(os.path.getsize(p) > 0 for p in pngs)
    npy2, pngs2 = vis.export_block_mask(mask[1], str(tmp_path), 0, 0)  # 2D mask, default head 0, no npy
    assert npy2 is None and pngs2 == [str(tmp_path / "step_000" / "layer_00" / "head_00_block_mask.png")]
    with pytest.raises(ValueError):
        vis.export_block_mask(mask, str(tmp_path), 0, 0, head_indices=(3,))
    with pytest.raises(ValueError):
        vis.export_block_mask(mask[None], str(tmp_path), 0, 0)


def test_other_heatmaps_are_written(tmp_path):
    g = torch.Generator().manual_seed(1)
    attn = torch.softmax(torch.randn(300, 300, generator=g), -1)
    mask = torch.rand(3, 3, generator=g) < 0.5
    paths = [vis.attention_map_visualization(attn, str(tmp_path), 1, 2, 0),
             vis.mask_visualization(mask, str(tmp_path), 1, 2, 0),
             vis.mask_visualization(mask, str(tmp_path), 1, 2, 0, suffix="dense"),
             vis.attention_map_with_mask_visualization(attn, mask, str(tmp_path), 1, 2, 0, block_size=128)]
    names = [os.path.basename(p) for p in paths]
    assert names == ["head_00.png", "head_00_mask.png", "head_00_mask_dense.png", "head_00_with_mask.png"]
    assert all(os.path.getsize(p) > 0 for p in paths)


def test_timing_csv_rows_and_columns(tmp_path):
    rec = AttentionTimingRecorder(enabled=True)
    cpu = torch.device("cpu")
    for phase in ("topk_mask", "topk_mask", "attention_execution", "qkv_permute", "flashinfer_plan"):
        rec.stop(rec.start(cpu), phase=phase, step_idx=12, layer_idx=0, device=cpu)
    rec.record_metrics({"fine_top_k": 4.0})
    rec.record_metrics({"fine_top_k": 6.0})
    out = tmp_path / "t" / "timing.csv"
    summary = rec.dump_csv(str(out), extra_totals={"total_pipeline": 1234.5})
    rows = list(csv.DictReader(open(out)))
    assert list(rows[0].keys()) == ["phase", "total_ms", "calls", "mean_ms", *AttentionTimingRecorder.METRIC_FIELDS]
    phases = [r["phase"] for r in rows]
    assert phases[:2] == ["top_k_selection", "attention_execution"]
    assert phases[2:2 + len(AttentionTimingRecorder.DETAILED_PHASES)] == list(AttentionTimingRecorder.DETAILED_PHASES)
    assert phases[-2:] == ["total_pipeline", "residual_route_stats"]
    by = {r["phase"]: r for r in rows}
    assert by["top_k_selection"]["calls"] == "2" and by["attention_execution"]["calls"] == "1"
    assert by["flashinfer_plan"]["calls"] == "1" and by["flashinfer_core_run"]["calls"] == "0"
    assert "qkv_permute" not in by  # recorded but not a CSV phase, as in the reference
    assert float(by["residual_route_stats"]["fine_top_k"]) == 5.0
    assert summary["total_pipeline"] == {"calls": 1.0, "total_ms": 1234.5, "mean_ms": 1234.5}
    disabled = AttentionTimingRecorder(enabled=False)
    assert disabled.start(cpu) is None


def test_density_records_csv(tmp_path, capsys):
    from dfsattn_amd.attention_wan import DFS_Attention
    DFS_Attention.execution_tile_records.clear()
    assert DFS_Attention.dump_density_records(str(tmp_path / "none.csv")) is None
    for step, layer, dens in ((24, 1, 0.25), (24, 0, 0.5), (12, 0, 1.0)):
        DFS_Attention.execution_tile_records.setdefault(step, {})[layer] = {
            "execution_backend": "native", "execution_tile_size": 128, "q_tile_rows": 8, "k_tile_cols": 8,
            "tile_k_mean": 8 * dens, "tile_k_min": 1, "tile_k_max": 8, "tiles_executed": int(64 * dens),
            "tiles_dense": 64, "execution_tile_density": dens}
    path = DFS_Attention.dump_density_records(str(tmp_path / "d" / "density.csv"))
    rows = list(csv.DictReader(open(path)))
    assert [(r["step_idx"], r["layer_idx"]) for r in rows] == [("12", "0"), ("24", "0"), ("24", "1")]
    assert list(rows[0].keys())[:4] == ["step_idx", "layer_idx", "execution_backend", "execution_tile_size"]
    printed = capsys.readouterr().out
    assert "Mean execution-tile density: 0.5833" in printed
    assert "Mean per-step execution-tile density: 0.6875" in printed
    DFS_Attention.execution_tile_records.clear()


@pytest.mark.parametrize("module, per_entry", [("attention_wan", 3), ("attention_hyvideo", 2)])
def test_cache_info_counts_reference_fields(module, per_entry):
    """get_cache_info counts the fields the reference stores per entry
    (attention_wan.py:466-470, 664-670; attention_hyvideo.py:1178-1183),
    not this build's extra CSR fields."""
    import importlib

    from dfsattn_amd.core import MaskEntry

    cls = importlib.import_module(f"dfsattn_amd.{module}").DFS_Attention
    saved = dict(cls._cached_metadata)
    try:
        cls._cached_metadata.clear()
        for layer in range(2):
            cls._cached_metadata[(layer, "native")] = MaskEntry(
                row_ptr=None, col_idx=None, policy=None, heads=1, **{f: None for f in cls._entry_fields})
        info = cls.get_cache_info()
        assert info["num_cached_steps"] == 2
        assert info["cached_steps"] == [(0, "native"), (1, "native")]
        assert info["total_cached_layers"] == 2 * per_entry
    finally:
        cls._cached_metadata.clear()
        cls._cached_metadata.update(saved)


def _hy_records(cls):
    cls.density_records.clear()
    cls.sparsity_records.clear()
    for step, layer, dens in ((20, 3, 0.2), (20, 1, 0.4), (13, 0, 0.9)):
        cls.density_records.setdefault(step, {})[layer] = dens
    cls.sparsity_records.setdefault(20, {})[1] = {"block_density": 0.4, "final_density": 0.4,
                                                  "residual_count_mean": 2.0, "fine_top_k": float("nan")}
    cls.sparsity_records.setdefault(13, {})[0] = {"block_density": 0.9, "residual_count_mean": 4.0,
                                                  "occupancy_histogram": [1] * 49}


def test_hunyuan_density_records_format(tmp_path, capsys):
    """The HunyuanVideo density table and CSV (attention_hyvideo.py:1511-1573):
    rows in (step, layer) order, the overall mean 0.5 and the per-step mean
    (0.9 + 0.3) / 2 = 0.6, and NaN where no route statistic was recorded."""
    from dfsattn_amd.attention_hyvideo import DFS_Attention
    _hy_records(DFS_Attention)
    try:
        path = DFS_Attention.dump_density_records(str(tmp_path / "x" / "density.csv"))
        printed = capsys.readouterr().out.splitlines()
        assert "===== DFS Attention actual density records =====" in printed
        assert " step_idx  layer_idx   density  density%" in printed
        assert "       13          0    0.9000     90.00" in printed
        assert "Mean density over all layers/steps: 0.5000 (50.00%)" in printed
        assert "Mean density per step (averaged over layers): 0.6000 (60.00%)" in printed
        rows = list(csv.DictReader(open(path)))
        assert list(rows[0])[:4] == ["step_idx", "layer_idx", "density", "residual_count_mean"]
        assert list(rows[0])[-1] == "occupancy_histogram" and len(rows[0]) == 13
        assert [(r["step_idx"], r["layer_idx"]) for r in rows] == [("13", "0"), ("20", "1"), ("20", "3")]
        assert rows[1]["residual_count_mean"] == "2.0" and rows[2]["residual_count_mean"] == "nan"
        sp = DFS_Attention.dump_sparsity_records(str(tmp_path / "sp.csv"))
        srows = list(csv.DictReader(open(sp)))
        assert list(srows[0])[:3] == ["step_idx", "layer_idx", "p_mass"] and list(srows[0])[-1] == "final_hybrid_sparsity"
        assert len(srows) == 2 and srows[0]["block_density"] == "0.9" and srows[0]["final_density"] == "nan"
    finally:
        DFS_Attention.density_records.clear()
        DFS_Attention.sparsity_records.clear()


def test_hunyuan_density_summary_appends(tmp_path):
    """One row per prompt (attention_hyvideo.py:1575-1691): the per-step mean
    of layer means, the record mean, counts, finite route-statistic means,
    the summed occupancy histogram; later prompts append; an old
    metric,value file becomes a row; a foreign header is refused."""
    from dfsattn_amd.attention_hyvideo import DFS_Attention
    _hy_records(DFS_Attention)
    out = tmp_path / "density_summary.csv"
    try:
        DFS_Attention.dump_density_summary(str(out), prompt_idx=0, prompt="a cat")
        DFS_Attention.dump_density_summary(str(out), prompt_idx=1, prompt="a dog")
        rows = list(csv.DictReader(open(out)))
        assert [r["prompt"] for r in rows] == ["a cat", "a dog"]
        r = rows[0]
        assert float(r["mean_final_density_sparse_steps_avg_over_layers"]) == pytest.approx(0.6)
        assert float(r["mean_density_per_sparse_step"]) == pytest.approx(0.6)
        assert float(r["mean_density_over_sparse_step_layer_records"]) == pytest.approx(0.5)
        assert (r["num_sparse_step_layer_records"], r["num_sparse_steps"], r["num_layers_with_records"]) == ("3", "2", "3")
        assert float(r["mean_residual_count_mean"]) == 3.0 and r["mean_fine_top_k"] == "nan"
        assert r["occupancy_histogram"] == str(tuple([1] * 49))
        legacy = tmp_path / "legacy.csv"
        legacy.write_text("metric,value\nmean_density_per_sparse_step,0.25\nnum_sparse_steps,7\n")
        DFS_Attention.dump_density_summary(str(legacy), prompt_idx=2)
        lrows = list(csv.DictReader(open(legacy)))
        assert len(lrows) == 2 and lrows[0]["mean_density_per_sparse_step"] == "0.25" and lrows[0]["prompt"] == ""
        bad = tmp_path / "bad.csv"
        bad.write_text("foo,bar\n1,2\n")
        with pytest.raises(ValueError):
            DFS_Attention.dump_density_summary(str(bad))
    finally:
        DFS_Attention.density_records.clear()
        DFS_Attention.sparsity_records.clear()
    assert DFS_Attention.dump_density_summary(str(out)) is None  # nothing recorded


def test_hunyuan_subblock_profile_api():
    from dfsattn_amd.attention_hyvideo import DFS_Attention
    DFS_Attention.configure_subblock_retention_profile(None)
    assert DFS_Attention.dump_subblock_retention_profile() is None
    with pytest.raises(NotImplementedError):
        DFS_Attention.configure_subblock_retention_profile("/tmp/x", (0.9,))

"""Block-mask export (dfsattn/utils/visualization.py:8-68): optional
``block_mask.npy`` bool [H, Qb, Kb] plus per-head PNG heatmaps under
``<dir>/step_XXX/layer_YY/``."""
from __future__ import annotations

import os

import numpy as np
import torch


def export_block_mask(mask, save_dir, step_idx, layer_idx, head_indices=(0,), save_bool=False):
    if isinstance(mask, torch.Tensor):
        mask_np = mask.detach().to(device="cpu", dtype=torch.bool).numpy()
    else:
        mask_np = np.asarray(mask, dtype=bool)
    if mask_np.ndim == 2:
        mask_np = mask_np[None, ...]
    if mask_np.ndim != 3:
        raise ValueError("block mask must have shape [heads, query_blocks, key_blocks] "
                         f"or [query_blocks, key_blocks], got {mask_np.shape}")
    layer_dir = os.path.join(save_dir, f"step_{step_idx:03d}", f"layer_{layer_idx:02d}")
    os.makedirs(layer_dir, exist_ok=True)
    bool_path = None
    if save_bool:
        bool_path = os.path.join(layer_dir, "block_mask.npy")
        np.save(bool_path, mask_np, allow_pickle=False)
    heads = range(mask_np.shape[0]) if head_indices is None else head_indices
    png_paths = []
    for head in heads:
        if head < 0 or head >= mask_np.shape[0]:
            raise ValueError(f"head index {head} is out of range for {mask_np.shape[0]} heads")
        png_paths.append(_heatmap(mask_np[head], layer_dir, head))
    return bool_path, png_paths


def _heatmap(mask2d: np.ndarray, layer_dir: str, head: int) -> str:
    path = os.path.join(layer_dir, f"head_{head:02d}.png")
    try:
        import matplotlib

        matplotlib.use("Agg")
        import matplotlib.pyplot as plt
    except ImportError:  # no plotting library: keep a raw PGM image instead
        path = path[:-4] + ".pgm"
        img = (mask2d.astype(np.uint8) * 255)
        with open(path, "wb") as fh:
            fh.write(b"P5 %d %d 255\n" % (img.shape[1], img.shape[0]))
            fh.write(img.tobytes())
        return path
    fig, ax = plt.subplots(figsize=(6, 6))
    ax.imshow(mask2d, cmap="Blues", interpolation="nearest")
    ax.set_xlabel("key block")
    ax.set_ylabel("query block")
    ax.set_title(f"head {head}: kept {mask2d.mean() * 100:.1f}%")
    fig.savefig(path, dpi=100, bbox_inches="tight")
    plt.close(fig)
    return path

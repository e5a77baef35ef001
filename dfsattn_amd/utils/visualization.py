"""Block-mask export and diagnostic heatmaps (dfsattn/utils/visualization.py).

Files go under ``<save_dir>/step_XXX/layer_YY/`` with the reference's names:
``block_mask.npy`` (bool [H, Qb, Kb], optional), ``head_HH_block_mask.png``
(selected blocks), ``head_HH.png`` (attention map), ``head_HH_mask[_sfx].png``
and ``head_HH_with_mask.png``. Heatmaps are drawn with matplotlib alone.
"""
from __future__ import annotations

import os
from typing import Optional, Sequence

import numpy as np
import torch


def _layer_dir(save_dir: str, step_idx: int, layer_idx: int) -> str:
    path = os.path.join(save_dir, f"step_{step_idx:03d}", f"layer_{layer_idx:02d}")
    os.makedirs(path, exist_ok=True)
    return path


def _as_bool(mask) -> np.ndarray:
    if isinstance(mask, torch.Tensor):
        return mask.detach().to(device="cpu", dtype=torch.bool).numpy()
    return np.asarray(mask, dtype=bool)


def _pyplot():
    import matplotlib

    matplotlib.use("Agg")
    import matplotlib.pyplot as plt

    return plt


def export_block_mask(mask, save_dir: str, step_idx: int, layer_idx: int,
                      head_indices: Optional[Sequence[int]] = (0,), save_bool: bool = False):
    """Per-head heatmaps of a [H, Qb, Kb] (or [Qb, Kb]) mask and, with
    ``save_bool``, the bool array itself (visualization.py:8-68). Returns
    (npy path or None, list of PNG paths); ``head_indices`` None renders
    every head."""
    mask_np = _as_bool(mask)
    if mask_np.ndim == 2:
        mask_np = mask_np[None, ...]
    if mask_np.ndim != 3:
        raise ValueError("block mask must have shape [heads, query_blocks, key_blocks] "
                         f"or [query_blocks, key_blocks], got {mask_np.shape}")
    layer_dir = _layer_dir(save_dir, step_idx, layer_idx)
    bool_path = None
    if save_bool:
        bool_path = os.path.join(layer_dir, "block_mask.npy")
        np.save(bool_path, mask_np, allow_pickle=False)
    heads = range(mask_np.shape[0]) if head_indices is None else head_indices
    pngs = []
    for head in heads:
        if head < 0 or head >= mask_np.shape[0]:
            raise ValueError(f"head index {head} is out of range for {mask_np.shape[0]} heads")
        pngs.append(block_mask_visualization(mask_np[head], save_dir, step_idx, layer_idx, head))
    return bool_path, pngs


def block_mask_visualization(mask, save_dir: str, step_idx: int, layer_idx: int, head_idx: int) -> str:
    """Selected blocks of one head with block-index axes
    (visualization.py:71-121)."""
    mask_np = _as_bool(mask)
    if mask_np.ndim != 2:
        raise ValueError(f"per-head block mask must be 2D, got {mask_np.shape}")
    q_blocks, k_blocks = mask_np.shape
    layer_dir = _layer_dir(save_dir, step_idx, layer_idx)
    plt = _pyplot()
    fig, ax = plt.subplots(figsize=(10, 10))
    image = ax.imshow(mask_np, cmap="Blues", vmin=0, vmax=1, origin="upper", interpolation="nearest",
                      aspect="equal")
    ax.set_xticks(np.arange(0, k_blocks, max(1, -(-k_blocks // 10))))
    ax.set_yticks(np.arange(0, q_blocks, max(1, -(-q_blocks // 10))))
    ax.set_xlabel("Key block index")
    ax.set_ylabel("Query block index")
    density = float(mask_np.mean()) if mask_np.size else 0.0
    ax.set_title(f"Top-k block mask - Step {step_idx}, Layer {layer_idx}, Head {head_idx}\n"
                 f"shape={q_blocks}x{k_blocks}, selected={density:.2%}")
    bar = fig.colorbar(image, ax=ax, ticks=[0, 1], fraction=0.046, pad=0.04)
    bar.ax.set_yticklabels(["not selected", "selected"])
    path = os.path.join(layer_dir, f"head_{head_idx:02d}_block_mask.png")
    fig.savefig(path, dpi=200, bbox_inches="tight")
    plt.close(fig)
    return path


def _attention_axes(ax, attn_np: np.ndarray, frame_block: int = 240):
    """Probabilities at or below uniform (1/N) left white, the colour scale
    capped at the 99.5th percentile, grid lines every ``frame_block`` tokens
    (visualization.py:124-166)."""
    n = attn_np.shape[1]
    threshold = 1 / max(n, 1)
    shown = np.ma.masked_where(attn_np <= threshold, attn_np)
    vmax = float(np.percentile(attn_np, 99.5)) if attn_np.size else 1.0
    image = ax.imshow(shown, cmap="Reds", vmin=threshold, vmax=max(vmax, threshold), interpolation="nearest",
                      aspect="equal")
    ax.set_facecolor("white")
    ticks = np.arange(0, attn_np.shape[0] + 1, frame_block)
    ax.set_xticks(ticks - 0.5, minor=True)
    ax.set_yticks(ticks - 0.5, minor=True)
    ax.grid(which="minor", color="#dddddd", linestyle="-", linewidth=0.4)
    ax.tick_params(left=False, bottom=False, labelleft=False, labelbottom=False)
    return image


def attention_map_visualization(attn_maps, save_dir: str, step_idx: int, layer_idx: int, head_idx: int) -> str:
    """Token-level attention probabilities [Lq, Lk] of one head
    (visualization.py:124-166)."""
    attn_np = attn_maps.detach().float().cpu().numpy() if isinstance(attn_maps, torch.Tensor) else np.asarray(attn_maps)
    layer_dir = _layer_dir(save_dir, step_idx, layer_idx)
    plt = _pyplot()
    fig, ax = plt.subplots(figsize=(10, 10))
    fig.colorbar(_attention_axes(ax, attn_np), ax=ax)
    ax.set_xlabel("Key")
    ax.set_ylabel("Query")
    ax.set_title(f"Attention Map - Step {step_idx}, Layer {layer_idx}, Head {head_idx}")
    path = os.path.join(layer_dir, f"head_{head_idx:02d}.png")
    fig.savefig(path, dpi=200, bbox_inches="tight")
    plt.close(fig)
    return path


def mask_visualization(mask, save_dir: str, step_idx: int, layer_idx: int, head_idx: int, suffix: str = "") -> str:
    """A 2D mask as a heatmap (visualization.py:169-215)."""
    mask_np = mask.detach().cpu().numpy().astype(float) if isinstance(mask, torch.Tensor) else \
        np.asarray(mask).astype(float)
    layer_dir = _layer_dir(save_dir, step_idx, layer_idx)
    plt = _pyplot()
    fig, ax = plt.subplots(figsize=(10, 10))
    fig.colorbar(ax.imshow(mask_np, cmap="Blues", vmin=0, vmax=1, interpolation="nearest", aspect="equal"), ax=ax)
    ax.set_xlabel("Key Blocks")
    ax.set_ylabel("Query Blocks")
    ax.set_title(f"Selected Mask - Step {step_idx}, Layer {layer_idx}, Head {head_idx}")
    ax.tick_params(left=False, bottom=False, labelleft=False, labelbottom=False)
    name = f"head_{head_idx:02d}_mask.png" if not suffix else f"head_{head_idx:02d}_mask_{suffix}.png"
    path = os.path.join(layer_dir, name)
    fig.savefig(path, dpi=200, bbox_inches="tight")
    plt.close(fig)
    return path


def attention_map_with_mask_visualization(attn_maps, block_mask, save_dir: str, step_idx: int, layer_idx: int,
                                          head_idx: int, block_size: int) -> str:
    """Attention map with the kept blocks outlined and tinted
    (visualization.py:218-330)."""
    from matplotlib.patches import Rectangle

    attn_np = attn_maps.detach().float().cpu().numpy() if isinstance(attn_maps, torch.Tensor) else np.asarray(attn_maps)
    mask_np = _as_bool(block_mask)
    lq, lk = attn_np.shape
    layer_dir = _layer_dir(save_dir, step_idx, layer_idx)
    plt = _pyplot()
    fig, ax = plt.subplots(figsize=(12, 10))
    fig.colorbar(_attention_axes(ax, attn_np), ax=ax)
    tint = np.zeros((lq, lk, 4))
    for qb, kb in zip(*np.nonzero(mask_np)):
        q0, k0 = qb * block_size, kb * block_size
        q1, k1 = min(q0 + block_size, lq), min(k0 + block_size, lk)
        if q0 >= lq or k0 >= lk:
            continue
        ax.add_patch(Rectangle((k0 - 0.5, q0 - 0.5), k1 - k0, q1 - q0, linewidth=2, edgecolor="cyan",
                               facecolor="none", alpha=0.8))
        tint[q0:q1, k0:k1] = (0.0, 1.0, 1.0, 0.15)
    ax.imshow(tint, interpolation="nearest", aspect="equal")
    ax.set_xlabel("Key Tokens")
    ax.set_ylabel("Query Tokens")
    ax.set_title(f"Attention Map with Selected Mask - Step {step_idx}, Layer {layer_idx}, Head {head_idx}")
    path = os.path.join(layer_dir, f"head_{head_idx:02d}_with_mask.png")
    fig.savefig(path, dpi=200, bbox_inches="tight")
    plt.close(fig)
    return path

"""Wan DFS attention core (mirrors dfsattn/attention_wan.py).

``dfs_attention(q, k, v, ...)`` keeps the reference's signature and
behaviour: a per-layer ``DFS_Attention`` instance, the refresh schedule with
Wan's CFG step doubling (attention_wan.py:792-800), a class-level mask cache
keyed by (layer, backend, block, q_tile, k_tile) (attention_wan.py:147-154),
and the native block-sparse execution. The work runs in the HIP kernels of
libdfsattn_amd.so; there is no CPU path.
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .core import DfsCore, MaskEntry, operand_dtype_for
from .layout import ScoringLayout, TopkPolicy, wan_policy
from .utils import records
from .utils.logger import logger
from .utils.timing import AttentionTimingRecorder

# Per-layer DFS_Attention instances (attention_wan.py:5).
_dfs_attention_instances: Dict[int, "DFS_Attention"] = {}


def _compute_cache_schedule(step_idx: int, skip_steps: int, cache_interval: int, sparsity: float,
                            sparsity_dcrt: float) -> Tuple[bool, float]:
    """(refresh?, current sparsity) of a step (attention_wan.py:41-66): a
    refresh every ``cache_interval`` steps from ``skip_steps`` on while the
    decremented sparsity stays positive; sparsity drops by ``sparsity_dcrt``
    per interval, clamped to [0, 1]."""
    if cache_interval <= 0:
        raise ValueError("cache_interval must be greater than 0.")
    if step_idx < skip_steps:
        return False, sparsity
    raw_interval_idx = (step_idx - skip_steps) // cache_interval
    if sparsity_dcrt > 0:
        max_valid_interval = max(0, math.ceil(sparsity / sparsity_dcrt) - 1)
    else:
        max_valid_interval = raw_interval_idx
    interval_idx = min(raw_interval_idx, max_valid_interval)
    is_cache_step = raw_interval_idx <= max_valid_interval and (step_idx - skip_steps) % cache_interval == 0
    current = sparsity - interval_idx * sparsity_dcrt
    return is_cache_step, min(1.0, max(0.0, current))


class DFS_Attention(DfsCore, nn.Module):
    """Per-layer DFS attention state (attention_wan.py:69-670)."""

    _cached_metadata: Dict[Tuple[Any, ...], Dict[str, Any]] = {}
    mask_output_dir: Optional[str] = None
    mask_head_indices: Optional[Tuple[int, ...]] = (0,)
    mask_layer_interval: int = 15
    mask_save_bool: bool = False
    record_density: bool = False
    density_records: Dict[int, Dict[int, float]] = {}
    execution_tile_records: Dict[int, Dict[int, Dict[str, Any]]] = {}
    timing_recorder = AttentionTimingRecorder()

    def __init__(self, step_idx: int, layer_idx: int, sparse_ratio: float = 0.5, cache_flag: bool = True,
                 video_perm: Optional[torch.Tensor] = None, block_size: int = 128, q_tile_size: int = 32,
                 k_tile_size: int = 32, sparse_execution: str = "native", hybrid_threshold: int = 8):
        super().__init__()
        self.step_idx = step_idx
        self.layer_idx = layer_idx
        self.sparse_ratio = sparse_ratio
        self.cache_flag = cache_flag
        self.video_perm = video_perm
        self.block_size = block_size
        self.q_tile_size = q_tile_size
        self.k_tile_size = k_tile_size
        self.sparse_execution = sparse_execution
        self.hybrid_threshold = hybrid_threshold

    # Wan: every token is a video token.
    def _video_len(self, seq_len: int) -> int:
        return seq_len

    def _policy(self, layout: ScoringLayout, sparse_ratio: float) -> TopkPolicy:
        return wan_policy(layout, sparse_ratio)

    def _mask_cache_key(self) -> Tuple[Any, ...]:
        return (self.layer_idx, self.sparse_execution, self.block_size, self.q_tile_size, self.k_tile_size)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                causal: bool = False, drop_rate: float = 0.0, cu_seqlens_q: Optional[torch.Tensor] = None,
                cu_seqlens_kv: Optional[torch.Tensor] = None, max_seqlen_q: Optional[int] = None,
                max_seqlen_kv: Optional[int] = None, batch_size: int = 1) -> torch.Tensor:
        """q, k, v [1, H, L, D] bf16/f16 -> new [1, H, L, D] (attention_wan.py:394-547)."""
        return self._dfs_forward(q, k, v, attn_mask, causal, drop_rate, cu_seqlens_q, cu_seqlens_kv, batch_size)

    def _record_density(self, entry: MaskEntry, seq_len: int) -> None:
        """Execution-tile records (attention_wan.py:514-532) from the policy's
        row counts: no device read-back."""
        counts = self._tile_counts(entry)
        pol: TopkPolicy = entry["policy"]
        executed = int(counts.sum())
        dense = entry["heads"] * pol.q_blocks * pol.k_blocks
        density = executed / dense
        DFS_Attention.density_records.setdefault(self.step_idx, {})[self.layer_idx] = density
        DFS_Attention.execution_tile_records.setdefault(self.step_idx, {})[self.layer_idx] = {
            "execution_backend": self.sparse_execution, "execution_tile_size": self.block_size,
            "q_tile_rows": pol.q_blocks, "k_tile_cols": pol.k_blocks, "tile_k_mean": float(counts.mean()),
            "tile_k_min": int(counts.min()), "tile_k_max": int(counts.max()), "tiles_executed": executed,
            "tiles_dense": dense, "execution_tile_density": density,
        }

    @classmethod
    def get_execution_tile_records(cls) -> Dict[int, Dict[int, Dict[str, Any]]]:
        return cls.execution_tile_records

    @classmethod
    def dump_density_records(cls, output_path: Optional[str] = None) -> Optional[str]:
        """Prints the execution-tile records as the reference's table and,
        with ``output_path``, writes them as its CSV (attention_wan.py:604-661
        define the format)."""
        if not cls.execution_tile_records:
            logger.warning("No density records found. Make sure record_density was enabled during generation.")
            return None
        for line in records.execution_tile_report(cls.execution_tile_records):
            print(line)
        if output_path is not None:
            records.write_execution_tiles(output_path, cls.execution_tile_records)
            print(f"Execution-tile records saved to: {output_path}")
        return output_path

    @classmethod
    def clear_cache(cls):
        """Clears the mask cache and the records (attention_wan.py:549-555)."""
        super().clear_cache()
        cls.execution_tile_records.clear()

    @classmethod
    def set_record_density(cls, enabled: bool):
        super().set_record_density(enabled)
        if not cls.record_density:
            cls.execution_tile_records.clear()


def dfs_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, step_idx: int = 0, skip_steps: int = 12,
                  cache_interval: int = 12, layer_idx: int = 0, sparsity: float = 0.25, sparsity_dcrt: float = 0.1,
                  tile_size: int = 32, block_size: int = 128, video_perm: Optional[torch.Tensor] = None,
                  cache_flag: bool = True, record_density: bool = False, cu_seqlens_q: Optional[torch.Tensor] = None,
                  cu_seqlens_kv: Optional[torch.Tensor] = None, max_seqlen_q: Optional[int] = None,
                  max_seqlen_kv: Optional[int] = None, sparse_execution: str = "native", hybrid_threshold: int = 8,
                  flashinfer64_top_p: float = 0.25, flashinfer64_token_top_k: Optional[int] = None,
                  flashinfer64_token_top_ratio: float = 0.10) -> torch.Tensor:
    """DFS attention of one Wan self-attention call (attention_wan.py:673-825).

    q, k, v: [B=1, H, L, D] bf16/f16 on the GPU. ``step_idx`` counts CFG passes,
    so the schedule runs on 2*skip_steps and 2*cache_interval. Returns a new
    [1, H, L, D] tensor in the input's dtype and token order."""
    if sparse_execution == "flashinfer64":
        raise ValueError("sparse_execution='flashinfer64' is a research backend not provided by this build; "
                         "use 'native'")
    if layer_idx not in _dfs_attention_instances:
        _dfs_attention_instances[layer_idx] = DFS_Attention(step_idx, layer_idx, sparsity, cache_flag, video_perm,
                                                            block_size, tile_size, tile_size, sparse_execution,
                                                            hybrid_threshold)
    attn = _dfs_attention_instances[layer_idx]
    attn.step_idx = step_idx
    is_cache_step, current = _compute_cache_schedule(step_idx, skip_steps * 2, cache_interval * 2, sparsity,
                                                     sparsity_dcrt)
    attn.sparse_ratio = current
    attn.cache_flag = cache_flag and is_cache_step
    attn.sparse_execution = sparse_execution
    attn.hybrid_threshold = hybrid_threshold
    if record_density and not DFS_Attention.record_density:
        DFS_Attention.set_record_density(True)
    return attn.forward(q=q, k=k, v=v, attn_mask=None, causal=False, drop_rate=0.0, cu_seqlens_q=cu_seqlens_q,
                        cu_seqlens_kv=cu_seqlens_kv, max_seqlen_q=max_seqlen_q, max_seqlen_kv=max_seqlen_kv,
                        batch_size=q.shape[0])

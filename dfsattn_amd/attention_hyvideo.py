"""HunyuanVideo DFS attention core (mirrors dfsattn/attention_hyvideo.py).

Differences from the Wan variant, all from the reference: appended text tokens
keep their order (identity tail of the permutation, attention_hyvideo.py:161-174),
scoring uses the padded layout [video | pad | text | pad] while execution runs
on the unpadded sequence, text key blocks are kept in every video row and text
query rows are dense (attention_hyvideo.py:424-501), the cache key includes the
sparsity (attention_hyvideo.py:196-208), and the schedule is not doubled for
CFG (attention_hyvideo.py:1944-1952). Only the native top-k selector is
provided; the block-top-p / frontier / kp research selectors are rejected.
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from .attention_wan import _compute_cache_schedule
from .core import DfsCore, MaskEntry, block_interactions
from .layout import ScoringLayout, TopkPolicy, hunyuan_policy
from .utils import records
from .utils.logger import logger
from .utils.timing import AttentionTimingRecorder

_dfs_attention_instances: Dict[int, "DFS_Attention"] = {}


class DFS_Attention(DfsCore, nn.Module):
    """Per-layer DFS attention state (attention_hyvideo.py:94-1286)."""

    _cached_metadata: Dict[Tuple[Any, ...], Dict[str, Any]] = {}
    mask_output_dir: Optional[str] = None
    mask_head_indices: Optional[Tuple[int, ...]] = (0,)
    mask_layer_interval: int = 15
    mask_save_bool: bool = False
    record_density: bool = False
    density_records: Dict[int, Dict[int, float]] = {}
    sparsity_records: Dict[int, Dict[int, Dict[str, Any]]] = {}
    timing_recorder = AttentionTimingRecorder()
    _entry_fields = ("block_mask", "frontier_mask")  # attention_hyvideo.py:1178-1183

    def __init__(self, step_idx: int, layer_idx: int, sparse_ratio: float = 0.5, cache_flag: bool = True,
                 video_len: int = 0, video_perm: Optional[torch.Tensor] = None, block_size: int = 128,
                 q_tile_size: int = 32, k_tile_size: int = 32, sparse_execution: str = "native",
                 hybrid_threshold: int = 8, block_top_p: Optional[float] = None, token_top_k: int = 0,
                 residual_candidate_blocks: int = 4, selector_mode: str = "topk", fine_top_p: float = 0.9):
        super().__init__()
        self.step_idx = step_idx
        self.layer_idx = layer_idx
        self.sparse_ratio = sparse_ratio
        self.cache_flag = cache_flag
        self.video_len = video_len
        self.video_perm = video_perm
        self.block_size = block_size
        self.q_tile_size = q_tile_size
        self.k_tile_size = k_tile_size
        self.sparse_execution = sparse_execution
        self.hybrid_threshold = hybrid_threshold
        self.block_top_p = block_top_p
        self.token_top_k = token_top_k
        self.residual_candidate_blocks = residual_candidate_blocks
        self.selector_mode = selector_mode
        self.fine_top_p = fine_top_p

    def _video_len(self, seq_len: int) -> int:
        vlen = self.video_len if self.video_len else seq_len
        if vlen > seq_len:
            raise ValueError(f"video_len={vlen} exceeds the sequence length {seq_len}")
        return vlen

    def _policy(self, layout: ScoringLayout, sparse_ratio: float) -> TopkPolicy:
        return hunyuan_policy(layout, sparse_ratio)

    def _mask_cache_key(self) -> Tuple[Any, ...]:
        return (self.layer_idx, self.block_size, self.q_tile_size, self.k_tile_size, self.sparse_ratio,
                self.block_top_p, self.token_top_k, self.residual_candidate_blocks, self.selector_mode,
                self.fine_top_p)

    def _check_selector(self) -> None:
        if self.block_top_p is not None or self.token_top_k > 0 or self.selector_mode != "topk":
            raise ValueError("only the native top-k block selector is provided (block_top_p=None, "
                             "token_top_k=0, selector_mode='topk')")

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                causal: bool = False, drop_rate: float = 0.0, cu_seqlens_q: Optional[torch.Tensor] = None,
                cu_seqlens_kv: Optional[torch.Tensor] = None, max_seqlen_q: Optional[int] = None,
                max_seqlen_kv: Optional[int] = None, batch_size: int = 1) -> torch.Tensor:
        """q, k, v [1, H, L, D] with the text tokens after the video ->
        new [1, H, L, D] (attention_hyvideo.py:1090-1286)."""
        self._check_selector()
        return self._dfs_forward(q, k, v, attn_mask, causal, drop_rate, cu_seqlens_q, cu_seqlens_kv, batch_size)

    def _record_density(self, entry: MaskEntry, seq_len: int) -> None:
        """Interaction density of the block mask without padding tokens
        (attention_hyvideo.py:1240-1284); reads the mask back once."""
        inter = block_interactions(entry["block_mask"], seq_len, self.block_size)
        total = entry["heads"] * seq_len * seq_len
        density = inter / total
        DFS_Attention.density_records.setdefault(self.step_idx, {})[self.layer_idx] = density
        DFS_Attention.sparsity_records.setdefault(self.step_idx, {})[self.layer_idx] = {
            "p_mass": float("nan"), "fine_top_p": float("nan"), "token_top_k": float(self.token_top_k),
            "residual_candidate_blocks": float(self.residual_candidate_blocks), "block_density": density,
            "realized_block_sparsity": 1.0 - density, "residual_token_interactions": 0.0,
            "final_density": density, "final_hybrid_sparsity": 1.0 - density,
        }

    @classmethod
    def clear_cache(cls):
        super().clear_cache()
        cls.sparsity_records.clear()

    @classmethod
    def get_sparsity_records(cls):
        return cls.sparsity_records

    @classmethod
    def set_record_density(cls, enabled: bool):
        super().set_record_density(enabled)
        if not cls.record_density:
            cls.sparsity_records.clear()

    @classmethod
    def dump_density_records(cls, output_path: Optional[str] = None) -> Optional[str]:
        """Prints the density records as the reference's table and, with
        ``output_path``, writes the density CSV with the route statistics
        columns (attention_hyvideo.py:1511-1573 define the format)."""
        if not cls.density_records:
            logger.warning("No density records found. Make sure record_density was enabled during generation.")
            return None
        for line in records.density_report(cls.density_records):
            print(line)
        if output_path is not None:
            records.write_density(output_path, cls.density_records, cls.sparsity_records)
            print(f"Density records saved to: {output_path}")
        return output_path

    @classmethod
    def dump_density_summary(cls, output_path: Optional[str] = None, prompt_idx: Optional[int] = None,
                             prompt: Optional[str] = None) -> Optional[str]:
        """Appends one prompt's density summary row to ``output_path``
        (attention_hyvideo.py:1575-1691; the HunyuanVideo driver calls it
        after generation, hyvideo_t2v_inference.py:390-396)."""
        if not cls.density_records:
            logger.warning("No density records found. Make sure record_density was enabled during generation.")
            return None
        row = records.density_summary(cls.density_records, cls.sparsity_records, prompt_idx, prompt)
        if output_path is not None:
            records.append_summary(output_path, row)
            logger.info("Sparse density summary saved to %s", output_path)
        return output_path

    @classmethod
    def dump_sparsity_records(cls, output_path: Optional[str] = None) -> Optional[str]:
        """Per-(step, layer) sparsity statistics as CSV
        (attention_hyvideo.py:1693-1727)."""
        if not cls.sparsity_records:
            logger.warning("No sparsity records found. Make sure --record_density true was enabled.")
            return None
        if output_path is not None:
            records.write_sparsity(output_path, cls.sparsity_records)
            logger.info("Sparsity records saved to %s", output_path)
        return output_path

    @classmethod
    def configure_subblock_retention_profile(cls, output_dir: Optional[str], masses: Tuple[float, ...] = (0.9,)):
        """The reference profiles fine-tile score mass inside selected blocks
        here (attention_hyvideo.py:1315-1324, utils/subblock_retention.py).
        The native scorer never materialises per-tile scores, so only
        ``output_dir=None`` (profiling off, the driver's default,
        hyvideo_t2v_inference.py:238) is accepted."""
        if output_dir is not None:
            raise NotImplementedError("sub-block retention profiling needs per-tile scores, which the native "
                                      "scoring kernel does not write; call with output_dir=None")

    @classmethod
    def dump_subblock_retention_profile(cls) -> Optional[str]:
        """Nothing is profiled (see configure_subblock_retention_profile): None,
        as the reference returns with profiling off."""
        return None


def dfs_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, step_idx: int = 0, skip_steps: int = 12,
                  cache_interval: int = 12, layer_idx: int = 0, sparsity: float = 0.25, sparsity_dcrt: float = 0.1,
                  tile_size: int = 32, block_size: int = 128, video_len: int = 0,
                  video_perm: Optional[torch.Tensor] = None, cache_flag: bool = True, record_density: bool = False,
                  cu_seqlens_q: Optional[torch.Tensor] = None, cu_seqlens_kv: Optional[torch.Tensor] = None,
                  max_seqlen_q: Optional[int] = None, max_seqlen_kv: Optional[int] = None,
                  sparse_execution: str = "native", hybrid_threshold: int = 8, block_top_p: Optional[float] = None,
                  token_top_k: int = 0, residual_candidate_blocks: int = 4, selector_mode: str = "topk",
                  fine_top_p: float = 0.9, flashinfer64_top_p: float = 0.25,
                  flashinfer64_token_top_k: Optional[int] = None, flashinfer64_token_top_ratio: float = 0.10,
                  flashinfer64_route_mode: str = "topk_topp", flashinfer64_tile_top_ratio: float = 0.25,
                  flashinfer64_dynamic_tile_ratio: bool = False, flashinfer64_fine_top_ratio: float = 0.2,
                  flashinfer64_fine_top_k: Optional[int] = None, flashinfer64_token_top_p: float = 0.9,
                  flashinfer64_promotion_threshold: int = 24, flashinfer64_dense_layer: int = -1,
                  flashinfer64_dense_heads=(), flashinfer64_high_omission_heads_file: Optional[str] = None,
                  flashinfer64_residual_scorer: str = "proxy", flashinfer64_residual_temperature: float = 1.0,
                  flashinfer64_residual_min_top_k: int = 20, flashinfer64_residual_max_top_k: int = 32,
                  flashinfer64_route_cache: bool = False, flashinfer64_core_only: bool = False,
                  flashinfer64_direct_macro_csr: bool = True,
                  flashinfer64_valid_sequence: Optional[int] = None) -> torch.Tensor:
    """DFS attention of one HunyuanVideo joint-attention call
    (attention_hyvideo.py:1743-1982). The flashinfer64_* arguments belong to a
    research backend and are accepted for signature compatibility only."""
    if sparse_execution == "flashinfer64":
        raise ValueError("sparse_execution='flashinfer64' is a research backend not provided by this build; "
                         "use 'native'")
    if layer_idx not in _dfs_attention_instances:
        _dfs_attention_instances[layer_idx] = DFS_Attention(
            step_idx, layer_idx, sparsity, cache_flag, video_len, video_perm, block_size, tile_size, tile_size,
            sparse_execution, hybrid_threshold, block_top_p, token_top_k, residual_candidate_blocks,
            selector_mode, fine_top_p)
    attn = _dfs_attention_instances[layer_idx]
    attn.step_idx = step_idx
    is_cache_step, current = _compute_cache_schedule(step_idx, skip_steps, cache_interval, sparsity, sparsity_dcrt)
    attn.sparse_ratio = current
    attn.cache_flag = cache_flag and is_cache_step
    attn.sparse_execution = sparse_execution
    attn.hybrid_threshold = hybrid_threshold
    attn.block_top_p = block_top_p
    attn.token_top_k = token_top_k
    attn.residual_candidate_blocks = residual_candidate_blocks
    attn.selector_mode = selector_mode
    attn.fine_top_p = fine_top_p
    # valid tokens before the padding segment of cu_seqlens [0, valid, L]
    # (the processor passes it; replace_hyvideo.py:384)
    attn.valid_sequence = flashinfer64_valid_sequence
    if record_density and not DFS_Attention.record_density:
        DFS_Attention.set_record_density(True)
    return attn.forward(q=q, k=k, v=v, attn_mask=None, causal=False, drop_rate=0.0, cu_seqlens_q=cu_seqlens_q,
                        cu_seqlens_kv=cu_seqlens_kv, max_seqlen_q=max_seqlen_q, max_seqlen_kv=max_seqlen_kv,
                        batch_size=q.shape[0])

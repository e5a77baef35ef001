"""Device flow shared by the Wan and HunyuanVideo ``DFS_Attention`` classes.

Per call: one fused gather of Q/K/V into Hilbert order (plus tile means when
the mask is refreshed), the fused scoring + top-k kernel on refresh steps, and
the block-sparse attention kernel whose epilogue writes rows straight back to
the original token order. Masks live on the device as CSR block lists; a
cached mask is reused without any host round-trip.
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import numpy as np
import torch

from . import ops
from .layout import ScoringLayout, TopkPolicy

SUPPORTED_EXECUTION = "native"

# Device copies of CSR row offsets, keyed by (policy, heads, device): the
# offsets depend only on the selection policy, never on the data.
_ROW_PTR_CACHE: Dict[Tuple[Any, ...], torch.Tensor] = {}


def row_ptr_for(policy: TopkPolicy, heads: int, device: torch.device) -> torch.Tensor:
    key = (policy, heads, str(device))
    ptr = _ROW_PTR_CACHE.get(key)
    if ptr is None:
        ptr = torch.from_numpy(policy.row_ptr(heads)).to(device)
        _ROW_PTR_CACHE[key] = ptr
    return ptr


class MaskEntry(dict):
    """Cached selection of one layer: CSR ``row_ptr`` / ``col_idx`` on the
    device. ``entry["block_mask"]`` materialises the reference's bool
    [H, Qb, Kb] mask on first access (attention_wan.py:465-470)."""

    def __getitem__(self, key):
        if key == "block_mask" and dict.get(self, "block_mask") is None:
            pol: TopkPolicy = dict.__getitem__(self, "policy")
            mask = ops.csr_to_mask(dict.__getitem__(self, "row_ptr"), dict.__getitem__(self, "col_idx"),
                                   dict.__getitem__(self, "heads"), pol.q_blocks, pol.k_blocks)
            dict.__setitem__(self, "block_mask", mask)
        return dict.__getitem__(self, key)

    def get(self, key, default=None):
        return self[key] if key in self else default

    def clone(self) -> "MaskEntry":
        out = MaskEntry(self)
        dict.__setitem__(out, "col_idx", dict.__getitem__(self, "col_idx").clone())
        if dict.get(self, "block_mask") is not None:
            dict.__setitem__(out, "block_mask", dict.__getitem__(self, "block_mask").clone())
        return out


def operand_dtype_for(dtype: torch.dtype, requested: Optional[torch.dtype]) -> torch.dtype:
    """Attention operand precision: f16 by default (Q * scale * log2(e), K, V
    and P rounded to 11 bits keep the output within 1e-3 mean-rel of fp32;
    heads beyond the f16 range are carried with exact power-of-two factors);
    bf16 keeps the inputs' bits and runs P in bf16, the reference kernel's
    precision class (~1.5e-3 mean-rel). f16 inputs always run in f16."""
    if dtype == torch.float16:
        return torch.float16
    return requested or torch.float16


class DfsCore:
    """Mixin with the device flow; subclasses provide ``_video_len`` and
    ``_policy`` and the class-level state dictionaries."""

    operand_dtype: Optional[torch.dtype] = None  # None -> operand_dtype_for default
    # The fields a cache entry holds in the reference (attention_wan.py:466-470);
    # get_cache_info counts these per entry, as the reference does (:664-670).
    _entry_fields: Tuple[str, ...] = ("block_mask", "block_indices", "flex_block_mask")

    def _prepare(self, q, k, v, perm, layout, pool: bool) -> "ops.Prepared":
        # No permuted Q: the attention kernel gathers Q rows from the input.
        return ops.prepare_qkv(q, k, v, perm, layout, operand_dtype=operand_dtype_for(q.dtype, self.operand_dtype),
                               pool=pool, q_operand=False)

    # --- permutation -----------------------------------------------------
    def _device_permutation(self, seq_len: int, device: torch.device) -> torch.Tensor:
        """int32 execution permutation on ``device`` (video order, then the
        text tail as identity), built once per (device, seq_len) instead of
        every call (attention_wan.py:113-125, 420-421)."""
        cache = self.__dict__.setdefault("_perm_cache", {})
        key = (str(device), seq_len)
        perm = cache.get(key)
        if perm is None:
            vlen = self._video_len(seq_len)
            if self.video_perm is None:
                full = torch.arange(seq_len, dtype=torch.long)
            else:
                vp = torch.as_tensor(self.video_perm).to("cpu", torch.long).flatten()
                if vp.numel() != vlen:
                    raise ValueError(f"video_perm has {vp.numel()} entries for {vlen} video tokens")
                full = torch.cat([vp, torch.arange(vlen, seq_len, dtype=torch.long)]) if seq_len > vlen else vp
            perm = ops.device_perm(full, device)
            cache[key] = perm
        return perm

    def _layout(self, seq_len: int) -> ScoringLayout:
        """Scoring layout with the instance's query and key tile sizes (each
        must divide the block, attention_wan.py:227-228)."""
        return ScoringLayout(seq_len, self._video_len(seq_len), self.q_tile_size, self.block_size,
                             k_tile=self.k_tile_size)

    # --- checks ---------------------------------------------------------------
    def _check_call(self, q, k, v, attn_mask, causal, drop_rate, batch_size):
        if self.sparse_execution != SUPPORTED_EXECUTION:
            raise ValueError(
                f"Unknown sparse_execution={self.sparse_execution!r}; this build provides 'native' only "
                "(the hybrid / flex64 / flashinfer64 research executors are not part of it).")
        if causal or drop_rate != 0.0 or attn_mask is not None:
            raise ValueError("native DFS attention is non-causal, without dropout or an extra token mask")
        if q.dim() != 4 or q.shape[0] != 1 or batch_size != 1:
            raise AssertionError("DFS Attention with block sparse currently supports batch size 1.")
        if q.device.type != "cuda":
            raise RuntimeError("DFS attention runs on a ROCm GPU (HIP kernels); got " + str(q.device))

    @staticmethod
    def _host_split(vals, seq_len: int, name: str = "cu_seqlens"):
        """Host cu_seqlens values checked against the forms the native path
        runs: None for one whole sequence ([0, L] or [0, L, L]), the values
        for a split [0, a, L]; anything else raises NotImplementedError."""
        ok = len(vals) in (2, 3) and vals[0] == 0 and vals[-1] == seq_len and all(
            0 <= a <= b for a, b in zip(vals, vals[1:]))
        if not ok:
            raise NotImplementedError(
                f"{name} {vals}: the native DFS path takes one sequence, optionally followed by one more "
                f"([0, L], [0, L, L] or [0, a, L] with L = {seq_len})")
        return None if len(vals) == 2 or vals[1] == seq_len else list(vals)

    @staticmethod
    def _sequences(cu: Optional[torch.Tensor], seq_len: int, device: torch.device,
                   name: str) -> Optional[torch.Tensor]:
        """cu_seqlens of one batch row as the device int32 vector the attention
        kernel reads, or None for one whole sequence. Host tensors are checked
        here ([0, L], [0, L, L] or [0, a, L] with 0 <= a <= L); device tensors
        keep their values on the device (no host read) and must hold 2 or 3
        entries, like the reference's block_sparse_attn_func cu_seqlens of
        batch 1 or 2 (attention_wan.py:365-386; replace_wan.py:247-250;
        replace_hyvideo.py:221-228)."""
        if cu is None:
            return None
        if cu.device.type == "cpu":
            vals = DfsCore._host_split([int(x) for x in cu.flatten().tolist()], seq_len, name)
            return None if vals is None else ops.device_cu_seqlens(vals, device)
        if cu.device != device:
            raise ValueError(f"{name} lives on {cu.device}, the inputs on {device}")
        flat = cu.reshape(-1)
        if flat.numel() not in (2, 3):
            raise NotImplementedError(
                f"{name} has {flat.numel()} entries: the native DFS path takes one sequence, optionally "
                "followed by one more")
        return flat.to(torch.int32).contiguous()

    # --- selection and execution --------------------------------------------
    def _select(self, prep: ops.Prepared, layout: ScoringLayout, sparse_ratio: float,
                want_scores: bool = False) -> MaskEntry:
        policy = self._policy(layout, sparse_ratio)
        row_ptr = row_ptr_for(policy, prep.heads, prep.device)
        col_idx, scores, _ = ops.block_score_topk(prep, policy, row_ptr, want_scores=want_scores)
        entry = MaskEntry(row_ptr=row_ptr, col_idx=col_idx, policy=policy, heads=prep.heads,
                          **{field: None for field in self._entry_fields})
        if want_scores:
            dict.__setitem__(entry, "block_scores", scores)
        return entry

    def _execute(self, prep: ops.Prepared, entry: MaskEntry, perm: torch.Tensor,
                 cu_q: Optional[torch.Tensor] = None, cu_k: Optional[torch.Tensor] = None) -> torch.Tensor:
        """block_sparse_attn_func of the selected mask (attention_wan.py:335-391,
        attention_hyvideo.py:1026-1087). With cu_seqlens [0, a, L] the
        second sequence's rows attend its own keys under the mask indexed from
        its start, as the external kernel does for the repeated mask; the split
        is read on the device."""
        return ops.bsa_fwd(prep, entry["row_ptr"], entry["col_idx"], scale=None, out_dtype=prep.dtype,
                           out_perm=perm, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k)

    @staticmethod
    def _tile_counts(entry: MaskEntry) -> np.ndarray:
        pol: TopkPolicy = entry["policy"]
        return np.tile(pol.row_counts(), entry["heads"])

    def _cache_entry(self, key, layout: ScoringLayout) -> Optional[MaskEntry]:
        entry = type(self)._cached_metadata.get(key)
        if entry is not None and entry["policy"].q_blocks != layout.q_blocks:
            return None  # a cached mask of another sequence length cannot be reused
        return entry

    def _dfs_forward(self, q, k, v, attn_mask, causal, drop_rate, cu_seqlens_q, cu_seqlens_kv, batch_size):
        """Common body of DFS_Attention.forward (attention_wan.py:394-547,
        attention_hyvideo.py:1090-1286): permute, refresh or reuse the mask,
        execute, unpermute."""
        cls = type(self)
        self._check_call(q, k, v, attn_mask, causal, drop_rate, batch_size)
        seq_len = q.shape[2]
        device = q.device
        cu_q = self._sequences(cu_seqlens_q, seq_len, device, "cu_seqlens_q")
        cu_k = self._sequences(cu_seqlens_kv, seq_len, device, "cu_seqlens_kv")
        valid = getattr(self, "valid_sequence", None)
        if cu_q is None and cu_k is None and valid is not None:
            if not 0 < valid <= seq_len:
                raise ValueError(f"valid sequence {valid} outside [1, {seq_len}]")
            if valid < seq_len:
                cu_q = cu_k = ops.device_cu_seqlens([0, valid, seq_len], device)
        if (cu_q is None) != (cu_k is None):
            # One side split, the other whole: the whole side is the first
            # sequence followed by an empty one.
            whole = ops.device_cu_seqlens([0, seq_len, seq_len], device)
            cu_q = whole if cu_q is None else cu_q
            cu_k = whole if cu_k is None else cu_k
        if cu_q is not None and cu_q.numel() != cu_k.numel():
            raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different sequence counts")
        perm = self._device_permutation(seq_len, device)
        layout = self._layout(seq_len)
        key = self._mask_cache_key()
        entry = self._cache_entry(key, layout)
        recompute = entry is None or self.cache_flag
        rec = cls.timing_recorder
        t_perm = rec.start(device)
        prep = self._prepare(q, k, v, perm, layout, pool=recompute)
        rec.stop(t_perm, phase="qkv_permute", step_idx=self.step_idx, layer_idx=self.layer_idx, device=device)
        if recompute:
            t_topk = rec.start(device)
            with torch.no_grad():
                entry = self._select(prep, layout, self.sparse_ratio)
            rec.stop(t_topk, phase="topk_mask", step_idx=self.step_idx, layer_idx=self.layer_idx, device=device)
            if self.cache_flag:
                self._store(key, entry)
            self._maybe_export(entry)
        if cls.record_density:
            self._record_density(entry, seq_len)
        t_att = rec.start(device)
        out = self._execute(prep, entry, perm, cu_q, cu_k)
        rec.stop(t_att, phase="attention_execution", step_idx=self.step_idx, layer_idx=self.layer_idx, device=device)
        return out

    def _store(self, key, entry: MaskEntry) -> None:
        type(self)._cached_metadata[key] = entry.clone()

    def _maybe_export(self, entry: MaskEntry) -> None:
        cls = type(self)
        if (cls.mask_output_dir is not None and cls.mask_layer_interval > 0
                and self.layer_idx % cls.mask_layer_interval == 0):
            from .utils.logger import logger
            from .utils.visualization import export_block_mask

            bool_path, pngs = export_block_mask(entry["block_mask"], cls.mask_output_dir, self.step_idx,
                                                self.layer_idx, cls.mask_head_indices, cls.mask_save_bool)
            logger.info("Saved top-k block heatmaps for step %s layer %s (%d heatmap(s))%s", self.step_idx,
                        self.layer_idx, len(pngs), " and bool mask to " + bool_path if bool_path else "")

    # --- class-level API shared by both variants ----------------------------
    @classmethod
    def clear_cache(cls):
        cls._cached_metadata.clear()
        cls.density_records.clear()

    @classmethod
    def configure_mask_export(cls, output_dir, head_indices=(0,), layer_interval: int = 15,
                              save_bool: bool = False):
        if layer_interval < 1:
            raise ValueError("layer_interval must be at least 1")
        cls.mask_output_dir = output_dir
        cls.mask_head_indices = head_indices
        cls.mask_layer_interval = layer_interval
        cls.mask_save_bool = bool(save_bool)

    @classmethod
    def set_record_density(cls, enabled: bool):
        cls.record_density = bool(enabled)
        if not cls.record_density:
            cls.density_records.clear()

    @classmethod
    def set_record_timing(cls, enabled: bool):
        cls.timing_recorder.reset(bool(enabled))

    @classmethod
    def dump_timing_records(cls, output_path: str, extra_totals=None):
        return cls.timing_recorder.dump_csv(output_path, extra_totals=extra_totals)

    @classmethod
    def get_density_records(cls):
        return cls.density_records

    @classmethod
    def get_cache_info(cls):
        return {
            "num_cached_steps": len(cls._cached_metadata),
            "cached_steps": list(cls._cached_metadata.keys()),
            "total_cached_layers": sum(sum(1 for f in cls._entry_fields if f in v)
                                       for v in cls._cached_metadata.values()),
        }



def block_interactions(mask: torch.Tensor, seq_len: int, block: int) -> int:
    """Selected query-key pairs of a bool [H, Qb, Kb] mask, excluding block
    padding (attention_hyvideo.py:521-546)."""
    q_last = seq_len - block * (mask.shape[-2] - 1)
    k_last = seq_len - block * (mask.shape[-1] - 1)
    interior = torch.count_nonzero(mask[:, :-1, :-1])
    last_q = torch.count_nonzero(mask[:, -1:, :-1])
    last_k = torch.count_nonzero(mask[:, :-1, -1:])
    corner = torch.count_nonzero(mask[:, -1:, -1:])
    total = interior * block * block + last_q * q_last * block + last_k * block * k_last + corner * q_last * k_last
    return int(total.item())

"""HunyuanVideo joint-attention processor with the DFS branch
(dfsattn/replace_hyvideo.py:32-464).

Drop-in for ``HunyuanVideo_DFSAttn_Processor2_0``: the same constructor
arguments (positional order of replace_hyvideo.py:32-82) and
``__call__(attn, hidden_states, encoder_hidden_states=None,
attention_mask=None, image_rotary_emb=None) -> (hidden_states,
encoder_hidden_states)``. ``attn`` is any module with the diffusers
``Attention`` members the processor uses; diffusers is not imported.

Projections, QK norms and RoPE are the model's (plain torch); the attention
runs on this library: ``dfs_attention`` on sparse steps, ``full_attention``
otherwise, chosen as at replace_hyvideo.py:314-386. The optional debug dump
(attention_debug_dir) writes the same files as replace_hyvideo.py:150-228.
"""
from __future__ import annotations

import json
import os
from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from .attention_hyvideo import DFS_Attention, dfs_attention
from .fullattention import full_attention
from .replace_wan import rms_norm_like
from .utils.logger import logger


class AttentionDebugComplete(RuntimeError):
    """Clean stop after the requested debug layers were dumped
    (replace_hyvideo.py:16-17)."""


def apply_rotary_emb(x: torch.Tensor, freqs_cis: Tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
    """RoPE as diffusers' ``apply_rotary_emb`` with its defaults (use_real,
    unbind dim -1), the function replace_hyvideo.py:342 imports: adjacent
    pairs (a, b) of D become (a cos - b sin, b cos + a sin), computed in fp32.
    x is [B, H, S, D]; cos and sin are [S, D]."""
    cos, sin = freqs_cis
    cos = cos[None, None].to(x.device)
    sin = sin[None, None].to(x.device)
    xr, xi = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    rotated = torch.stack([-xi, xr], dim=-1).flatten(3)
    return (x.float() * cos + rotated.float() * sin).to(x.dtype)


def fused_qkv_heads_per_head(attn, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                             image_rotary_emb, rope_rows: int):
    """[B, L, H*D] projections -> [B, H, L, D] q, k, v in the library's fused
    kernel: per-head RMSNorm (attn.norm_q / norm_k over D) and real RoPE of
    the first rope_rows tokens of q and k (the text after them is not
    rotated), where the reference runs its RMSNorm and RoPE kernels
    (replace_hyvideo.py:252-268)."""
    from .ops import head_norm_rope_heads
    from .replace_wan import _norm_args

    heads = attn.heads
    d = query.shape[-1] // heads
    cos = sin = None
    if image_rotary_emb is not None:
        cos, sin = (t.to(device=query.device, dtype=torch.float32).reshape(-1, d).contiguous()
                    for t in image_rotary_emb)
    wq, eq = _norm_args(attn.norm_q, d, query)
    wk, ek = _norm_args(attn.norm_k, d, key)
    q = head_norm_rope_heads(query, heads, wq, eq, cos, sin, rope_rows)
    k = head_norm_rope_heads(key, heads, wk, ek, cos, sin, rope_rows)
    v = head_norm_rope_heads(value, heads)
    return q, k, v


class HunyuanVideo_DFSAttn_Processor2_0:
    def __init__(self, mode, sparsity, tile_size, block_size, video_len, video_perm, processor_id, skip_layers,
                 skip_steps, cache_interval, sparsity_dcrt, cache_flag, dense_interval=0, rest_steps=0,
                 skip_steps2=0, record_density=False, sparse_execution="native", hybrid_threshold=8,
                 block_top_p=None, token_top_k=0, residual_candidate_blocks=4, selector_mode="topk",
                 fine_top_p=0.9, flashinfer64_top_p=0.25, flashinfer64_token_top_k=None,
                 flashinfer64_token_top_ratio=0.10, flashinfer64_route_mode="topk_topp",
                 flashinfer64_tile_top_ratio=0.25, flashinfer64_dynamic_tile_ratio=False,
                 flashinfer64_fine_top_ratio=0.2, flashinfer64_fine_top_k=None, flashinfer64_token_top_p=0.9,
                 flashinfer64_promotion_threshold=24, flashinfer64_dense_layer=-1, flashinfer64_dense_heads=(),
                 flashinfer64_high_omission_heads_file=None, flashinfer64_residual_scorer="proxy",
                 flashinfer64_residual_temperature=1.0, flashinfer64_residual_min_top_k=20,
                 flashinfer64_residual_max_top_k=32, flashinfer64_route_cache=False, flashinfer64_core_only=False,
                 flashinfer64_direct_macro_csr=True, attention_debug_dir=None, attention_debug_step=-1,
                 attention_debug_layers=(0,), attention_debug_stop=True, attention_debug_steps=None):
        self.mode = mode
        self.sparsity = sparsity
        self.tile_size = tile_size
        self.block_size = block_size
        self.video_len = video_len
        self.video_perm = video_perm
        self.step_idx = 0
        self.layer_idx = processor_id
        self.skip_layers = skip_layers
        self.skip_steps = skip_steps
        self.cache_interval = cache_interval
        self.sparsity_dcrt = sparsity_dcrt
        self.cache_flag = cache_flag
        self.dense_interval = dense_interval
        self.rest_steps = rest_steps
        self.skip_steps2 = skip_steps2
        self.record_density = record_density
        self.sparse_execution = sparse_execution
        self.hybrid_threshold = hybrid_threshold
        self.block_top_p = block_top_p
        self.token_top_k = token_top_k
        self.residual_candidate_blocks = residual_candidate_blocks
        self.selector_mode = selector_mode
        self.fine_top_p = fine_top_p
        # research-backend (flashinfer64) settings: forwarded to dfs_attention,
        # which accepts them for signature compatibility
        self.flashinfer64 = dict(
            flashinfer64_top_p=flashinfer64_top_p, flashinfer64_token_top_k=flashinfer64_token_top_k,
            flashinfer64_token_top_ratio=flashinfer64_token_top_ratio, flashinfer64_route_mode=flashinfer64_route_mode,
            flashinfer64_tile_top_ratio=flashinfer64_tile_top_ratio,
            flashinfer64_dynamic_tile_ratio=flashinfer64_dynamic_tile_ratio,
            flashinfer64_fine_top_ratio=flashinfer64_fine_top_ratio, flashinfer64_fine_top_k=flashinfer64_fine_top_k,
            flashinfer64_token_top_p=flashinfer64_token_top_p,
            flashinfer64_promotion_threshold=flashinfer64_promotion_threshold,
            flashinfer64_dense_layer=flashinfer64_dense_layer, flashinfer64_dense_heads=flashinfer64_dense_heads,
            flashinfer64_high_omission_heads_file=flashinfer64_high_omission_heads_file,
            flashinfer64_residual_scorer=flashinfer64_residual_scorer,
            flashinfer64_residual_temperature=flashinfer64_residual_temperature,
            flashinfer64_residual_min_top_k=flashinfer64_residual_min_top_k,
            flashinfer64_residual_max_top_k=flashinfer64_residual_max_top_k,
            flashinfer64_route_cache=flashinfer64_route_cache, flashinfer64_core_only=flashinfer64_core_only,
            flashinfer64_direct_macro_csr=flashinfer64_direct_macro_csr)
        for name, value in self.flashinfer64.items():
            setattr(self, name, value)
        self.attention_debug_dir = attention_debug_dir
        resolved = skip_steps if attention_debug_step < 0 else attention_debug_step
        self.attention_debug_steps = ((resolved,) if attention_debug_steps is None
                                      else tuple(dict.fromkeys(int(s) for s in attention_debug_steps)))
        if not self.attention_debug_steps or any(s < 0 for s in self.attention_debug_steps):
            raise ValueError("attention_debug_steps must contain non-negative steps")
        self.attention_debug_step = self.attention_debug_steps[0]
        self.attention_debug_layers = tuple(attention_debug_layers)
        self.attention_debug_stop = bool(attention_debug_stop)
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("HunyuanVideoAttnProcessor2_0 requires PyTorch 2.0.")

    # --- branch selection (replace_hyvideo.py:314-324) -----------------------
    def branch(self) -> str:
        """'dfs', 'dense' (dfs mode off-phase) or the full-attention mode."""
        if self.mode != "dfs":
            return self.mode
        rest_end = self.skip_steps + self.rest_steps
        sparse2_start = rest_end + self.skip_steps2
        in_sparse = (self.skip_steps <= self.step_idx < rest_end) or self.step_idx >= sparse2_start
        periodic_dense = (self.dense_interval > 0 and self.step_idx >= self.skip_steps
                          and (self.step_idx - self.skip_steps + 1) % self.dense_interval == 0)
        if self.layer_idx not in self.skip_layers and in_sparse and not periodic_dense:
            return "dfs"
        return "dense"

    @staticmethod
    def get_cu_max_seqlen(attention_mask: torch.Tensor, device):
        """[0, valid, total] for queries and keys (replace_hyvideo.py:221-228),
        built on the mask's device: the valid count never visits the host."""
        total = attention_mask.numel()
        cu = torch.full((3,), total, dtype=torch.int32, device=device)
        cu[0] = 0
        cu[1] = attention_mask.reshape(-1).sum(dtype=torch.int32).to(device)
        return cu, cu.clone(), total, total

    def _dump_attention_debug(self, query, key, value, sparse_output, dense_output, valid_sequence):
        """Tensors (.pt) and error metrics (.json) of one layer
        (replace_hyvideo.py:150-219)."""
        os.makedirs(self.attention_debug_dir, exist_ok=True)
        backend = f"dfsattn_{self.sparse_execution}_{self.selector_mode}"
        stem = f"step{self.step_idx:03d}_layer{self.layer_idx:03d}_{backend}"
        tensor_path = os.path.join(self.attention_debug_dir, stem + ".pt")
        summary_path = os.path.join(self.attention_debug_dir, stem + ".json")
        diff = sparse_output.float() - dense_output.float()
        dense_norm = torch.linalg.vector_norm(dense_output.float()).clamp_min(1e-20)
        summary = {
            "step_idx": self.step_idx, "layer_idx": self.layer_idx, "backend": backend,
            "shape": list(query.shape), "dtype": str(query.dtype), "video_len": int(self.video_len),
            "valid_sequence": int(valid_sequence), "padding_sequence": int(query.shape[2] - valid_sequence),
            "max_abs_error_vs_dense": float(diff.abs().max()), "mean_abs_error_vs_dense": float(diff.abs().mean()),
            "relative_l2_error_vs_dense": float(torch.linalg.vector_norm(diff) / dense_norm),
            "per_head_mean_abs_error": diff.abs().mean(dim=(0, 2, 3)).cpu().tolist(),
            "per_head_max_abs_error": diff.abs().amax(dim=(0, 2, 3)).cpu().tolist(),
        }
        payload = {"metadata": summary, "query": query.detach().cpu(), "key": key.detach().cpu(),
                   "value": value.detach().cpu(), "sparse_output": sparse_output.detach().cpu(),
                   "dense_output": dense_output.detach().cpu()}
        torch.save(payload, tensor_path + ".tmp")
        os.replace(tensor_path + ".tmp", tensor_path)
        with open(summary_path + ".tmp", "w", encoding="utf-8") as fh:
            json.dump(summary, fh, indent=2)
        os.replace(summary_path + ".tmp", summary_path)
        logger.info(f"Attention debug dump saved to {tensor_path}")

    @staticmethod
    def _torch_qkv_heads(attn, query, key, value, image_rotary_emb, text: Optional[torch.Tensor]):
        """Head split, the model's QK norm modules and diffusers-style RoPE in
        torch (the reference's fallback, replace_hyvideo.py:247-290); with
        ``text`` the RoPE covers the video tokens before it."""
        query = query.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        key = key.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        value = value.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        if attn.norm_q is not None:
            query = attn.norm_q(query)
        if attn.norm_k is not None:
            key = attn.norm_k(key)
        if image_rotary_emb is not None:
            if text is not None:  # RoPE on the video part only; text follows the video
                n_text = text.shape[1]
                query = torch.cat([apply_rotary_emb(query[:, :, :-n_text], image_rotary_emb),
                                   query[:, :, -n_text:]], dim=2)
                key = torch.cat([apply_rotary_emb(key[:, :, :-n_text], image_rotary_emb),
                                 key[:, :, -n_text:]], dim=2)
            else:
                query = apply_rotary_emb(query, image_rotary_emb)
                key = apply_rotary_emb(key, image_rotary_emb)
        return query, key, value

    def __call__(self, attn, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None, image_rotary_emb=None):
        single_stream = attn.add_q_proj is None and encoder_hidden_states is not None
        if single_stream:
            hidden_states = torch.cat([hidden_states, encoder_hidden_states], dim=1)
        query = attn.to_q(hidden_states)
        key = attn.to_k(hidden_states)
        value = attn.to_v(hidden_states)
        head_dim = query.shape[-1] // attn.heads
        if (self.mode != "flash" and query.is_cuda and head_dim % 8 == 0 and head_dim <= 512
                and head_dim & (head_dim - 1) == 0 and query.shape[-1] <= 8192
                and rms_norm_like(attn.norm_q, head_dim) and rms_norm_like(attn.norm_k, head_dim)):
            # fused per-head QK-RMSNorm + RoPE + head split on the GPU, where
            # the reference runs its fast kernels (replace_hyvideo.py:252-268)
            rope_rows = query.shape[1] - (encoder_hidden_states.shape[1] if single_stream else 0)
            query, key, value = fused_qkv_heads_per_head(attn, query, key, value, image_rotary_emb, rope_rows)
        else:
            query, key, value = self._torch_qkv_heads(attn, query, key, value, image_rotary_emb,
                                                      encoder_hidden_states if single_stream else None)
        if attn.add_q_proj is not None and encoder_hidden_states is not None:  # double stream
            eq = attn.add_q_proj(encoder_hidden_states).unflatten(2, (attn.heads, -1)).transpose(1, 2)
            ek = attn.add_k_proj(encoder_hidden_states).unflatten(2, (attn.heads, -1)).transpose(1, 2)
            ev = attn.add_v_proj(encoder_hidden_states).unflatten(2, (attn.heads, -1)).transpose(1, 2)
            if attn.norm_added_q is not None:
                eq = attn.norm_added_q(eq)
            if attn.norm_added_k is not None:
                ek = attn.norm_added_k(ek)
            query = torch.cat([query, eq], dim=2).contiguous()
            key = torch.cat([key, ek], dim=2).contiguous()
            value = torch.cat([value, ev], dim=2).contiguous()

        if attention_mask is None:
            attention_mask = torch.ones(query.shape[2], dtype=torch.bool, device=query.device)
        cu_q, cu_kv, max_q, max_kv = self.get_cu_max_seqlen(attention_mask, query.device)
        mode = self.branch()
        ran_sparse = False
        if mode == "dfs":
            ran_sparse = True
            hidden_states = dfs_attention(
                query, key, value, step_idx=self.step_idx, skip_steps=self.skip_steps,
                cache_interval=self.cache_interval, layer_idx=self.layer_idx, sparsity=self.sparsity,
                sparsity_dcrt=self.sparsity_dcrt, tile_size=self.tile_size, block_size=self.block_size,
                video_len=self.video_len, video_perm=self.video_perm, cache_flag=self.cache_flag,
                record_density=self.record_density, cu_seqlens_q=cu_q, cu_seqlens_kv=cu_kv, max_seqlen_q=max_q,
                max_seqlen_kv=max_kv, sparse_execution=self.sparse_execution, hybrid_threshold=self.hybrid_threshold,
                block_top_p=self.block_top_p, token_top_k=self.token_top_k,
                residual_candidate_blocks=self.residual_candidate_blocks, selector_mode=self.selector_mode,
                fine_top_p=self.fine_top_p, **self.flashinfer64)
        else:
            full_mode = "flash" if mode == "dense" else mode
            start = DFS_Attention.timing_recorder.start(query.device)
            hidden_states = full_attention(query, key, value, mode=full_mode, drop_rate=0.0,
                                           attn_mask=attention_mask, causal=False, cu_seqlens_q=cu_q,
                                           cu_seqlens_kv=cu_kv, max_seqlen_q=max_q, max_seqlen_kv=max_kv,
                                           batch_size=query.shape[0], operand_dtype=DFS_Attention.operand_dtype)
            DFS_Attention.timing_recorder.stop(start, phase="attention_execution", step_idx=self.step_idx,
                                               layer_idx=self.layer_idx, device=query.device)

        if (ran_sparse and self.attention_debug_dir is not None and self.step_idx in self.attention_debug_steps
                and self.layer_idx in self.attention_debug_layers):
            dense = full_attention(query, key, value, mode="flash", attn_mask=attention_mask, cu_seqlens_q=cu_q,
                                   cu_seqlens_kv=cu_kv, max_seqlen_q=max_q, max_seqlen_kv=max_kv,
                                   batch_size=query.shape[0])
            self._dump_attention_debug(query, key, value, hidden_states, dense, int(cu_q[1].item()))
            del dense
            if (self.attention_debug_stop and self.step_idx == max(self.attention_debug_steps)
                    and self.layer_idx == max(self.attention_debug_layers)):
                raise AttentionDebugComplete(
                    f"completed attention debug dump at step {self.step_idx}, layer {self.layer_idx}")

        hidden_states = hidden_states.transpose(1, 2).flatten(2, 3).to(query.dtype)
        if encoder_hidden_states is not None:
            n_text = encoder_hidden_states.shape[1]
            hidden_states, encoder_hidden_states = hidden_states[:, :-n_text], hidden_states[:, -n_text:]
            if getattr(attn, "to_out", None) is not None:
                hidden_states = attn.to_out[0](hidden_states)
                hidden_states = attn.to_out[1](hidden_states)
            if getattr(attn, "to_add_out", None) is not None:
                encoder_hidden_states = attn.to_add_out(encoder_hidden_states)

        self.step_idx += 1
        if self.step_idx == 50:
            self.step_idx = 0
        return hidden_states, encoder_hidden_states

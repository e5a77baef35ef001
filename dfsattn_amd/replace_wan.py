"""Wan 2.1 attention processor with the DFS branch
(dfsattn/replace_wan.py:81-324).

Drop-in for ``Wan_DFSAttn_Processor2_0``: the same positional constructor
arguments and ``__call__(attn, hidden_states, encoder_hidden_states=None,
attention_mask=None, rotary_emb=None)``. ``attn`` is any module with the
diffusers ``Attention`` members the processor uses (``to_q``, ``to_k``,
``to_v``, ``norm_q``, ``norm_k``, ``heads``, ``add_k_proj``, ``add_v_proj``,
``norm_added_k``, ``to_out``); diffusers itself is not imported.

The projections are the model's own. On the GPU (mode other than "flash",
as at replace_wan.py:162, 190) the QK RMSNorm, the complex RoPE and the head
split run in this library's fused kernel (``fused_qkv_heads``); elsewhere the
model's norm modules and the float64 complex product of the reference's
fallback (replace_wan.py:166-218) run in torch. The attention runs on this
library: ``dfs_attention`` for sparse steps and ``full_attention`` (the
block-sparse kernel with every block kept) for dense ones, chosen as at
replace_wan.py:252-308.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .attention_wan import DFS_Attention as WanDFSAttention
from .attention_wan import dfs_attention
from .fullattention import full_attention


def apply_rotary_emb_complex(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, H, L, D] rotated by complex freqs [.., L, D/2]: adjacent pairs of
    D are (real, imag), multiplied in float64 (replace_wan.py:209-213)."""
    dtype = torch.float32 if x.device.type == "mps" else torch.float64
    xc = torch.view_as_complex(x.to(dtype).unflatten(3, (-1, 2)))
    return torch.view_as_real(xc * freqs).flatten(3, 4).type_as(x)


def rope_tables(rotary_emb: torch.Tensor):
    """fp32 (cos, sin) [L, D/2] of complex RoPE frequencies [.., L, D/2], the
    conversion the reference makes for its RoPE kernel (replace_wan.py:193-198)."""
    f = rotary_emb.reshape(-1, rotary_emb.shape[-1])
    return f.real.to(torch.float32).contiguous(), f.imag.to(torch.float32).contiguous()


def rms_norm_like(norm, channels: int) -> bool:
    """True for None or an RMSNorm-style module (eps, optional [channels]
    scale, no bias) that the fused kernels can apply."""
    if norm is None:
        return True
    if isinstance(norm, torch.nn.LayerNorm) or getattr(norm, "bias", None) is not None or not hasattr(norm, "eps"):
        return False
    weight = getattr(norm, "weight", None)
    return weight is None or (weight.dim() == 1 and weight.numel() == channels)


def _norm_args(norm, channels: int, x: torch.Tensor):
    """(weight, eps) of an RMSNorm module for the fused kernel (None: no norm)."""
    if norm is None:
        return None, 0.0
    weight = getattr(norm, "weight", None)
    if weight is None:
        weight = torch.ones(channels, dtype=torch.float32, device=x.device)
    eps = getattr(norm, "eps", None)
    if eps is None:  # torch.nn.RMSNorm's default
        eps = torch.finfo(x.dtype).eps
    return weight.contiguous(), float(eps)


def fused_qkv_heads(attn, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    rotary_emb: Optional[torch.Tensor]):
    """[B, L, H*D] projections -> [B, H, L, D] q, k, v: RMSNorm over all heads
    (attn.norm_q / norm_k) and complex RoPE on q and k, and the head split, in
    the library's fused kernel (one pass per tensor)."""
    from .ops import norm_rope_heads

    heads = attn.heads
    cos = sin = None
    if rotary_emb is not None:
        cos, sin = rope_tables(rotary_emb)
    wq, eq = _norm_args(attn.norm_q, query.shape[-1], query)
    wk, ek = _norm_args(attn.norm_k, key.shape[-1], key)
    q = norm_rope_heads(query, heads, wq, eq, cos, sin)
    k = norm_rope_heads(key, heads, wk, ek, cos, sin)
    v = norm_rope_heads(value, heads)
    return q, k, v


class Wan_DFSAttn_Processor2_0:
    """Positional arguments as the Wan driver passes them
    (wan21_t2v_inference.py:150-173; replace_wan.py:81-105)."""

    def __init__(self, mode, sparsity, tile_size, block_size, video_perm, processor_id, skip_layers, skip_steps,
                 cache_interval, sparsity_dcrt, cache_flag, cross_flag, dense_step_idx=-1, dense_interval=0,
                 rest_steps=0, skip_steps2=0, record_density=False, sparse_execution="native",
                 hybrid_threshold=8, flashinfer64_top_p=0.25, flashinfer64_token_top_k=None,
                 flashinfer64_token_top_ratio=0.10):
        self.mode = mode
        self.sparsity = sparsity
        self.tile_size = tile_size
        self.block_size = block_size
        self.video_perm = video_perm
        self.step_idx = 0
        self.layer_idx = processor_id
        self.skip_layers = skip_layers
        self.skip_steps = skip_steps
        self.cache_interval = cache_interval
        self.sparsity_dcrt = sparsity_dcrt
        self.cache_flag = cache_flag
        self.cross_flag = cross_flag
        self.dense_step_idx = dense_step_idx
        self.dense_interval = dense_interval
        self.rest_steps = rest_steps
        self.skip_steps2 = skip_steps2
        self.record_density = record_density
        self.sparse_execution = sparse_execution
        self.hybrid_threshold = hybrid_threshold
        self.flashinfer64_top_p = flashinfer64_top_p
        self.flashinfer64_token_top_k = flashinfer64_token_top_k
        self.flashinfer64_token_top_ratio = flashinfer64_token_top_ratio
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("WanAttnProcessor requires PyTorch 2.0 or higher.")

    # --- branch selection (replace_wan.py:252-271) ---------------------------
    def branch(self) -> str:
        """'dfs' or 'dense' for the current call."""
        if self.mode != "dfs" or self.cross_flag is not False:
            return "dense"
        real_step = self.step_idx // 2  # the step counter counts CFG passes
        rest_end = self.skip_steps + self.rest_steps
        sparse2_start = rest_end + self.skip_steps2
        in_sparse = (self.skip_steps <= real_step < rest_end) or real_step >= sparse2_start
        periodic_dense = (self.dense_interval > 0 and real_step >= self.skip_steps
                          and (real_step - self.skip_steps + 1) % self.dense_interval == 0)
        if self.step_idx == self.dense_step_idx or periodic_dense:
            return "dense"
        if self.layer_idx not in self.skip_layers and in_sparse:
            return "dfs"
        return "dense"

    def __call__(self, attn, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None,
                 rotary_emb: Optional[torch.Tensor] = None) -> torch.Tensor:
        encoder_hidden_states_img = None
        if attn.add_k_proj is not None:
            # the text encoder's 512 tokens follow the image context (replace_wan.py:143-147)
            image_context_length = encoder_hidden_states.shape[1] - 512
            encoder_hidden_states_img = encoder_hidden_states[:, :image_context_length]
            encoder_hidden_states = encoder_hidden_states[:, image_context_length:]
        if encoder_hidden_states is None:
            encoder_hidden_states = hidden_states

        query = attn.to_q(hidden_states)
        key = attn.to_k(encoder_hidden_states)
        value = attn.to_v(encoder_hidden_states)
        if (self.mode != "flash" and query.is_cuda and query.shape[-1] <= 8192
                and (query.shape[-1] // attn.heads) % 8 == 0 and rms_norm_like(attn.norm_q, query.shape[-1])
                and rms_norm_like(attn.norm_k, key.shape[-1])):
            # fused QK-RMSNorm + RoPE + head split on the GPU, where the
            # reference runs its RMSNorm and RoPE kernels (replace_wan.py:159-205)
            query, key, value = fused_qkv_heads(attn, query, key, value, rotary_emb)
        else:
            if attn.norm_q is not None:
                query = attn.norm_q(query)
            if attn.norm_k is not None:
                key = attn.norm_k(key)
            query = query.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
            key = key.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
            value = value.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
            if rotary_emb is not None:
                query = apply_rotary_emb_complex(query, rotary_emb)
                key = apply_rotary_emb_complex(key, rotary_emb)

        hidden_states_img = None
        if encoder_hidden_states_img is not None:  # I2V image context (replace_wan.py:221-244)
            key_img = attn.add_k_proj(encoder_hidden_states_img)
            value_img = attn.add_v_proj(encoder_hidden_states_img)
            if attn.norm_added_k is not None:
                key_img = attn.norm_added_k(key_img)
            key_img = key_img.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
            value_img = value_img.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
            hidden_states_img = F.scaled_dot_product_attention(query, key_img, value_img)
            hidden_states_img = hidden_states_img.transpose(1, 2).flatten(2, 3).type_as(query)

        _, _, s_q, _ = query.shape
        s_k_total = key.shape[2]
        s_k = int(attention_mask.sum().item()) if attention_mask is not None else s_k_total
        # The reference builds these on the device (replace_wan.py:247-250);
        # their values are host integers here, so host tensors carry them and
        # no per-call synchronous copy is made (the attention paths move a
        # real split to the device themselves).
        cu_seqlens_q = torch.tensor([0, s_q, s_q], dtype=torch.int32)
        cu_seqlens_kv = torch.tensor([0, s_k, s_k_total], dtype=torch.int32)

        if self.branch() == "dfs":
            hidden_states = dfs_attention(
                query, key, value, step_idx=self.step_idx, skip_steps=self.skip_steps,
                cache_interval=self.cache_interval, layer_idx=self.layer_idx, sparsity=self.sparsity,
                sparsity_dcrt=self.sparsity_dcrt, tile_size=self.tile_size, block_size=self.block_size,
                video_perm=self.video_perm, cache_flag=self.cache_flag, record_density=self.record_density,
                cu_seqlens_q=cu_seqlens_q, cu_seqlens_kv=cu_seqlens_kv, max_seqlen_q=s_q, max_seqlen_kv=s_k_total,
                sparse_execution=self.sparse_execution, hybrid_threshold=self.hybrid_threshold,
                flashinfer64_top_p=self.flashinfer64_top_p, flashinfer64_token_top_k=self.flashinfer64_token_top_k,
                flashinfer64_token_top_ratio=self.flashinfer64_token_top_ratio)
        else:
            hidden_states = full_attention(
                query, key, value, mode="flash", drop_rate=0.0, attn_mask=attention_mask, causal=False,
                cu_seqlens_q=cu_seqlens_q, cu_seqlens_kv=cu_seqlens_kv, max_seqlen_q=s_q, max_seqlen_kv=s_k_total,
                batch_size=query.shape[0], operand_dtype=WanDFSAttention.operand_dtype)

        hidden_states = hidden_states.transpose(1, 2).flatten(2, 3).type_as(query)
        if hidden_states_img is not None:
            hidden_states = hidden_states + hidden_states_img
        hidden_states = attn.to_out[0](hidden_states)
        hidden_states = attn.to_out[1](hidden_states)

        self.step_idx += 1
        if self.step_idx == 50 * 2:  # 50 inference steps x 2 CFG passes (replace_wan.py:320-323)
            self.step_idx = 0
        return hidden_states

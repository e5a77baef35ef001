"""Dense attention of the processors' non-sparse branches
(dfsattn/fullattention.py:60-153).

``full_attention`` keeps the reference's signature and modes. Tensors are
[B, H, L, D], as the processors pass them.

* ``"flash"`` (varlen semantics of ``flash_attn_varlen_func``): query
  segment i of ``cu_seqlens_q`` attends key segment i of ``cu_seqlens_kv``.
  Self-attention segments (same range for queries and keys, bf16/f16) run on
  this library's block-sparse kernel with every block kept. Rectangular
  segments (cross-attention, e.g. Wan's 512 text tokens) run on torch's
  ``scaled_dot_product_attention``.
* ``"torch"``: ``scaled_dot_product_attention`` on the tensors as given.
* ``"vanilla"``: explicit softmax(Q K^T / sqrt(D) + bias) V.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import ops
from .layout import ScoringLayout, dense_policy

_DENSE_CSR: Dict[Tuple[torch.device, int, int], Tuple[torch.Tensor, torch.Tensor]] = {}


def _dense_csr(device: torch.device, heads: int, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Device CSR keeping every key block of every row, cached per shape."""
    key = (device, heads, seq_len)
    if key not in _DENSE_CSR:
        layout = ScoringLayout(seq_len, seq_len, 16)
        pol = dense_policy(layout)
        row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(device)
        col_idx = torch.arange(pol.k_blocks, dtype=torch.int32, device=device).repeat(heads * pol.q_blocks)
        _DENSE_CSR[key] = (row_ptr, col_idx)
    return _DENSE_CSR[key]


def dense_attention_native(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(Q K^T / sqrt(D)) V of one [1, H, L, D] bf16/f16 sequence on the
    block-sparse kernel with a full mask (no permutation)."""
    _, heads, length, _ = q.shape
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32, device=q.device)
    prep = ops.prepare_qkv(q, k, v, ident, layout, pool=False)
    row_ptr, col_idx = _dense_csr(q.device, heads, length)
    return ops.bsa_fwd(prep, row_ptr, col_idx)


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """torch's SDPA; on the GPU restricted to its fused flash / memory-efficient
    kernels (it raises rather than fall back to the math path)."""
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v)
    return F.scaled_dot_product_attention(q, k, v)


def _segments(cu: Optional[torch.Tensor], total: int) -> List[Tuple[int, int]]:
    """[(start, end)] of the varlen segments of one batch row."""
    if cu is None:
        return [(0, total)]
    vals = [int(x) for x in cu.flatten().tolist()]
    return [(vals[i], vals[i + 1]) for i in range(len(vals) - 1)]


def _flash(q, k, v, cu_seqlens_q, cu_seqlens_kv, batch_size):
    b, h, sq, d = q.shape
    sk = k.shape[2]
    out = torch.zeros_like(q)
    # cu_seqlens index the batch-flattened sequence (B * S); the processors
    # build them for one batch row and reuse them per row.
    seg_q = _segments(cu_seqlens_q, sq)
    seg_k = _segments(cu_seqlens_kv, sk)
    if len(seg_q) != len(seg_k):
        raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different segment counts")
    for bi in range(b):
        for (q0, q1), (k0, k1) in zip(seg_q, seg_k):
            if q1 <= q0:
                continue
            if k1 <= k0:
                continue  # no keys: the reference kernel writes zeros
            qs, ks, vs = (x[bi:bi + 1, :, r0:r1].contiguous()
                          for x, (r0, r1) in ((q, (q0, q1)), (k, (k0, k1)), (v, (k0, k1))))
            if (q0, q1) == (k0, k1) and q.dtype in (torch.bfloat16, torch.float16) and q.is_cuda:
                out[bi:bi + 1, :, q0:q1] = dense_attention_native(qs, ks, vs)
            else:
                out[bi:bi + 1, :, q0:q1] = _sdpa(qs, ks, vs)
    return out


def full_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mode: str = "flash", drop_rate: float = 0,
                   attn_mask: Optional[torch.Tensor] = None, causal: bool = False,
                   cu_seqlens_q: Optional[torch.Tensor] = None, cu_seqlens_kv: Optional[torch.Tensor] = None,
                   max_seqlen_q: Optional[int] = None, max_seqlen_kv: Optional[int] = None,
                   batch_size: int = 1) -> torch.Tensor:
    """Dense attention, [B, H, S, D] in and out (fullattention.py:60-153)."""
    if mode == "flash":
        if causal:
            raise NotImplementedError("causal attention is not used by the DFS processors")
        if drop_rate:
            raise NotImplementedError("dropout is not used by the DFS processors (inference)")
        return _flash(q, k, v, cu_seqlens_q, cu_seqlens_kv, batch_size)
    if mode == "torch":
        if attn_mask is not None and attn_mask.dtype != torch.bool:
            attn_mask = attn_mask.to(q.dtype)
        return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, dropout_p=drop_rate, is_causal=causal)
    if mode == "vanilla":
        b, a, s, _ = q.shape
        s1 = k.shape[2]
        bias = torch.zeros(b, a, s, s1, dtype=q.dtype, device=q.device)
        if causal:
            if attn_mask is not None:
                raise AssertionError("Causal mask and attn_mask cannot be used together")
            keep = torch.ones(s, s, dtype=torch.bool, device=q.device).tril()
            bias.masked_fill_(~keep, float("-inf"))
        if attn_mask is not None:
            if attn_mask.dtype == torch.bool:
                bias.masked_fill_(~attn_mask, float("-inf"))
            else:
                bias = bias + attn_mask
        scores = (q @ k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(q.shape[-1])) + bias
        probs = torch.dropout(scores.softmax(dim=-1), p=drop_rate, train=True)
        return probs @ v
    raise NotImplementedError(f"Unsupported attention mode: {mode}")

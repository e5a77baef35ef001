"""Dense attention of the processors' non-sparse branches
(dfsattn/fullattention.py:60-153).

``full_attention`` keeps the reference's signature and modes. Tensors are
[B, H, L, D], as the processors pass them.

* ``"flash"`` (varlen semantics of ``flash_attn_varlen_func``): query
  segment i of ``cu_seqlens_q`` attends key segment i of ``cu_seqlens_kv``.
  Self-attention (bf16/f16 on the GPU) runs on this library's block-sparse
  kernel with every block kept, the segment split read on the device (host
  cu_seqlens of more than two segments run one segment per call).
  Rectangular attention (cross-attention, e.g. Wan's 512 text tokens) runs on
  torch's ``scaled_dot_product_attention``, with a segment mask built on the
  device when device cu_seqlens are given. Host cu_seqlens are read on the
  host; nothing here reads a device tensor back.
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


_IDENT: Dict[Tuple[torch.device, int], torch.Tensor] = {}


def _identity(device: torch.device, length: int) -> torch.Tensor:
    key = (device, length)
    if key not in _IDENT:
        _IDENT[key] = torch.arange(length, dtype=torch.int32, device=device)
    return _IDENT[key]


def dense_attention_native(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           cu_seqlens_q: Optional[torch.Tensor] = None, cu_seqlens_k: Optional[torch.Tensor] = None,
                           operand_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """softmax(Q K^T / sqrt(D)) V of one [1, H, L, D] bf16/f16 row on the
    block-sparse kernel with a full mask (no permutation); device
    cu_seqlens (2 or 3 entries) split it into sequences as the varlen
    kernel does, without a host read."""
    _, heads, length, _ = q.shape
    layout = ScoringLayout(length, length, 16)
    prep = ops.prepare_qkv(q, k, v, _identity(q.device, length), layout, operand_dtype=operand_dtype, pool=False,
                           q_operand=False)
    row_ptr, col_idx = _dense_csr(q.device, heads, length)
    return ops.bsa_fwd(prep, row_ptr, col_idx, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k)


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """torch's SDPA; on the GPU restricted to its fused flash / memory-efficient
    kernels (it raises rather than fall back to the math path)."""
    if q.is_cuda:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        backends = [SDPBackend.EFFICIENT_ATTENTION] if mask is not None else [SDPBackend.FLASH_ATTENTION,
                                                                              SDPBackend.EFFICIENT_ATTENTION]
        with sdpa_kernel(backends):
            return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)


def _host_segments(cu: Optional[torch.Tensor], total: int) -> List[Tuple[int, int]]:
    """[(start, end)] of the varlen segments of one batch row (host tensor)."""
    if cu is None:
        return [(0, total)]
    vals = [int(x) for x in cu.flatten().tolist()]
    return [(vals[i], vals[i + 1]) for i in range(len(vals) - 1)]


def _device_cu(cu: Optional[torch.Tensor], total: int, device: torch.device) -> Optional[torch.Tensor]:
    """cu_seqlens as a device int32 vector (host values copied once, cached),
    or None for one whole sequence."""
    if cu is None:
        return None
    if cu.device.type == "cpu":
        vals = [int(x) for x in cu.flatten().tolist()]
        if len(vals) == 2 and vals == [0, total]:
            return None
        return ops.device_cu_seqlens(vals, device)
    return cu.reshape(-1).to(device=device, dtype=torch.int32).contiguous()


def _segment_mask(cu_q: torch.Tensor, cu_k: torch.Tensor, sq: int, sk: int) -> torch.Tensor:
    """bool [sq, sk]: query i may attend key j when both lie in the same
    segment (device cu_seqlens of 2 or 3 entries, compared on the device)."""
    dev = cu_q.device
    qi = torch.arange(sq, device=dev, dtype=torch.int32)
    kj = torch.arange(sk, device=dev, dtype=torch.int32)
    seg_q = (qi[:, None] >= cu_q[1:-1][None, :]).sum(-1) if cu_q.numel() > 2 else torch.zeros_like(qi)
    seg_k = (kj[:, None] >= cu_k[1:-1][None, :]).sum(-1) if cu_k.numel() > 2 else torch.zeros_like(kj)
    in_q = (qi >= cu_q[0]) & (qi < cu_q[-1])
    in_k = (kj >= cu_k[0]) & (kj < cu_k[-1])
    return (seg_q[:, None] == seg_k[None, :]) & in_q[:, None] & in_k[None, :]


def _flash(q, k, v, cu_seqlens_q, cu_seqlens_kv, batch_size, operand_dtype=None):
    b, h, sq, d = q.shape
    sk = k.shape[2]
    on_host = all(c is None or c.device.type == "cpu" for c in (cu_seqlens_q, cu_seqlens_kv))
    native = q.is_cuda and q.dtype in (torch.bfloat16, torch.float16) and sq == sk
    # The device varlen path takes at most two sequences; host splits into
    # more run segment by segment below (each square segment on the native
    # kernel).
    many = on_host and any(c is not None and c.numel() > 3 for c in (cu_seqlens_q, cu_seqlens_kv))
    if q.is_cuda and (native or not on_host) and not many:
        # Device path: the segment split stays on the device.
        cq = _device_cu(cu_seqlens_q, sq, q.device)
        ck = _device_cu(cu_seqlens_kv, sk, q.device)
        if (cq is None) != (ck is None):
            whole_q = ops.device_cu_seqlens([0, sq, sq], q.device)
            whole_k = ops.device_cu_seqlens([0, sk, sk], q.device)
            cq = whole_q if cq is None else cq
            ck = whole_k if ck is None else ck
        if cq is not None and cq.numel() != ck.numel():
            raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different segment counts")
        if native:
            out = torch.empty_like(q)
            for bi in range(b):
                out[bi:bi + 1] = dense_attention_native(q[bi:bi + 1], k[bi:bi + 1], v[bi:bi + 1], cq, ck,
                                                        operand_dtype)
            return out
        if cq is None:
            return _sdpa(q, k, v)
        mask = _segment_mask(cq, ck, sq, sk)
        out = _sdpa(q, k, v, mask)
        return out.masked_fill(~mask.any(-1)[:, None], 0)  # rows without keys are zero, as in the varlen kernel
    out = torch.zeros_like(q)
    # cu_seqlens index the batch-flattened sequence (B * S); the processors
    # build them for one batch row and reuse them per row.
    seg_q = _host_segments(cu_seqlens_q, sq)
    seg_k = _host_segments(cu_seqlens_kv, sk)
    if len(seg_q) != len(seg_k):
        raise ValueError("cu_seqlens_q and cu_seqlens_kv describe different segment counts")
    for bi in range(b):
        for (q0, q1), (k0, k1) in zip(seg_q, seg_k):
            if q1 <= q0 or k1 <= k0:
                continue  # no queries, or no keys: the reference kernel writes zeros
            qs, ks, vs = (x[bi:bi + 1, :, r0:r1].contiguous()
                          for x, (r0, r1) in ((q, (q0, q1)), (k, (k0, k1)), (v, (k0, k1))))
            if native and q1 - q0 == k1 - k0:
                out[bi:bi + 1, :, q0:q1] = dense_attention_native(qs, ks, vs, operand_dtype=operand_dtype)
            else:
                out[bi:bi + 1, :, q0:q1] = _sdpa(qs, ks, vs)
    return out


def full_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mode: str = "flash", drop_rate: float = 0,
                   attn_mask: Optional[torch.Tensor] = None, causal: bool = False,
                   cu_seqlens_q: Optional[torch.Tensor] = None, cu_seqlens_kv: Optional[torch.Tensor] = None,
                   max_seqlen_q: Optional[int] = None, max_seqlen_kv: Optional[int] = None,
                   batch_size: int = 1, operand_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Dense attention, [B, H, S, D] in and out (fullattention.py:60-153).
    ``operand_dtype`` picks the native kernel's operand precision (f16 by
    default, with every finite bf16 input kept; bf16 for the reference
    kernel's precision class), as ``DFS_Attention.operand_dtype`` does for
    the sparse path."""
    if mode == "flash":
        if causal:
            raise NotImplementedError("causal attention is not used by the DFS processors")
        if drop_rate:
            raise NotImplementedError("dropout is not used by the DFS processors (inference)")
        return _flash(q, k, v, cu_seqlens_q, cu_seqlens_kv, batch_size, operand_dtype)
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

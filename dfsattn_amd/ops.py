"""Device operations of the DFS hot path: thin wrappers over the C-ABI.

torch supplies device memory and the current stream; every computation runs
in the HIP kernels of libdfsattn_amd.so. Tensors must live on a ROCm device —
there is deliberately no CPU path here.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import torch

from . import _lib
from .layout import ScoringLayout, TopkPolicy

DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_device(*tensors: Optional[torch.Tensor]) -> None:
    """Every given tensor lives on one and the same ROCm device."""
    first = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "DFS kernels run on a ROCm GPU only; got a tensor on " + str(t.device))
        if first is None:
            first = t.device
        elif t.device != first:
            raise RuntimeError(f"DFS kernel operands must share one device, got {first} and {t.device}")


def _require_int32(**tensors: Optional[torch.Tensor]) -> None:
    """Index operands (permutations, CSR offsets and columns) are contiguous int32."""
    for name, t in tensors.items():
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int32 tensor, got {t.dtype}"
                             f"{'' if t.is_contiguous() else ' (non-contiguous)'}")


def _heads_rows(x: torch.Tensor) -> Tuple[int, int, int]:
    if x.dim() == 4:
        if x.shape[0] != 1:
            raise AssertionError("DFS Attention with block sparse currently supports batch size 1.")
        return x.shape[1], x.shape[2], x.shape[3]
    if x.dim() == 3:
        return x.shape[0], x.shape[1], x.shape[2]
    raise ValueError(f"expected [1,H,L,D] or [H,L,D], got {tuple(x.shape)}")


def device_perm(perm: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32 copy of a permutation on the device (validated on the host)."""
    p = torch.as_tensor(perm)
    if p.dim() != 1:
        raise ValueError("permutation must be 1-D")
    if p.device.type == "cpu":
        n = p.numel()
        if n and (int(p.min()) < 0 or int(p.max()) >= n or torch.unique(p).numel() != n):
            raise ValueError("video_perm is not a permutation of range(len)")
    return p.to(device=device, dtype=torch.int32).contiguous()


def permute_gather(src: torch.Tensor, perm: torch.Tensor, rows: Optional[int] = None) -> torch.Tensor:
    """out[..., i, :] = src[..., perm[i], :] (rows >= len(perm) zero)."""
    _require_device(src, perm)
    _require_int32(perm=perm)
    heads, length, dim = _heads_rows(src)
    src = src.contiguous()
    n = perm.numel()
    rows = n if rows is None else rows
    out = torch.empty((*src.shape[:-2], rows, dim), dtype=src.dtype, device=src.device)
    _lib.call("dfs_permute_gather", _ptr(src), _ptr(perm), _ptr(out), heads, length, n, rows,
              dim * src.element_size(), _stream(src))
    return out


def permute_scatter(src: torch.Tensor, perm: torch.Tensor, out: Optional[torch.Tensor] = None,
                    rows: Optional[int] = None) -> torch.Tensor:
    """out[..., perm[i], :] = src[..., i, :] for i < len(perm)."""
    _require_device(src, perm, out)
    _require_int32(perm=perm)
    if out is not None and (out.dtype != src.dtype or not out.is_contiguous() or out.shape[-1] != src.shape[-1]):
        raise ValueError("out must be a contiguous tensor of src's dtype and row width")
    heads, length, dim = _heads_rows(src)
    src = src.contiguous()
    n = perm.numel()
    if out is None:
        rows = n if rows is None else rows
        out = torch.empty((*src.shape[:-2], rows, dim), dtype=src.dtype, device=src.device)
    _, out_rows, _ = _heads_rows(out)
    _lib.call("dfs_permute_scatter", _ptr(src), _ptr(perm), _ptr(out), heads, length, n, out_rows,
              dim * src.element_size(), _stream(src))
    return out


@dataclass
class Prepared:
    """Operands of one DFS call in execution (permuted) order."""

    layout: ScoringLayout
    heads: int
    head_dim: int
    dtype: torch.dtype          # input dtype (and the default output dtype)
    operand_dtype: torch.dtype  # dtype of q_perm, k_perm and v_t
    q_perm: Optional[torch.Tensor]  # [H, R, D]; None: the attention reads q_src through q_rows
    k_perm: torch.Tensor  # [H, R, D]
    v_t: torch.Tensor     # [H, R/128, D, 128]
    q_hi: Optional[torch.Tensor] = None  # [H, q_tiles, D] bf16
    q_lo: Optional[torch.Tensor] = None
    k_hi: Optional[torch.Tensor] = None  # [H, k_tiles, D] bf16
    k_lo: Optional[torch.Tensor] = None
    # int32 [3, H] power-of-two exponents of the f16 operands (q_perm, k_perm
    # and v_t hold x * 2^-e for heads whose bf16 inputs exceed the f16 range);
    # None when the operands keep the inputs' dtype.
    exps: Optional[torch.Tensor] = None
    # Without q_perm: the contiguous input Q [H, L, D] and the int32
    # permutation (execution row r reads input row q_rows[r]).
    q_src: Optional[torch.Tensor] = None
    q_rows: Optional[torch.Tensor] = None

    @property
    def device(self) -> torch.device:
        return self.k_perm.device


def prepare_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, perm: torch.Tensor,
                layout: ScoringLayout, operand_dtype: Optional[torch.dtype] = None, pool: bool = True,
                q_operand: bool = True) -> Prepared:
    """Gathers Q, K, V into execution order (V block-transposed) and, with
    ``pool``, writes the tile means used for scoring. ``operand_dtype`` (f16
    by default) is the dtype of the attention operands: f16 rounds bf16
    inputs to f16; bf16 keeps their bits. With f16 operands from bf16 inputs
    every finite input is kept: a head whose values exceed the f16 range is
    stored scaled by an exact power of two (``Prepared.exps``), decided and
    applied on the device without a host round trip. Without ``q_operand``
    no permuted Q is written: the attention kernel gathers each Q row from
    the input itself (one read per row either way), which saves one write
    of Q per call."""
    _require_device(q, k, v, perm)
    _require_int32(perm=perm)
    heads, length, dim = _heads_rows(q)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("DFS native attention only supports fp16 and bf16 inputs")
    if k.shape != q.shape or v.shape != q.shape or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share shape and dtype")
    if length != layout.seq_len:
        raise ValueError(f"sequence length {length} does not match the layout ({layout.seq_len})")
    if perm.numel() != length:
        raise ValueError(f"permutation has {perm.numel()} entries for {length} tokens")
    operand_dtype = operand_dtype or torch.float16
    if operand_dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"operand_dtype must be bf16 or f16, got {operand_dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    dev = q.device
    rows = layout.rows
    prep = Prepared(
        layout=layout, heads=heads, head_dim=dim, dtype=q.dtype, operand_dtype=operand_dtype,
        q_perm=torch.empty((heads, rows, dim), dtype=operand_dtype, device=dev) if q_operand else None,
        k_perm=torch.empty((heads, rows, dim), dtype=operand_dtype, device=dev),
        v_t=torch.empty((heads, rows // 128, dim, 128), dtype=operand_dtype, device=dev),
    )
    if not q_operand:
        prep.q_src, prep.q_rows = q, perm
    if pool:
        prep.q_hi = torch.empty((heads, layout.q_tiles, dim), dtype=torch.bfloat16, device=dev)
        prep.q_lo = torch.empty_like(prep.q_hi)
        prep.k_hi = torch.empty((heads, layout.k_tiles, dim), dtype=torch.bfloat16, device=dev)
        prep.k_lo = torch.empty_like(prep.k_hi)
    rounds = q.dtype == torch.bfloat16 and operand_dtype == torch.float16
    flags = torch.zeros(3 * heads, dtype=torch.int32, device=dev) if rounds else None
    _lib.call("dfs_prepare_qkv", _ptr(q), _ptr(k), _ptr(v), _ptr(perm), heads, length, dim,
              DTYPE_CODE[q.dtype], layout.video_len, layout.q_tile, layout.k_tile, DTYPE_CODE[operand_dtype],
              _ptr(prep.q_perm), _ptr(prep.k_perm), _ptr(prep.v_t), _ptr(prep.q_hi), _ptr(prep.q_lo),
              _ptr(prep.k_hi), _ptr(prep.k_lo), _ptr(flags), _stream(q))
    if rounds:
        prep.exps = torch.empty((3, heads), dtype=torch.int32, device=dev)
        _lib.call("dfs_prepare_fixup", _ptr(q), _ptr(k), _ptr(v), _ptr(perm), heads, length, dim,
                  _ptr(prep.q_perm), _ptr(prep.k_perm), _ptr(prep.v_t), _ptr(flags), _ptr(prep.exps), _stream(q))
    return prep


def _policy_args(policy: TopkPolicy):
    return (policy.q_blocks, policy.k_blocks, policy.scored_rows, policy.n_cand, policy.k_pick,
            policy.dense_col, policy.dense_row)


def score_workspace_bytes(heads: int, q_tile: int, k_tile: int, q_blocks: int, k_blocks: int) -> int:
    """Bytes of the one-pass scoring workspace (per-tile partial block sums);
    0 when these tile sizes have no one-pass form (the scorer then runs its
    two passes)."""
    n = int(_lib.lib().dfs_block_score_topk_workspace_size(heads, q_tile, k_tile, q_blocks, k_blocks))
    if n < 0:
        raise ValueError(f"no scoring workspace for heads={heads} tiles={q_tile}/{k_tile} "
                         f"blocks={q_blocks}x{k_blocks}")
    return n


def block_score_topk(prep: Prepared, policy: TopkPolicy, row_ptr: torch.Tensor,
                     want_scores: bool = False, want_mask: bool = False, one_pass: bool = True):
    """Scores + top-k: returns (col_idx int32 [nnz], scores fp32 [H,Vb,Kb] or
    None, mask uint8 [H,Qb,Kb] or None). With ``one_pass`` a workspace of
    per-tile partial sums lets the kernel score every tile pair once instead
    of twice (normaliser pass, then block-sum pass), and the score matrix is
    written only when asked for. The two-pass form (and rows wider than the
    one-pass form's 16 * head_dim columns) always gets the score matrix,
    where it keeps its block sums rather than in LDS (more workgroups per
    CU)."""
    if prep.q_hi is None:
        raise ValueError("prepare_qkv was called without pooling")
    _require_device(prep.q_hi, row_ptr)
    _require_int32(row_ptr=row_ptr)
    if row_ptr.numel() != prep.heads * policy.q_blocks + 1:
        raise ValueError(f"row_ptr has {row_ptr.numel()} entries for {prep.heads} x {policy.q_blocks} rows")
    dev = prep.device
    nnz = policy.nnz(prep.heads)
    col_idx = torch.empty(nnz, dtype=torch.int32, device=dev)
    q_tile, k_tile = prep.layout.q_tile, prep.layout.k_tile
    ws_bytes = 0
    if one_pass and policy.k_blocks <= 16 * prep.head_dim:
        ws_bytes = score_workspace_bytes(prep.heads, q_tile, k_tile, policy.q_blocks, policy.k_blocks)
    one_pass_rows = ws_bytes > 0
    scores = (torch.empty((prep.heads, policy.scored_rows, policy.k_blocks), dtype=torch.float32, device=dev)
              if want_scores or not one_pass_rows else None)
    mask = (torch.empty((prep.heads, policy.q_blocks, policy.k_blocks), dtype=torch.uint8, device=dev)
            if want_mask else None)
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=dev) if one_pass_rows else None
    _lib.call("dfs_block_score_topk", _ptr(prep.q_hi), _ptr(prep.q_lo), _ptr(prep.k_hi), _ptr(prep.k_lo),
              prep.heads, prep.head_dim, q_tile, k_tile, *_policy_args(policy), _ptr(row_ptr),
              _ptr(col_idx), _ptr(scores), _ptr(mask), _ptr(ws), ws_bytes, _stream(prep.k_perm))
    return col_idx, (scores if want_scores else None), mask


def block_score_topk_noalloc(prep: Prepared, policy: TopkPolicy, row_ptr: torch.Tensor,
                             want_mask: bool = False):
    """block_score_topk through the allocation-free entry point: the block
    sums live in the library's static per-GPU scratch (at most 96 MiB), so
    the kernels allocate nothing; only col_idx (and the optional mask) are
    the caller's. Returns (col_idx, mask or None)."""
    if prep.q_hi is None:
        raise ValueError("prepare_qkv was called without pooling")
    _require_device(prep.q_hi, row_ptr)
    _require_int32(row_ptr=row_ptr)
    if row_ptr.numel() != prep.heads * policy.q_blocks + 1:
        raise ValueError(f"row_ptr has {row_ptr.numel()} entries for {prep.heads} x {policy.q_blocks} rows")
    dev = prep.device
    col_idx = torch.empty(policy.nnz(prep.heads), dtype=torch.int32, device=dev)
    mask = (torch.empty((prep.heads, policy.q_blocks, policy.k_blocks), dtype=torch.uint8, device=dev)
            if want_mask else None)
    # The library takes its scratch from the stream's device; the tensors'
    # device is also made current so that the launch and the stream agree
    # whichever device the caller has current.
    with torch.cuda.device(dev):
        _lib.call("dfs_block_score_topk_noalloc", _ptr(prep.q_hi), _ptr(prep.q_lo), _ptr(prep.k_hi),
                  _ptr(prep.k_lo), prep.heads, prep.head_dim, prep.layout.q_tile, prep.layout.k_tile,
                  *_policy_args(policy), _ptr(row_ptr), _ptr(col_idx), _ptr(mask), _stream(prep.k_perm))
    return col_idx, mask


def topk_from_scores(scores: torch.Tensor, policy: TopkPolicy, row_ptr: torch.Tensor,
                     want_mask: bool = False):
    """Top-k of given fp32 block scores [H, scored_rows, Kb] under ``policy``;
    returns (col_idx, mask or None)."""
    _require_device(scores, row_ptr)
    _require_int32(row_ptr=row_ptr)
    if scores.dtype != torch.float32 or scores.dim() != 3:
        raise ValueError("scores must be fp32 [H, rows, Kb]")
    heads = scores.shape[0]
    if scores.shape[1:] != (policy.scored_rows, policy.k_blocks):
        raise ValueError(f"scores shape {tuple(scores.shape)} does not match the policy")
    scores = scores.contiguous()
    col_idx = torch.empty(policy.nnz(heads), dtype=torch.int32, device=scores.device)
    mask = (torch.empty((heads, policy.q_blocks, policy.k_blocks), dtype=torch.uint8, device=scores.device)
            if want_mask else None)
    _lib.call("dfs_topk_from_scores", _ptr(scores), heads, *_policy_args(policy), _ptr(row_ptr),
              _ptr(col_idx), _ptr(mask), _stream(scores))
    return col_idx, mask


def _check_cu(cu: torch.Tensor, name: str, device: torch.device) -> int:
    """A device int32 cu_seqlens vector of 2 or 3 entries; returns n_seq."""
    if cu.device != device or cu.dtype != torch.int32 or not cu.is_contiguous() or cu.dim() != 1:
        raise ValueError(f"{name} must be a contiguous int32 vector on {device}")
    if cu.numel() not in (2, 3):
        raise NotImplementedError(
            f"{name} has {cu.numel()} entries: the native DFS path runs one sequence, optionally "
            "followed by one more (cu_seqlens [0, L], [0, L, L] or [0, a, L])")
    return cu.numel() - 1


def bsa_fwd(prep: Prepared, row_ptr: torch.Tensor, col_idx: torch.Tensor, scale: Optional[float] = None,
            out_dtype: Optional[torch.dtype] = None, out_perm: Optional[torch.Tensor] = None,
            want_lse: bool = False, out: Optional[torch.Tensor] = None,
            cu_seqlens_q: Optional[torch.Tensor] = None, cu_seqlens_k: Optional[torch.Tensor] = None):
    """Block-sparse attention over the CSR mask. Returns out [1, H, L, D] —
    original token order when ``out_perm`` is given, execution order otherwise —
    and the fp32 log-sum-exp [H, L] (execution order) when ``want_lse``.
    ``cu_seqlens_q`` / ``cu_seqlens_k`` (device int32, 2 or 3 entries, both
    or neither) split the call into sequences as the reference's varlen
    kernel does: sequence i's queries [cq[i], cq[i+1]) attend its keys
    [ck[i], ck[i+1]) under the mask indexed from each sequence's start; rows
    in no query sequence are zero. The offsets stay on the device."""
    _require_device(prep.k_perm, prep.q_perm, prep.q_src, row_ptr, col_idx, out_perm, out, cu_seqlens_q, cu_seqlens_k)
    _require_int32(row_ptr=row_ptr, col_idx=col_idx, out_perm=out_perm)
    if row_ptr.numel() != prep.heads * prep.layout.q_blocks + 1:
        raise ValueError(f"row_ptr has {row_ptr.numel()} entries for {prep.heads} x {prep.layout.q_blocks} rows")
    if (cu_seqlens_q is None) != (cu_seqlens_k is None):
        raise ValueError("pass both cu_seqlens_q and cu_seqlens_k or neither")
    n_seq = 1
    if cu_seqlens_q is not None:
        n_seq = _check_cu(cu_seqlens_q, "cu_seqlens_q", prep.device)
        if _check_cu(cu_seqlens_k, "cu_seqlens_k", prep.device) != n_seq:
            raise ValueError("cu_seqlens_q and cu_seqlens_k describe different sequence counts")
    L = prep.layout.seq_len
    out_dtype = out_dtype or prep.dtype
    if out is None:
        out = torch.empty((1, prep.heads, L, prep.head_dim), dtype=out_dtype, device=prep.device)
    elif out.dtype != out_dtype or not out.is_contiguous() or out.numel() != prep.heads * L * prep.head_dim:
        raise ValueError("out must be a contiguous [1, H, L, D] tensor of out_dtype")
    lse = torch.empty((prep.heads, L), dtype=torch.float32, device=out.device) if want_lse else None
    scale = 1.0 / math.sqrt(prep.head_dim) if scale is None else float(scale)
    _lib.call("dfs_bsa_fwd", _ptr(prep.q_perm), _ptr(prep.k_perm), _ptr(prep.v_t), _ptr(row_ptr),
              _ptr(col_idx), prep.heads, L, prep.head_dim, DTYPE_CODE[prep.operand_dtype],
              DTYPE_CODE[prep.operand_dtype], scale, _ptr(out), DTYPE_CODE[out_dtype], _ptr(out_perm),
              _ptr(lse), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), n_seq, _ptr(prep.exps), _ptr(prep.q_src),
              _ptr(prep.q_rows), DTYPE_CODE[prep.dtype], _stream(prep.k_perm))
    return (out, lse) if want_lse else out


_CU_CACHE: Dict[Tuple[Tuple[int, ...], str], torch.Tensor] = {}


def device_cu_seqlens(values: Sequence[int], device: torch.device) -> torch.Tensor:
    """Device int32 copy of host cu_seqlens values, cached per (values,
    device) and copied from pinned memory without waiting for the device."""
    key = (tuple(int(x) for x in values), str(device))
    t = _CU_CACHE.get(key)
    if t is None:
        host = torch.tensor(key[0], dtype=torch.int32).pin_memory()
        t = host.to(device, non_blocking=True)
        _CU_CACHE[key] = t
    return t


def mask_to_csr(mask: torch.Tensor, exact: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """bool/uint8 [H, Qb, Kb] mask -> (row_ptr int32 [H*Qb+1], col_idx int32).
    With ``exact`` the total count is read back to the host once to size
    col_idx; otherwise col_idx has room for every block (no host sync) and
    only its first row_ptr[-1] entries are meaningful."""
    _require_device(mask)
    m = mask.contiguous()
    if m.dtype == torch.bool:
        m = m.view(torch.uint8)
    rows = m.numel() // m.shape[-1]
    counts = torch.empty(rows, dtype=torch.int32, device=m.device)
    _lib.call("dfs_mask_row_counts", _ptr(m), rows, m.shape[-1], _ptr(counts), _stream(m))
    row_ptr = torch.zeros(rows + 1, dtype=torch.int32, device=m.device)
    torch.cumsum(counts, 0, out=row_ptr[1:])
    nnz = int(row_ptr[-1].item()) if exact else m.numel()
    col_idx = torch.empty(max(nnz, 1), dtype=torch.int32, device=m.device)
    _lib.call("dfs_mask_to_csr", _ptr(m), rows, m.shape[-1], _ptr(row_ptr), _ptr(col_idx), _stream(m))
    return row_ptr, col_idx[:nnz]  # storage of at least one element: never a NULL pointer


def csr_to_mask(row_ptr: torch.Tensor, col_idx: torch.Tensor, heads: int, q_blocks: int,
                k_blocks: int) -> torch.Tensor:
    """CSR -> bool mask [H, Qb, Kb] on the device."""
    _require_device(row_ptr, col_idx)
    _require_int32(row_ptr=row_ptr, col_idx=col_idx)
    if row_ptr.numel() != heads * q_blocks + 1:
        raise ValueError(f"row_ptr has {row_ptr.numel()} entries for {heads} x {q_blocks} rows")
    mask = torch.empty((heads, q_blocks, k_blocks), dtype=torch.uint8, device=row_ptr.device)
    _lib.call("dfs_csr_to_mask", _ptr(row_ptr), _ptr(col_idx), heads * q_blocks, k_blocks, _ptr(mask),
              _stream(row_ptr))
    return mask.view(torch.bool)


def hilbert3d_perm(f: int, h: int, w: int) -> torch.Tensor:
    """3D Hilbert order of an f x h x w grid (host function of the library)."""
    out = torch.empty(f * h * w, dtype=torch.int64)
    _lib.call("dfs_hilbert3d_perm", f, h, w, _ptr(out))
    return out


def _norm_rope_call(entry: str, x: torch.Tensor, out: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
                    cos: Optional[torch.Tensor], sin: Optional[torch.Tensor], rope_param: int,
                    weight_len: int, table_shape: Tuple[int, int]) -> None:
    _require_device(x, out, weight, cos, sin)
    if x.dim() != 4 or out.shape != x.shape:
        raise ValueError(f"{entry}: x and out must be 4-D [B, L, H, D] of one shape, got "
                         f"{tuple(x.shape)} and {tuple(out.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float16) or out.dtype != x.dtype:
        raise ValueError(f"{entry}: x and out must both be bf16 or f16, got {x.dtype} and {out.dtype}")
    if x.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError(f"{entry}: the channel (last) stride must be 1")
    B, L, H, D = x.shape
    w_code = 0
    if weight is not None:
        if weight.dim() != 1 or weight.numel() != weight_len or not weight.is_contiguous():
            raise ValueError(f"{entry}: weight must be a contiguous [{weight_len}] vector")
        if weight.dtype not in DTYPE_CODE:
            raise ValueError(f"{entry}: weight dtype {weight.dtype} is not supported")
        w_code = DTYPE_CODE[weight.dtype]
    if (cos is None) != (sin is None):
        raise ValueError(f"{entry}: pass both cos and sin or neither")
    if cos is not None:
        for name, t in (("cos", cos), ("sin", sin)):
            if t.dtype != torch.float32 or tuple(t.shape) != table_shape or not t.is_contiguous():
                raise ValueError(f"{entry}: {name} must be contiguous float32 {table_shape}, got "
                                 f"{t.dtype} {tuple(t.shape)}")
    _lib.call(entry, _ptr(x), x.stride(0), x.stride(1), x.stride(2), _ptr(out), out.stride(0),
              out.stride(1), out.stride(2), B, L, H, D, DTYPE_CODE[x.dtype], _ptr(weight), w_code, float(eps),
              _ptr(cos), _ptr(sin), int(rope_param), _stream(x))


def norm_rope(x: torch.Tensor, out: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
              cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None, rope_skip: int = 0) -> None:
    """RMSNorm over the H*D channels of each token and/or complex RoPE of each
    head, from x into out. Both are 4-D [B, L, H, D] views with channel
    stride 1 (any other strides, e.g. a [B, H, L, D] tensor permuted to
    (0, 2, 1, 3)); x and out may be the same tensor. weight None skips the
    norm, cos/sin None (fp32 [L - rope_skip, D/2]) skip the rotation."""
    L, H, D = x.shape[1:4] if x.dim() == 4 else (0, 0, 0)
    _norm_rope_call("dfs_norm_rope", x, out, weight, eps, cos, sin, rope_skip, H * D, (L - rope_skip, D // 2))


def head_norm_rope(x: torch.Tensor, out: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                   cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                   rope_rows: Optional[int] = None) -> None:
    """The HunyuanVideo form: RMSNorm of each head's D channels (weight [D])
    and real RoPE with fp32 tables [rope_rows, D] on tokens l < rope_rows
    (default: all); same views as norm_rope."""
    L, H, D = x.shape[1:4] if x.dim() == 4 else (0, 0, 0)
    rows = L if rope_rows is None else int(rope_rows)
    _norm_rope_call("dfs_head_norm_rope", x, out, weight, eps, cos, sin, rows, D, (rows, D))


def _split_heads(fn, x: torch.Tensor, heads: int, *args) -> torch.Tensor:
    if x.dim() != 3 or x.shape[-1] % heads:
        raise ValueError(f"expected [B, L, H*D] with H = {heads}, got {tuple(x.shape)}")
    B, L, C = x.shape
    D = C // heads
    src = x if x.stride(2) == 1 else x.contiguous()
    out = torch.empty((B, heads, L, D), dtype=x.dtype, device=x.device)
    fn(src.unflatten(2, (heads, D)), out.permute(0, 2, 1, 3), *args)
    return out


def norm_rope_heads(x: torch.Tensor, heads: int, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                    cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                    rope_skip: int = 0) -> torch.Tensor:
    """Projection output [B, L, H*D] -> new [B, H, L, D] tensor, normalised
    and rotated on the way (the head split of the attention inputs)."""
    return _split_heads(norm_rope, x, heads, weight, eps, cos, sin, rope_skip)


def head_norm_rope_heads(x: torch.Tensor, heads: int, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                         cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                         rope_rows: Optional[int] = None) -> torch.Tensor:
    """norm_rope_heads with the per-head norm and real RoPE of head_norm_rope."""
    return _split_heads(head_norm_rope, x, heads, weight, eps, cos, sin, rope_rows)


def _vec(t: Optional[torch.Tensor], channels: int, name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    v = t.reshape(-1)
    if v.numel() != channels or v.dtype != torch.float32:
        raise ValueError(f"{name} must hold {channels} float32 values, got {v.dtype} {tuple(t.shape)}")
    return v.contiguous()


def adaln_modulate(x: torch.Tensor, eps: float, weight: Optional[torch.Tensor] = None,
                   bias: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None,
                   shift: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(LayerNorm(x) * weight + bias) * (1 + scale) + shift over the last
    axis in fp32, returned in x's dtype; every vector is optional and holds
    one fp32 value per channel (broadcast over the rows)."""
    _require_device(x, weight, bias, scale, shift)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"adaln_modulate: x must be bf16 or f16, got {x.dtype}")
    C = x.shape[-1]
    vecs = [_vec(t, C, n) for t, n in ((weight, "weight"), (bias, "bias"), (scale, "scale"), (shift, "shift"))]
    xc = x.contiguous()
    out = torch.empty_like(xc)
    _lib.call("dfs_adaln_modulate", _ptr(xc), xc.numel() // C, C, DTYPE_CODE[x.dtype], *(_ptr(v) for v in vecs),
              float(eps), _ptr(out), _stream(xc))
    return out


def gated_residual(x: torch.Tensor, y: torch.Tensor, gate: torch.Tensor,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x + y * gate in fp32, returned in x's dtype (gate: one fp32 value per
    channel); ``out`` may be x itself."""
    _require_device(x, y, gate, out)
    if x.dtype not in (torch.bfloat16, torch.float16) or y.dtype != x.dtype or y.shape != x.shape:
        raise ValueError("gated_residual: x and y must be bf16 or f16 tensors of one shape and dtype")
    C = x.shape[-1]
    g = _vec(gate, C, "gate")
    xc, yc = x.contiguous(), y.contiguous()
    if out is None:
        out = torch.empty_like(xc)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("gated_residual: out must be contiguous and shaped like x")
    _lib.call("dfs_gated_residual", _ptr(xc), _ptr(yc), _ptr(g), xc.numel() // C, C, DTYPE_CODE[x.dtype],
              _ptr(out), _stream(xc))
    return out

"""Host-side shape and selection-policy logic of the DFS hot path.

Everything here is plain Python / numpy: block and tile counts, the scoring
layout, the per-row top-k policy of the Wan and HunyuanVideo variants, and the
CSR row offsets that follow from a policy. The GPU kernels receive these
numbers; nothing here touches a device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

BLOCK = 128
# Smallest tile the scoring kernel takes (32 tiles per 128-token block).
MIN_TILE = 4


@dataclass(frozen=True)
class ScoringLayout:
    """Token layout of one DFS call.

    Execution order is the permuted sequence [video | text] padded with zero
    rows to ``rows`` = ceil(L/128)*128. Scoring order inserts zero rows after
    the video up to a block multiple (dfsattn/attention_hyvideo.py:331-365;
    for Wan video_len == seq_len, attention_wan.py:176-189)."""

    seq_len: int
    video_len: int
    tile: int  # query tile (q_tile_size)
    block: int = BLOCK
    k_tile: Optional[int] = None  # key tile (k_tile_size); None: the query tile

    def __post_init__(self):
        if self.k_tile is None:
            object.__setattr__(self, "k_tile", self.tile)
        if self.block != BLOCK:
            raise ValueError(f"native DFS execution requires block_size == {BLOCK}, got {self.block}")
        # attention_wan.py:227-228; attention_hyvideo.py:406-407
        if self.tile <= 0 or self.block % self.tile != 0:
            raise AssertionError(
                f"block_dim ({self.block}) must be divisible by q_tile_size ({self.tile})")
        if self.k_tile <= 0 or self.block % self.k_tile != 0:
            raise AssertionError(
                f"block_dim ({self.block}) must be divisible by k_tile_size ({self.k_tile})")
        for name, t in (("q_tile_size", self.tile), ("k_tile_size", self.k_tile)):
            if t < MIN_TILE:
                raise NotImplementedError(
                    f"{name} {t}: the scoring kernel takes tiles of {MIN_TILE} to {self.block} tokens "
                    f"(at most {self.block // MIN_TILE} tiles per block)")
        if not 0 < self.video_len <= self.seq_len:
            raise ValueError(f"need 0 < video_len ({self.video_len}) <= seq_len ({self.seq_len})")
        padded = self.video_blocks * self.block + self.text_len
        if padded > self.k_blocks * self.block:
            raise RuntimeError(
                f"scoring layout of {padded} tokens does not fit {self.k_blocks} blocks of "
                f"{self.block}; the reference's tile view fails for this video/text split")

    @property
    def text_len(self) -> int:
        return self.seq_len - self.video_len

    @property
    def q_blocks(self) -> int:
        return math.ceil(self.seq_len / self.block)

    @property
    def k_blocks(self) -> int:
        return self.q_blocks

    @property
    def rows(self) -> int:
        return self.q_blocks * self.block

    @property
    def video_blocks(self) -> int:
        return math.ceil(self.video_len / self.block)

    @property
    def q_tile(self) -> int:
        return self.tile

    @property
    def q_tiles(self) -> int:
        return self.video_blocks * self.block // self.tile

    @property
    def k_tiles(self) -> int:
        return self.k_blocks * self.block // self.k_tile


@dataclass(frozen=True)
class TopkPolicy:
    """Which columns each mask row keeps (see dfs_block_score_topk in
    include/dfsattn_amd.h): rows < dense_row keep the k_pick best of
    columns [0, n_cand) plus columns [dense_col, Kb); rows >= dense_row keep all."""

    q_blocks: int
    k_blocks: int
    scored_rows: int
    n_cand: int
    k_pick: int
    dense_col: int
    dense_row: int

    def row_counts(self) -> np.ndarray:
        counts = np.full(self.q_blocks, self.k_blocks, dtype=np.int64)
        counts[: self.dense_row] = self.k_pick + (self.k_blocks - self.dense_col)
        return counts

    def row_ptr(self, heads: int) -> np.ndarray:
        counts = np.tile(self.row_counts(), heads)
        ptr = np.zeros(counts.size + 1, dtype=np.int64)
        np.cumsum(counts, out=ptr[1:])
        if ptr[-1] >= 2 ** 31:
            raise ValueError("block mask too large for int32 CSR offsets")
        return ptr.astype(np.int32)

    def nnz(self, heads: int) -> int:
        return int(self.row_counts().sum()) * heads


def topk_count(sparse_ratio: float, k_blocks: int) -> int:
    """k = max(1, int(sparsity * Kb)) in Python float arithmetic
    (attention_wan.py:248; attention_hyvideo.py:432)."""
    return max(1, int(sparse_ratio * k_blocks))


def wan_policy(layout: ScoringLayout, sparse_ratio: float) -> TopkPolicy:
    """attention_wan.py:248-253: every row keeps its top-k columns."""
    kb = layout.k_blocks
    k = topk_count(sparse_ratio, kb)
    if k > kb:
        raise RuntimeError(f"selected index k out of range (k={k}, columns={kb})")
    return TopkPolicy(layout.q_blocks, kb, layout.q_blocks, kb, k, kb, layout.q_blocks)


def hunyuan_policy(layout: ScoringLayout, sparse_ratio: float) -> TopkPolicy:
    """attention_hyvideo.py:424-501 (top-k selector): the columns from
    video_len // 128 on are kept in every video row, the video budget is
    k - text_blocks, and rows from video_len // 128 on are dense when text
    tokens exist."""
    kb = layout.k_blocks
    dense_start = layout.video_len // layout.block
    text_blocks = max(0, kb - dense_start)
    k = topk_count(sparse_ratio, kb)
    dense_row = dense_start if layout.text_len > 0 else layout.q_blocks
    if text_blocks > 0:
        budget = k - text_blocks
        if budget <= 0:
            raise AssertionError("num_video_blocks_to_select must be non-negative")
        if budget > dense_start:
            raise RuntimeError(f"selected index k out of range (k={budget}, columns={dense_start})")
        return TopkPolicy(layout.q_blocks, kb, layout.video_blocks, dense_start, budget, dense_start, dense_row)
    if k > kb:
        raise RuntimeError(f"selected index k out of range (k={k}, columns={kb})")
    return TopkPolicy(layout.q_blocks, kb, layout.video_blocks, kb, k, kb, dense_row)


def dense_policy(layout: ScoringLayout) -> TopkPolicy:
    """Every block kept (dense attention through the block-sparse kernel)."""
    return TopkPolicy(layout.q_blocks, layout.k_blocks, layout.q_blocks, 0, 0, 0, 0)


def block_flops(mask_rows: np.ndarray, seq_len: int, head_dim: int, block: int = BLOCK) -> int:
    """Exact attention FLOPs of a block mask: sum over kept (h, i, j) of
    4 * nq(i) * nk(j) * D with valid-token block sizes."""
    mask = np.asarray(mask_rows, dtype=bool)
    nblk = mask.shape[-1]
    sizes = np.full(nblk, block, dtype=np.int64)
    sizes[-1] = seq_len - block * (nblk - 1)
    per_row = (mask * sizes[None, None, :]).sum(axis=-1)  # [H, Qb] kept key tokens
    return int(4 * head_dim * (per_row * sizes[None, :]).sum())


def csr_flops(row_ptr: np.ndarray, col_idx: np.ndarray, heads: int, seq_len: int, head_dim: int,
              block: int = BLOCK) -> int:
    """block_flops for a CSR mask."""
    nblk = math.ceil(seq_len / block)
    sizes = np.full(nblk, block, dtype=np.int64)
    sizes[-1] = seq_len - block * (nblk - 1)
    row_ptr = np.asarray(row_ptr, dtype=np.int64)
    col = np.asarray(col_idx, dtype=np.int64)
    cum = np.zeros(col.size + 1, dtype=np.int64)
    np.cumsum(sizes[col], out=cum[1:])
    key_tok = (cum[row_ptr[1:]] - cum[row_ptr[:-1]]).reshape(heads, nblk)
    return int(4 * head_dim * (key_tok * sizes[None, :]).sum())

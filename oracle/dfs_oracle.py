"""CPU restatement of DFSAttn's sparse-attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this module: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or the timed CPU baseline),
never as a fallback for the HIP path.

Each function restates the reference (``codesiena/DFSattn``) at the cited
``file:line`` in plain numpy / fp32 torch on the CPU. How each is pinned
(see ``tests/test_oracle.py``):

* ``hilbert_encode`` / ``hilbert3d_perm`` (dfsattn/utils/order.py:206-258,
  numpy-hilbert-curve>=1.0.0 ``encode``, requirements.txt:19): pinned by
  closed forms (1 bit per axis = inverse Gray code of the interleaved
  coordinate bits, axis 0 most significant), the Hilbert-curve invariants
  (bijection, unit steps on full 2^b cubes, index 0 at the origin), the
  package's published usage example (2-D, 3 bits: it fixes the axis order at
  the finest level), a round trip through a separate restatement of the
  package's ``decode`` on full cubes and on 3-D 7-bit points (an encoder with
  its bit or axis loops reversed, its axes swapped, the exchange step dropped
  or the inversion on the wrong axis fails it) and an independent C
  implementation on the benchmark grids. Together these fix the package's
  convention: every plausible variant of the encoder that was tried fails one
  of them. No fixture of the package's own output exists (it is absent
  offline and the reference ships none), so that is the anchor.
* ``compute_cache_schedule`` (dfsattn/attention_wan.py:41-66): pinned by the
  reference's own known-answer test (tests/test_flashinfer64_attention.py:122-157).
* ``tile_scores`` / ``block_scores`` (attention_wan.py:157-246,
  attention_hyvideo.py:310-422), with equal or unequal query and key tiles:
  pinned by a brute-force loop restatement on tiny inputs and the invariant
  that every scored row of block scores sums to block/q_tile (softmax rows
  sum to one).
* ``mask_from_scores_*`` (attention_wan.py:248-253, attention_hyvideo.py:424-501):
  pinned against ``torch.topk`` + ``scatter_`` (the reference's own calls) on
  tie-free scores, and by policy invariants (row counts, dense text columns/rows).
* ``masked_attention`` (block_sparse_attn_func semantics,
  attention_wan.py:379-386): pinned against dense ``torch.softmax`` attention
  with an explicit token mask, and equals dense attention for an all-True mask.
  The external kernel's own rounding is parity unpinned (no fixture exists);
  the contract is the fp32 masked-dense closed form.
* ``segment_attention`` (the varlen call with cu_seqlens [0, valid, L],
  attention_hyvideo.py:1054-1082): pinned against dense attention under an
  explicit block-diagonal token mask whose blocks are counted from each
  segment's start.
* ``rmsnorm_rows`` (kernels/triton/rmsnorm.py:9-48): pinned against
  ``torch.nn.functional.rms_norm`` (the library routine) in fp32 and within
  one bf16 unit in the last place after rounding.
* ``rope_complex_pairs`` (rope_enc_complex.cuh, ops.h:207-261): pinned
  bit-exactly against the reference's own torch fallback, a complex128
  product through ``torch.view_as_complex`` (replace_wan.py:209-213), and by
  the rotation invariants (angle 0 is the identity, pair norms are kept,
  rotating by -angle undoes +angle).
* ``rope_real_pairs`` (rope_enc_txtlast.cuh; replace_hyvideo.py:271-290):
  pinned within fp32 rounding against the float64 complex rotation of the
  same angles (tables repeat each angle over a pair), and by the rotation
  invariants; ``head_rmsnorm`` reduces to ``rmsnorm_rows`` over one head.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch

BLOCK = 128


# --------------------------------------------------------------------------
# a1: Hilbert order (dfsattn/utils/order.py:206-258)
# --------------------------------------------------------------------------

def hilbert_encode(locs: np.ndarray, num_dims: int, num_bits: int) -> np.ndarray:
    """Hilbert integers of integer points ``locs[..., num_dims]``.

    Restates numpy-hilbert-curve's ``encode`` (called at order.py:250) in its
    bit-array form: big-endian coordinate bits; for each bit level (most
    significant first) and each axis, invert the lower bits of axis 0 where the
    axis bit is set, else exchange the lower bits of axis 0 and the axis
    (Skilling 2004); interleave level by level with axis 0 first; Gray-decode.
    """
    locs = np.asarray(locs, dtype=np.int64)
    if locs.shape[-1] != num_dims:
        raise ValueError("last dimension of locs must equal num_dims")
    if num_dims * num_bits > 63:
        raise ValueError("num_dims * num_bits must not exceed 63")
    flat = locs.reshape(-1, num_dims)
    shifts = np.arange(num_bits - 1, -1, -1, dtype=np.int64)
    # gray[n, dim, bit] with bit 0 the most significant.
    gray = ((flat[:, :, None] >> shifts[None, None, :]) & 1).astype(bool)
    for bit in range(num_bits):
        for dim in range(num_dims):
            mask = gray[:, dim, bit][:, None]
            gray[:, 0, bit + 1:] ^= mask
            to_flip = (~mask) & (gray[:, 0, bit + 1:] ^ gray[:, dim, bit + 1:])
            gray[:, dim, bit + 1:] ^= to_flip
            gray[:, 0, bit + 1:] ^= to_flip
    inter = np.swapaxes(gray, 1, 2).reshape(-1, num_bits * num_dims)
    binary = np.logical_xor.accumulate(inter, axis=1)
    weights = (np.uint64(1) << np.arange(inter.shape[1] - 1, -1, -1, dtype=np.uint64))
    codes = (binary.astype(np.uint64) * weights[None, :]).sum(axis=1, dtype=np.uint64)
    return codes.reshape(locs.shape[:-1])


def hilbert_decode(codes: np.ndarray, num_dims: int, num_bits: int) -> np.ndarray:
    """Integer points of Hilbert integers: numpy-hilbert-curve's ``decode``,
    restated separately from ``hilbert_encode`` in the package's own steps:
    the index bits (most significant first) Gray-encoded, split level by level
    with axis 0 first, then for each bit level (least significant first) and
    each axis (last first) the same invert/exchange of the lower bits of
    axis 0. Kept as the second half of a round trip that pins the encoder's
    loop orders and axis order (an exchange rule applied in another order, or
    left out, does not invert)."""
    codes = np.asarray(codes, dtype=np.uint64)
    flat = codes.reshape(-1)
    nb = num_dims * num_bits
    if nb > 63:
        raise ValueError("num_dims * num_bits must not exceed 63")
    shifts = np.arange(nb - 1, -1, -1, dtype=np.uint64)
    hbits = ((flat[:, None] >> shifts[None, :]) & np.uint64(1)).astype(bool)
    gray = hbits.copy()
    gray[:, 1:] ^= hbits[:, :-1]
    gray = np.swapaxes(gray.reshape(-1, num_bits, num_dims), 1, 2).copy()
    for bit in range(num_bits - 1, -1, -1):
        for dim in range(num_dims - 1, -1, -1):
            mask = gray[:, dim, bit][:, None]
            gray[:, 0, bit + 1:] ^= mask
            to_flip = (~mask) & (gray[:, 0, bit + 1:] ^ gray[:, dim, bit + 1:])
            gray[:, dim, bit + 1:] ^= to_flip
            gray[:, 0, bit + 1:] ^= to_flip
    weights = (np.int64(1) << np.arange(num_bits - 1, -1, -1, dtype=np.int64))
    locs = (gray.astype(np.int64) * weights[None, None, :]).sum(axis=-1)
    return locs.reshape(codes.shape + (num_dims,))


def hilbert3d_perm(f: int, h: int, w: int) -> np.ndarray:
    """order.py:206-258: linear indices z*h*w + y*w + x in Hilbert order, with
    coordinate columns [x, y, z] and num_bits = max(1, ceil(log2(max dim)))."""
    max_dim = max(w, h, f)
    num_bits = max(1, math.ceil(math.log2(max_dim))) if max_dim > 1 else 1
    z, y, x = np.meshgrid(np.arange(f), np.arange(h), np.arange(w), indexing="ij")
    linear = (z * (h * w) + y * w + x).reshape(-1)
    coords = np.stack([x.reshape(-1), y.reshape(-1), z.reshape(-1)], axis=1)
    codes = hilbert_encode(coords, 3, num_bits)
    order = np.argsort(codes, kind="stable")
    return linear[order].astype(np.int64)


# --------------------------------------------------------------------------
# Other token orders (dfsattn/utils/order.py:8-203, 260-436): per-token loops
# --------------------------------------------------------------------------

def _gilbert_region(x, y, ax, ay, bx, by):
    """Published recursive gilbert2d (J. Cervený), one region."""
    sgn = lambda v: (v > 0) - (v < 0)  # noqa: E731
    w, h = abs(ax + ay), abs(bx + by)
    dax, day, dbx, dby = sgn(ax), sgn(ay), sgn(bx), sgn(by)
    if h == 1:
        for _ in range(w):
            yield x, y
            x, y = x + dax, y + day
        return
    if w == 1:
        for _ in range(h):
            yield x, y
            x, y = x + dbx, y + dby
        return
    ax2, ay2, bx2, by2 = ax // 2, ay // 2, bx // 2, by // 2
    w2, h2 = abs(ax2 + ay2), abs(bx2 + by2)
    if 2 * w > 3 * h:
        if w2 % 2 and w > 2:
            ax2, ay2 = ax2 + dax, ay2 + day
        yield from _gilbert_region(x, y, ax2, ay2, bx, by)
        yield from _gilbert_region(x + ax2, y + ay2, ax - ax2, ay - ay2, bx, by)
    else:
        if h2 % 2 and h > 2:
            bx2, by2 = bx2 + dbx, by2 + dby
        yield from _gilbert_region(x, y, bx2, by2, ax2, ay2)
        yield from _gilbert_region(x + bx2, y + by2, ax, ay, bx - bx2, by - by2)
        yield from _gilbert_region(x + (ax - dax) + (bx2 - dbx), y + (ay - day) + (by2 - dby),
                                   -bx2, -by2, -(ax - ax2), -(ay - ay2))


def gilbert2d(width: int, height: int):
    """order.py:8-72: (x, y) cells along the generalised Hilbert curve."""
    if width >= height:
        return list(_gilbert_region(0, 0, width, 0, 0, height))
    return list(_gilbert_region(0, 0, 0, height, width, 0))


def hilbert_d2xy(n: int, d: int):
    """Textbook Hilbert curve on an n x n grid (n a power of two): the d-th
    cell (x, y), starting at (0, 0) and ending at (n - 1, 0)."""
    x = y = 0
    s, t = 1, d
    while s < n:
        rx = 1 & (t // 2)
        ry = 1 & (t ^ rx)
        if ry == 0:
            if rx == 1:
                x, y = s - 1 - x, s - 1 - y
            x, y = y, x
        x, y = x + s * rx, y + s * ry
        t //= 4
        s *= 2
    return x, y


def hilbert2d_perm(f: int, h: int, w: int) -> np.ndarray:
    """order.py:75-90."""
    frame = [y * w + x for x, y in gilbert2d(w, h)]
    return np.array([z * h * w + i for z in range(f) for i in frame], dtype=np.int64)


def _morton_less(a, b):
    """Morton order without building codes (T. Chan's most-significant-bit
    comparison): the coordinate whose XOR has the highest set bit decides;
    on equal highest bits the later axis wins, as it holds the higher bit of
    each interleaved group."""
    def msb_less(u, v):
        return u < v and u < (u ^ v)
    axis, top = len(a) - 1, a[-1] ^ b[-1]
    for k in range(len(a) - 2, -1, -1):
        d = a[k] ^ b[k]
        if msb_less(top, d):
            axis, top = k, d
    return (a[axis] > b[axis]) - (a[axis] < b[axis])


def morton_perm(f: int, h: int, w: int, per_frame: bool) -> np.ndarray:
    """order.py:139-203: Morton order of (x, y, z) over all tokens, or of
    (x, y) within each frame with frames in order (``per_frame``)."""
    from functools import cmp_to_key
    if per_frame:
        cells = sorted(((x, y) for y in range(h) for x in range(w)), key=cmp_to_key(_morton_less))
        return np.array([z * h * w + y * w + x for z in range(f) for x, y in cells], dtype=np.int64)
    pts = sorted(((x, y, z) for z in range(f) for y in range(h) for x in range(w)), key=cmp_to_key(_morton_less))
    return np.array([z * h * w + y * w + x for x, y, z in pts], dtype=np.int64)


def axis_order_perm(f: int, h: int, w: int, target: str) -> np.ndarray:
    """order.py:260-354: perm[target_index] = original index for the target
    axis order "hwf" (y*(w*f) + x*f + z) or "fwh" (z*(w*h) + x*h + y)."""
    perm = np.zeros(f * h * w, dtype=np.int64)
    for z in range(f):
        for y in range(h):
            for x in range(w):
                t = y * (w * f) + x * f + z if target == "hwf" else z * (w * h) + x * h + y
                perm[t] = z * h * w + y * w + x
    return perm


def block3d_perm(f: int, h: int, w: int, a: int, b: int, c: int) -> np.ndarray:
    """order.py:357-436: bricks in (z, y, x) order, tokens of a brick in
    (z, y, x) order."""
    out = []
    for bz in range(0, f, a):
        for by in range(0, h, b):
            for bx in range(0, w, c):
                for z in range(bz, min(bz + a, f)):
                    for y in range(by, min(by + b, h)):
                        for x in range(bx, min(bx + c, w)):
                            out.append(z * h * w + y * w + x)
    return np.array(out, dtype=np.int64)


# --------------------------------------------------------------------------
# a4: refresh schedule (attention_wan.py:41-66 == attention_hyvideo.py:40-65)
# --------------------------------------------------------------------------

def compute_cache_schedule(step_idx: int, skip_steps: int, cache_interval: int,
                           sparsity: float, sparsity_dcrt: float) -> Tuple[bool, float]:
    if cache_interval <= 0:
        raise ValueError("cache_interval must be greater than 0.")
    if step_idx < skip_steps:
        return False, sparsity
    raw = (step_idx - skip_steps) // cache_interval
    max_valid = max(0, math.ceil(sparsity / sparsity_dcrt) - 1) if sparsity_dcrt > 0 else raw
    idx = min(raw, max_valid)
    refresh = raw <= max_valid and (step_idx - skip_steps) % cache_interval == 0
    cur = min(1.0, max(0.0, sparsity - idx * sparsity_dcrt))
    return refresh, cur


def topk_count(sparse_ratio: float, k_blocks: int) -> int:
    """attention_wan.py:248 / attention_hyvideo.py:432."""
    return max(1, int(sparse_ratio * k_blocks))


# --------------------------------------------------------------------------
# a2/a3: permutation (attention_wan.py:113-145, attention_hyvideo.py:154-194)
# --------------------------------------------------------------------------

def full_permutation(video_perm: torch.Tensor, seq_len: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """perm = cat(video_perm, arange(video_len, seq_len)); inv[perm] = arange."""
    video_perm = torch.as_tensor(video_perm, dtype=torch.long)
    vlen = video_perm.numel()
    perm = torch.cat([video_perm, torch.arange(vlen, seq_len, dtype=torch.long)]) if seq_len > vlen else video_perm
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), dtype=torch.long)
    return perm, inv


def apply_permutation(x: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """tensor[:, :, perm, :] (attention_wan.py:134)."""
    return x[:, :, perm, :].contiguous()


# --------------------------------------------------------------------------
# a5/a6: tile scores, block scores and the top-k mask
# --------------------------------------------------------------------------

def _scoring_layout(x_perm: torch.Tensor, seq_len: int, video_len: int, block: int) -> torch.Tensor:
    """[video | zeros to a block multiple | text | zeros to ceil(L/block)*block]
    (attention_wan.py:176-189; attention_hyvideo.py:331-365)."""
    bsz, heads, _, dim = x_perm.shape
    vb = math.ceil(video_len / block)
    kb = math.ceil(seq_len / block)
    parts = [x_perm[:, :, :video_len]]
    pad = vb * block - video_len
    if pad:
        parts.append(x_perm.new_zeros(bsz, heads, pad, dim))
    if seq_len > video_len:
        parts.append(x_perm[:, :, video_len:])
    out = torch.cat(parts, dim=2)
    if out.shape[2] > kb * block:
        raise RuntimeError("scoring layout exceeds ceil(L/block) blocks; the reference's .view fails")
    if out.shape[2] < kb * block:
        out = torch.cat([out, x_perm.new_zeros(bsz, heads, kb * block - out.shape[2], dim)], dim=2)
    return out


def _check_tiles(block: int, q_tile: int, k_tile: int) -> None:
    """attention_wan.py:227-228; attention_hyvideo.py:406-407."""
    assert block % q_tile == 0, f"block_dim ({block}) must be divisible by q_tile_size ({q_tile})"
    assert block % k_tile == 0, f"block_dim ({block}) must be divisible by k_tile_size ({k_tile})"


def pooled_tiles(q_perm: torch.Tensor, k_perm: torch.Tensor, tile: int, block: int = BLOCK,
                 video_len: Optional[int] = None, k_tile: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tile means of the scoring layout: queries over the video part in
    ``tile``-token tiles, keys over everything in ``k_tile``-token tiles
    (default: ``tile``) (attention_wan.py:192-205; attention_hyvideo.py:367-381)."""
    k_tile = tile if k_tile is None else k_tile
    _check_tiles(block, tile, k_tile)
    seq_len = q_perm.shape[2]
    video_len = seq_len if video_len is None else video_len
    qs = _scoring_layout(q_perm.float(), seq_len, video_len, block)
    ks = _scoring_layout(k_perm.float(), seq_len, video_len, block)
    bsz, heads, _, dim = qs.shape
    vpad_len = math.ceil(video_len / block) * block
    qt = qs[:, :, :vpad_len].reshape(bsz, heads, vpad_len // tile, tile, dim).mean(dim=3)
    kt = ks.reshape(bsz, heads, ks.shape[2] // k_tile, k_tile, dim).mean(dim=3)
    return qt, kt


def tile_scores(q_perm: torch.Tensor, k_perm: torch.Tensor, tile: int, block: int = BLOCK,
                video_len: Optional[int] = None, k_tile: Optional[int] = None) -> torch.Tensor:
    """fp32 softmax(Qt Kt^T / sqrt(D)) over all key tiles, [B, H, Qt, Kt]
    (attention_wan.py:207; attention_hyvideo.py:383)."""
    qt, kt = pooled_tiles(q_perm, k_perm, tile, block, video_len, k_tile)
    scale = 1.0 / math.sqrt(q_perm.shape[-1])
    return (qt @ kt.transpose(-2, -1) * scale).softmax(dim=-1)


def block_scores(q_perm: torch.Tensor, k_perm: torch.Tensor, tile: int, block: int = BLOCK,
                 video_len: Optional[int] = None, head_chunk: int = 4, k_tile: Optional[int] = None) -> torch.Tensor:
    """Block sums of tile probabilities, fp32 [H, Vb, Kb]: the sum over a
    block's block/tile query tiles and block/k_tile key tiles
    (attention_wan.py:243-246; attention_hyvideo.py:419-422), computed a few
    heads at a time to bound memory at the full configurations."""
    heads = q_perm.shape[1]
    k_tile = tile if k_tile is None else k_tile
    tpq, tpk = block // tile, block // k_tile
    outs = []
    for h0 in range(0, heads, head_chunk):
        ts = tile_scores(q_perm[:, h0:h0 + head_chunk], k_perm[:, h0:h0 + head_chunk], tile, block, video_len,
                         k_tile)
        b, hh, qt, kt = ts.shape
        outs.append(ts.view(b, hh, qt // tpq, tpq, kt // tpk, tpk).sum(dim=(3, 5))[0])
    return torch.cat(outs, dim=0)


def select_topk(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Bool mask of the k largest entries per row under the total order
    (score descending, column ascending)."""
    s = scores.detach().cpu().double().numpy()
    rows = s.reshape(-1, s.shape[-1])
    order = np.lexsort((np.broadcast_to(np.arange(rows.shape[1]), rows.shape), -rows), axis=1)
    mask = np.zeros(rows.shape, dtype=bool)
    np.put_along_axis(mask, order[:, :k], True, axis=1)
    return torch.from_numpy(mask.reshape(s.shape))


def boundary_ties(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Rows whose k-th and (k+1)-th largest scores are equal (where torch.topk's
    choice is implementation-defined)."""
    if k >= scores.shape[-1]:
        return torch.zeros(scores.shape[:-1], dtype=torch.bool)
    srt = torch.sort(scores.double(), dim=-1, descending=True).values
    return srt[..., k - 1] == srt[..., k]


def mask_from_scores_wan(scores: torch.Tensor, sparse_ratio: float) -> torch.Tensor:
    """attention_wan.py:248-253: k = max(1, int(s * Kb)); top-k per row."""
    return select_topk(scores, topk_count(sparse_ratio, scores.shape[-1]))


def mask_from_scores_hunyuan(scores: torch.Tensor, sparse_ratio: float, seq_len: int,
                             video_len: int, block: int = BLOCK) -> torch.Tensor:
    """attention_hyvideo.py:424-501 (top-k branch): the video budget
    k - text_blocks is chosen among the first video_len // block columns, the
    remaining columns are kept, and rows >= video_len // block are dense when
    text tokens exist."""
    heads, vb, kb = scores.shape
    qb = kb
    dense_start = video_len // block
    text_blocks = max(0, kb - dense_start)
    topk = topk_count(sparse_ratio, kb)
    video_mask = torch.zeros(heads, vb, kb, dtype=torch.bool)
    if text_blocks > 0:
        budget = topk - text_blocks
        if budget <= 0:
            raise AssertionError("num_video_blocks_to_select must be non-negative")
        if budget > dense_start:
            raise RuntimeError("selected index k out of range")
        video_mask[..., :dense_start] = select_topk(scores[..., :dense_start], budget)
        video_mask[..., dense_start:] = True
    else:
        video_mask = select_topk(scores, topk)
    mask = torch.zeros(heads, qb, kb, dtype=torch.bool)
    mask[:, :vb] = video_mask
    if seq_len > video_len:
        mask[:, dense_start:] = True
    return mask


def mask_from_scores_torch(scores: torch.Tensor, k: int) -> torch.Tensor:
    """The reference's literal calls: torch.topk + scatter_ (attention_wan.py:249-253)."""
    _, idx = torch.topk(scores, k=k, dim=-1)
    return torch.zeros_like(scores, dtype=torch.bool).scatter_(-1, idx, True)


# --------------------------------------------------------------------------
# a8: block-masked attention (block_sparse_attn_func semantics)
# --------------------------------------------------------------------------

def masked_attention(q_perm: torch.Tensor, k_perm: torch.Tensor, v_perm: torch.Tensor,
                     mask: torch.Tensor, block: int = BLOCK, scale: Optional[float] = None,
                     heads: Optional[list] = None, q_blocks: Optional[list] = None) -> torch.Tensor:
    """fp32 softmax(Q K^T * scale) V where query block i sees the key blocks
    kept in mask[h, i] (tokens and mask columns past L excluded). Returns [B, H, L, D] fp32 with
    rows outside the requested heads / query blocks left at zero.
    Rows with no kept block are zero."""
    q = q_perm.float()
    k = k_perm.float()
    v = v_perm.float()
    _, n_heads, seq_len, dim = q.shape
    scale = 1.0 / math.sqrt(dim) if scale is None else scale
    out = torch.zeros_like(q)
    n_blocks = math.ceil(seq_len / block)
    heads = range(n_heads) if heads is None else heads
    for h in heads:
        for i in (range(n_blocks) if q_blocks is None else q_blocks):
            cols = torch.nonzero(mask[h, i, :n_blocks]).flatten().tolist()
            if not cols:
                continue
            tok = torch.cat([torch.arange(c * block, min((c + 1) * block, seq_len)) for c in cols])
            qi = q[0, h, i * block:(i + 1) * block]
            s = (qi @ k[0, h, tok].T) * scale
            p = torch.softmax(s, dim=-1)
            out[0, h, i * block:(i + 1) * block] = p @ v[0, h, tok]
    return out


def varlen_attention(q_perm: torch.Tensor, k_perm: torch.Tensor, v_perm: torch.Tensor, mask: torch.Tensor,
                     cu_q, cu_k, block: int = BLOCK, scale: Optional[float] = None) -> torch.Tensor:
    """block_sparse_attn_func's varlen semantics (attention_wan.py:359-386,
    attention_hyvideo.py:1054-1082): sequence i's queries [cq[i], cq[i+1])
    attend its keys [ck[i], ck[i+1]) under mask[h, a, b], where a and b count
    128-token blocks from the sequence's own first query and first key (the
    reference repeats ``base_blockmask`` per sequence). Rows in no query
    sequence, and sequences without keys, give zero."""
    q, k, v = q_perm.float(), k_perm.float(), v_perm.float()
    _, n_heads, _, dim = q.shape
    scale = 1.0 / math.sqrt(dim) if scale is None else scale
    out = torch.zeros_like(q)
    bq = [int(x) for x in cu_q]
    bk = [int(x) for x in cu_k]
    for (q0, q1), (k0, k1) in zip(zip(bq, bq[1:]), zip(bk, bk[1:])):
        nq, nk = q1 - q0, k1 - k0
        if nq <= 0 or nk <= 0:
            continue
        nkb = math.ceil(nk / block)
        for h in range(n_heads):
            for a in range(math.ceil(nq / block)):
                cols = torch.nonzero(mask[h, a, :nkb]).flatten().tolist()
                if not cols:
                    continue
                tok = torch.cat([torch.arange(k0 + c * block, min(k0 + (c + 1) * block, k1)) for c in cols])
                rows = slice(q0 + a * block, min(q0 + (a + 1) * block, q1))
                p = torch.softmax((q[0, h, rows] @ k[0, h, tok].T) * scale, dim=-1)
                out[0, h, rows] = p @ v[0, h, tok]
    return out


def segment_attention(q_perm: torch.Tensor, k_perm: torch.Tensor, v_perm: torch.Tensor,
                      mask: torch.Tensor, cu_seqlens, block: int = BLOCK) -> torch.Tensor:
    """Varlen block-masked attention (attention_hyvideo.py:1054-1082): each
    segment [cu[i], cu[i+1]) attends only within itself, under the same block
    mask indexed from the segment's own first token (the reference repeats
    ``base_blockmask`` per sequence)."""
    out = torch.zeros_like(q_perm, dtype=torch.float32)
    bounds = [int(x) for x in cu_seqlens]
    for start, end in zip(bounds, bounds[1:]):
        if end > start:
            sl = slice(start, end)
            out[:, :, sl] = masked_attention(q_perm[:, :, sl], k_perm[:, :, sl], v_perm[:, :, sl], mask, block)
    return out


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    token_mask: Optional[torch.Tensor] = None, scale: Optional[float] = None) -> torch.Tensor:
    """fp32 attention with an optional [H, L, L] bool token mask (closed form)."""
    q, k, v = q.float(), k.float(), v.float()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    s = (q @ k.transpose(-2, -1)) * scale
    if token_mask is not None:
        s = s.masked_fill(~token_mask, float("-inf"))
    return torch.softmax(s, dim=-1) @ v


def expand_block_mask(mask: torch.Tensor, seq_len: int, block: int = BLOCK) -> torch.Tensor:
    """[H, Qb, Kb] block mask -> [H, L, L] token mask."""
    tok = mask.repeat_interleave(block, dim=1).repeat_interleave(block, dim=2)
    return tok[:, :seq_len, :seq_len]


# --------------------------------------------------------------------------
# Whole call (attention_wan.py:394-547 native path; attention_hyvideo.py:1090-1286)
# --------------------------------------------------------------------------

def dfs_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, video_perm: torch.Tensor,
                            sparse_ratio: float, tile: int, block: int = BLOCK,
                            video_len: Optional[int] = None, valid: Optional[int] = None,
                            k_tile: Optional[int] = None):
    """Permute, score, select, attend, unpermute. Returns (out fp32 [1,H,L,D]
    in the original order, bool mask [H,Qb,Kb], fp32 block scores). With
    ``valid`` < L (cu_seqlens [0, valid, L]) the mask is still selected over
    the whole sequence and the attention runs per segment."""
    seq_len = q.shape[2]
    perm, inv = full_permutation(video_perm, seq_len)
    qp, kp, vp = apply_permutation(q, perm), apply_permutation(k, perm), apply_permutation(v, perm)
    scores = block_scores(qp, kp, tile, block, video_len, k_tile=k_tile)
    if video_len is None:
        mask = mask_from_scores_wan(scores, sparse_ratio)
    else:
        mask = mask_from_scores_hunyuan(scores, sparse_ratio, seq_len, video_len, block)
    if valid is None or valid == seq_len:
        out = masked_attention(qp, kp, vp, mask, block)
    else:
        out = segment_attention(qp, kp, vp, mask, [0, valid, seq_len], block)
    return out[:, :, inv, :], mask, scores


# --------------------------------------------------------------------------
# DiT attention inputs: QK RMSNorm, complex RoPE, head split
# (kernels/triton/rmsnorm.py:9-48; kernels/include/rope/rope_enc_complex.cuh;
# replace_wan.py:159-218)
# --------------------------------------------------------------------------

def rmsnorm_rows(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last axis as the reference's fused kernel computes it
    (rmsnorm.py:28-44): x in fp32, var = sum(x*x)/N, rstd = 1/sqrt(var+eps),
    y = (x*rstd)*w in fp32, stored in x's dtype."""
    xf = x.float()
    var = (xf * xf).sum(-1, keepdim=True) / xf.shape[-1]
    rstd = 1.0 / torch.sqrt(var + eps)
    return ((xf * rstd) * weight.float()).to(x.dtype)


def rope_complex_pairs(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotation of the (even, odd) channel pairs of x [..., L, D] by fp32
    (cos, sin) [L, D/2] (rope_enc_complex.cuh: out[2i] = x[2i] c - x[2i+1] s,
    out[2i+1] = x[2i+1] c + x[2i] s in float64), rounded float64 -> float32 ->
    x's dtype."""
    xd = x.double()
    c, s = cos.double(), sin.double()
    xe, xo = xd[..., 0::2], xd[..., 1::2]
    out = torch.stack([xe * c - xo * s, xo * c + xe * s], dim=-1).flatten(-2)
    return out.float().to(x.dtype)


def norm_rope_heads(x: torch.Tensor, heads: int, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                    cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                    rope_skip: int = 0) -> torch.Tensor:
    """[B, L, H*D] -> [B, H, L, D]: RMSNorm over all channels (if weight),
    head split (replace_wan.py:181-183), RoPE of tokens l >= rope_skip by
    row l - rope_skip of the tables (if cos)."""
    y = rmsnorm_rows(x, weight, eps) if weight is not None else x
    y = y.unflatten(-1, (heads, -1)).transpose(1, 2).contiguous()
    if cos is not None:
        y = y.clone()
        y[:, :, rope_skip:] = rope_complex_pairs(y[:, :, rope_skip:], cos, sin)
    return y


def head_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm of each head's D channels (last axis) as the reference's
    narrow RMSNorm kernel (kernels/include/norm/narrow_rms_norm.cuh): fp32
    sum of squares, (x * rstd) * w, stored in x's dtype."""
    return rmsnorm_rows(x, weight, eps)


def rope_real_pairs(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Real RoPE of adjacent channel pairs with fp32 tables [L, D]
    (rope_enc_txtlast.cuh; the torch fallback at replace_hyvideo.py:271-290):
    out[2i] = x[2i] cos[2i] - x[2i+1] sin[2i], out[2i+1] = x[2i+1] cos[2i+1] +
    x[2i] sin[2i+1], every product and sum rounded in fp32."""
    xf = x.float()
    xe, xo = xf[..., 0::2], xf[..., 1::2]
    ce, co = cos[..., 0::2], cos[..., 1::2]
    se, so = sin[..., 0::2], sin[..., 1::2]
    out = torch.stack([xe * ce + (-xo) * se, xo * co + xe * so], dim=-1).flatten(-2)
    return out.to(x.dtype)


def head_norm_rope_heads(x: torch.Tensor, heads: int, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
                         cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                         rope_rows: Optional[int] = None) -> torch.Tensor:
    """[B, L, H*D] -> [B, H, L, D]: head split, per-head RMSNorm (if weight),
    real RoPE of tokens l < rope_rows (if cos; default all) by table row l."""
    y = x.unflatten(-1, (heads, -1)).transpose(1, 2).contiguous()
    if weight is not None:
        y = head_rmsnorm(y, weight, eps)
    if cos is not None:
        rows = y.shape[2] if rope_rows is None else rope_rows
        y = y.clone()
        y[:, :, :rows] = rope_real_pairs(y[:, :, :rows], cos, sin)
    return y

"""Token orders of a video latent grid (dfsattn/utils/order.py).

Every ``*_perm`` function returns a LongTensor ``perm`` of length f*h*w over
the row-major linear index ``z*h*w + y*w + x`` (z frame, y row, x column):
``tokens[perm]`` lists the tokens in the new order, the form the processors
take as ``video_perm``. ``hilbert3d_perm`` (the default order) runs in the
native library; the others are host-side numpy, built once per process.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np
import torch


def _as_perm(idx: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(idx, dtype=np.int64)).to(device)


def _grid(f: int, h: int, w: int):
    """(z, y, x) coordinate arrays in row-major linear order."""
    z, y, x = np.meshgrid(np.arange(f, dtype=np.int64), np.arange(h, dtype=np.int64),
                          np.arange(w, dtype=np.int64), indexing="ij")
    return z.ravel(), y.ravel(), x.ravel()


# --------------------------------------------------------------------------
# 3D Hilbert curve (order.py:206-258)
# --------------------------------------------------------------------------

def hilbert3d_perm(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """Tokens along the 3D Hilbert curve of axes (x, y, z) with
    ceil(log2(max(f, h, w))) bits per axis (order.py:206-258)."""
    from ..ops import hilbert3d_perm as _perm

    return _perm(int(f), int(h), int(w)).to(device)


# --------------------------------------------------------------------------
# Generalised 2D Hilbert curve per frame (order.py:8-90)
# --------------------------------------------------------------------------

def _sgn(v: int) -> int:
    return (v > 0) - (v < 0)


def gilbert2d_fast(width: int, height: int) -> List[Tuple[int, int]]:
    """(x, y) cells of a width x height rectangle along the generalised
    Hilbert ("gilbert") curve of J. Cervený: the curve starts at (0, 0) and
    runs along the longer side, and is the classic Hilbert curve on
    2^n x 2^n squares (order.py:8-72). Each region is (origin, major axis
    vector a, minor axis vector b); regions are split in two along a when it
    is much longer than b, else in three (b-half, the rest, the way back).
    Iterative: a work stack holds the pending regions, last-pushed first."""
    out: List[Tuple[int, int]] = []
    work = [(0, 0, width, 0, 0, height) if width >= height else (0, 0, 0, height, width, 0)]
    while work:
        x, y, ax, ay, bx, by = work.pop()
        n_major, n_minor = abs(ax + ay), abs(bx + by)
        ux, uy = _sgn(ax), _sgn(ay)
        vx, vy = _sgn(bx), _sgn(by)
        if n_minor == 1 or n_major == 1:
            step_x, step_y, n = (ux, uy, n_major) if n_minor == 1 else (vx, vy, n_minor)
            out.extend((x + i * step_x, y + i * step_y) for i in range(n))
            continue
        ax2, ay2, bx2, by2 = ax // 2, ay // 2, bx // 2, by // 2  # floor division, as the curve needs
        if 2 * n_major > 3 * n_minor:
            if abs(ax2 + ay2) % 2 and n_major > 2:
                ax2, ay2 = ax2 + ux, ay2 + uy
            regions = [(x, y, ax2, ay2, bx, by),
                       (x + ax2, y + ay2, ax - ax2, ay - ay2, bx, by)]
        else:
            if abs(bx2 + by2) % 2 and n_minor > 2:
                bx2, by2 = bx2 + vx, by2 + vy
            regions = [(x, y, bx2, by2, ax2, ay2),
                       (x + bx2, y + by2, ax, ay, bx - bx2, by - by2),
                       (x + (ax - ux) + (bx2 - vx), y + (ay - uy) + (by2 - vy),
                        -bx2, -by2, -(ax - ax2), -(ay - ay2))]
        work.extend(reversed(regions))
    return out


def hilbert2d_perm(f: int, h: int, w: int, device: str = "cpu") -> torch.Tensor:
    """Each frame along the gilbert curve of its w x h cells, frames in
    order (order.py:75-90)."""
    cells = np.asarray(gilbert2d_fast(w, h), dtype=np.int64).reshape(-1, 2)
    frame = cells[:, 1] * w + cells[:, 0]
    return _as_perm((np.arange(f, dtype=np.int64)[:, None] * (h * w) + frame[None, :]).ravel(), device)


# --------------------------------------------------------------------------
# Morton (Z-order) codes (order.py:93-203)
# --------------------------------------------------------------------------

def _spread(n: torch.Tensor, bits: int, stride: int) -> torch.Tensor:
    """Bit i of the low ``bits`` bits of n moved to bit i*stride."""
    n = n.to(torch.long)
    out = torch.zeros_like(n)
    for i in range(bits):
        out |= ((n >> i) & 1) << (i * stride)
    return out


def part1by2_tensor(n: torch.Tensor) -> torch.Tensor:
    """Low 21 bits of each value with two zero bits after each (order.py:93-106)."""
    return _spread(n, 21, 3)


def part1by1_tensor(n: torch.Tensor) -> torch.Tensor:
    """Low 32 bits of each value with one zero bit after each (order.py:109-121)."""
    return _spread(n, 32, 2)


def morton3D_tensor(x: torch.Tensor, y: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    """Interleaved code with x in the lowest bit of each triple (order.py:124-128)."""
    return part1by2_tensor(x) | (part1by2_tensor(y) << 1) | (part1by2_tensor(z) << 2)


def morton2D_tensor(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Interleaved code with x in the lowest bit of each pair (order.py:131-136)."""
    return part1by1_tensor(x) | (part1by1_tensor(y) << 1)


def _sorted_by(codes: torch.Tensor, linear: torch.Tensor) -> torch.Tensor:
    # codes are unique, so any sort gives the one order
    return linear[torch.argsort(codes)]


def morton2d_perm(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """Each frame in 2D Morton order of (x, y), frames in order (order.py:139-172)."""
    _, y, x = (torch.from_numpy(a) for a in _grid(1, h, w))
    frame = _sorted_by(morton2D_tensor(x, y), y * w + x)
    return (torch.arange(f, dtype=torch.long)[:, None] * (h * w) + frame[None, :]).reshape(-1).to(device)


def morton3d_perm(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """All tokens in 3D Morton order of (x, y, z) (order.py:175-203)."""
    z, y, x = (torch.from_numpy(a) for a in _grid(f, h, w))
    return _sorted_by(morton3D_tensor(x, y, z), torch.arange(f * h * w, dtype=torch.long)).to(device)


# --------------------------------------------------------------------------
# Axis transposes and blocks (order.py:260-436)
# --------------------------------------------------------------------------

def hwf(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """(f, h, w) -> (h, w, f) order: every frame of a pixel together
    (order.py:260-306). Equals the index grid transposed."""
    return _as_perm(np.arange(f * h * w, dtype=np.int64).reshape(f, h, w).transpose(1, 2, 0).ravel(), device)


def fwh(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """(f, h, w) -> (f, w, h) order: each frame column by column
    (order.py:309-354)."""
    return _as_perm(np.arange(f * h * w, dtype=np.int64).reshape(f, h, w).transpose(0, 2, 1).ravel(), device)


def block3d_perm(f: int, h: int, w: int, a: int, b: int, c: int, device="cpu") -> torch.Tensor:
    """(a, b, c) bricks in (frame, row, column) order, each brick's tokens
    in (frame, row, column) order; edge bricks are partial (order.py:357-436)."""
    z, y, x = _grid(f, h, w)
    # np.lexsort sorts by the last key first
    order = np.lexsort((x % c, y % b, z % a, x // c, y // b, z // a))
    return _as_perm(order, device)


# --------------------------------------------------------------------------
# Driver dispatch (wan21_t2v_inference.py:133-144, hyvideo_t2v_inference.py:243-254)
# --------------------------------------------------------------------------

ORDERS = ("org", "morton", "blk", "hwf", "fwh", "hilbert3d", "hilbert2d")


def video_perm_for(order: str, f: int, h: int, w: int) -> Optional[torch.Tensor]:
    """The ``video_perm`` the reference drivers build for ``--order``:
    None (original order) for "org", 4x4x4 bricks for "blk"."""
    if order == "org":
        return None
    if order == "morton":
        return morton3d_perm(f, h, w)
    if order == "blk":
        return block3d_perm(f, h, w, a=4, b=4, c=4)
    if order == "hwf":
        return hwf(f, h, w)
    if order == "fwh":
        return fwh(f, h, w)
    if order == "hilbert3d":
        return hilbert3d_perm(f, h, w)
    if order == "hilbert2d":
        return hilbert2d_perm(f, h, w)
    raise ValueError(f"unknown order {order!r}; expected one of {ORDERS}")

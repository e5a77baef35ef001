"""Token orders (dfsattn/utils/order.py). Only the order the hot path uses,
``hilbert3d``, is provided; it is computed by the library's host code."""
from __future__ import annotations

import torch


def hilbert3d_perm(f: int, h: int, w: int, device="cpu") -> torch.Tensor:
    """LongTensor of length f*h*w: the linear indices z*h*w + y*w + x in 3D
    Hilbert-curve order (dfsattn/utils/order.py:206-258). ``tensor[perm]``
    rearranges tokens along the curve."""
    from ..ops import hilbert3d_perm as _perm

    return _perm(int(f), int(h), int(w)).to(device)

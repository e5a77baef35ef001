"""Synthetic workloads of the benchmark configurations (no datasets offline).

Per head, Q and K share one 3D Gaussian-smoothed N(0, 1) field over the
(F, H, W) latent grid (sigma = 2 tokens, separable, truncated at 3 sigma, zero
boundary, rescaled to unit std), each with its own iid N(0, noise_std) noise,
then RMS-normalised over head_dim; V is iid N(0, 1). Text tokens (HunyuanVideo)
are iid N(0, 1), RMS-normalised for Q and K, appended after the video. Sharing
the field between Q and K gives attention the spatial locality that makes
block selection meaningful. Inputs are generated in the original (f, h, w)
token order.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch


@dataclass(frozen=True)
class DfsConfig:
    name: str
    grid: Tuple[int, int, int]  # (F, H, W) latent grid
    heads: int
    head_dim: int
    dtype: torch.dtype
    text_len: int = 0
    tile: int = 16
    block: int = 128
    sparsity: float = 0.3
    seed: int = 0

    @property
    def video_len(self) -> int:
        f, h, w = self.grid
        return f * h * w

    @property
    def seq_len(self) -> int:
        return self.video_len + self.text_len


CONFIGS = {
    0: DfsConfig("cfg0-cpu-plumbing", (4, 16, 16), 2, 64, torch.float32, seed=0),
    1: DfsConfig("cfg1-wan-75.6k", (21, 45, 80), 40, 128, torch.bfloat16, seed=1),
    2: DfsConfig("cfg2-hunyuan-118.8k+256", (33, 45, 80), 24, 128, torch.bfloat16, text_len=256, seed=2),
}


def _gauss_kernel(sigma: float) -> torch.Tensor:
    r = int(math.ceil(3 * sigma))
    x = torch.arange(-r, r + 1, dtype=torch.float32)
    k = torch.exp(-0.5 * (x / sigma) ** 2)
    return k / k.sum()


def _smooth_axis(x: torch.Tensor, kern: torch.Tensor, dim: int) -> torch.Tensor:
    """Zero-boundary 'same' convolution along ``dim`` as a product with the
    banded (symmetric) Toeplitz matrix of the kernel."""
    n = x.shape[dim]
    r = kern.numel() // 2
    idx = torch.arange(n)
    off = idx[None, :] - idx[:, None]
    band = torch.where(off.abs() <= r, kern[(off + r).clamp(0, 2 * r)], torch.zeros(()))
    return (x.movedim(dim, -1) @ band.to(x.device)).movedim(-1, dim)


def smoothed_field(grid: Tuple[int, int, int], heads: int, dim: int, sigma: float,
                   gen: torch.Generator, device) -> torch.Tensor:
    """[heads, F*H*W, dim] unit-std Gaussian-smoothed N(0, 1) field."""
    f, h, w = grid
    x = torch.randn((heads, dim, f, h, w), generator=gen, device=device, dtype=torch.float32)
    kern = _gauss_kernel(sigma)
    for axis in (2, 3, 4):
        x = _smooth_axis(x, kern, axis)
    x = x / x.std()
    return x.reshape(heads, dim, f * h * w).transpose(1, 2).contiguous()


def rms_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)


def synth_qkv(cfg: DfsConfig, device="cpu", dtype: Optional[torch.dtype] = None, seed: Optional[int] = None,
              noise_std: float = 0.5, sigma: float = 2.0, independent_keys: bool = False):
    """(q, k, v) as [1, H, L, D] tensors of ``dtype`` (default cfg.dtype).

    Q and K share one smoothed field, so a query block scores highest on the
    key blocks near it in the video (a local mask, as in real video DiTs).
    With ``independent_keys`` K gets a field of its own: block scores then
    carry no locality and the top-k mask spreads over the whole row at the
    same density."""
    gen = torch.Generator(device=device)
    gen.manual_seed(cfg.seed if seed is None else seed)
    dtype = dtype or cfg.dtype
    field = smoothed_field(cfg.grid, cfg.heads, cfg.head_dim, sigma, gen, device)
    shape = field.shape
    q = rms_norm(field + noise_std * torch.randn(shape, generator=gen, device=device))
    if independent_keys:
        field = smoothed_field(cfg.grid, cfg.heads, cfg.head_dim, sigma, gen, device)
    k = rms_norm(field + noise_std * torch.randn(shape, generator=gen, device=device))
    del field
    if cfg.text_len:
        tshape = (cfg.heads, cfg.text_len, cfg.head_dim)
        q = torch.cat([q, rms_norm(torch.randn(tshape, generator=gen, device=device))], dim=1)
        k = torch.cat([k, rms_norm(torch.randn(tshape, generator=gen, device=device))], dim=1)
    v = torch.randn((cfg.heads, cfg.seq_len, cfg.head_dim), generator=gen, device=device)
    return tuple(t.unsqueeze(0).to(dtype).contiguous() for t in (q, k, v))


def drift(x: torch.Tensor, std: float, gen: torch.Generator) -> torch.Tensor:
    """x + N(0, std) (the mask-cache regime's step-to-step evolution)."""
    return (x.float() + std * torch.randn(x.shape, generator=gen, device=x.device)).to(x.dtype)

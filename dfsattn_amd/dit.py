"""Wan-style DiT denoising step on this library's kernels (the end-to-end
harness around the DFS path).

The transformer follows the structure of the Wan 2.1 text-to-video DiT that
the reference's Wan driver loads through diffusers (wan21_t2v_inference.py,
processors installed at :150-173): patch embedding, timestep and text
conditioning, N blocks of [adaLN-modulated self-attention with QK-RMSNorm
across heads and 3D complex RoPE, cross-attention to the text context, GELU
(tanh) FFN], adaLN output head. Its attention modules expose the members the
reference's processors use (``to_q``, ``to_k``, ``to_v``, ``norm_q``,
``norm_k``, ``to_out``, ``heads``), so ``Wan_DFSAttn_Processor2_0`` drives
them exactly as it drives diffusers' ``Attention``.

Weights are random (N(0, init_std), norms at one): there is no checkpoint
offline. The GEMMs and layer norms are torch (hipBLASLt); QK-norm + RoPE +
head split and the attention run in this library's HIP kernels through the
processor.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class DiTConfig:
    name: str
    layers: int = 40
    dim: int = 5120
    heads: int = 40
    ffn_dim: int = 13824
    grid: Tuple[int, int, int] = (21, 45, 80)  # latent tokens (F, H, W) after patching
    in_channels: int = 16
    patch: Tuple[int, int, int] = (1, 2, 2)
    text_len: int = 512
    text_dim: int = 4096
    freq_dim: int = 256
    eps: float = 1e-6
    init_std: float = 0.02
    theta: float = 10000.0
    seed: int = 4

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def seq_len(self) -> int:
        f, h, w = self.grid
        return f * h * w

    @property
    def latent_shape(self) -> Tuple[int, int, int, int, int]:
        f, h, w = self.grid
        pf, ph, pw = self.patch
        return (1, self.in_channels, f * pf, h * ph, w * pw)

    def params(self) -> int:
        """Parameter count of the transformer."""
        d, p_in = self.dim, self.in_channels * math.prod(self.patch)
        block = 8 * (d * d + d) + 2 * (d * self.ffn_dim) + self.ffn_dim + d + 4 * d + 2 * d + 6 * d
        head = p_in * d + d + d * p_in + p_in + 2 * d
        cond = (self.text_dim * d + d + d * d + d) + (self.freq_dim * d + d + d * d + d) + (d * 6 * d + 6 * d)
        return self.layers * block + head + cond


DIT_CONFIGS = {
    # the benchmark configuration: 40 Wan 14B-sized blocks at 21x45x80 tokens
    "cfg4": DiTConfig("cfg4-wan-dit-40x5120"),
    # a small model of the same structure for tests
    "tiny": DiTConfig("tiny-dit", layers=2, dim=256, heads=2, ffn_dim=512, grid=(4, 16, 16), text_len=16,
                      text_dim=64, freq_dim=32),
}


# --------------------------------------------------------------------------
# 3D complex RoPE frequencies (Wan: head_dim split into t, h, w parts)
# --------------------------------------------------------------------------

def _rope_1d(dim: int, n: int, theta: float) -> torch.Tensor:
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
    angles = torch.outer(torch.arange(n, dtype=torch.float64), freqs)
    return torch.polar(torch.ones_like(angles), angles)


def wan_rope_freqs(grid: Tuple[int, int, int], head_dim: int, theta: float = 10000.0) -> torch.Tensor:
    """complex128 [1, 1, F*H*W, head_dim/2]: the h and w parts get
    2*(head_dim//6) channels each, the frame part the rest; token (f, h, w)
    in row-major order takes the frame, row and column frequencies of its
    coordinates."""
    f, h, w = grid
    hw_dim = 2 * (head_dim // 6)
    t_dim = head_dim - 2 * hw_dim
    ft, fh, fw = _rope_1d(t_dim, f, theta), _rope_1d(hw_dim, h, theta), _rope_1d(hw_dim, w, theta)
    out = torch.cat([ft[:, None, None, :].expand(f, h, w, -1),
                     fh[None, :, None, :].expand(f, h, w, -1),
                     fw[None, None, :, :].expand(f, h, w, -1)], dim=-1)
    return out.reshape(1, 1, f * h * w, -1)


def timestep_embedding(t: torch.Tensor, dim: int) -> torch.Tensor:
    """Sinusoidal embedding [B, dim], cosines first."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    arg = t.float()[:, None] * freqs[None, :]
    return torch.cat([torch.cos(arg), torch.sin(arg)], dim=-1)


# --------------------------------------------------------------------------
# Modules
# --------------------------------------------------------------------------

class FP32LayerNorm(nn.LayerNorm):
    """LayerNorm evaluated in float32, returned in the input dtype."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self.weight.float() if self.weight is not None else None
        b = self.bias.float() if self.bias is not None else None
        return F.layer_norm(x.float(), self.normalized_shape, w, b, self.eps).to(x.dtype)


class DiTAttention(nn.Module):
    """Projections and QK-RMSNorm (over all heads) of one attention layer; the
    attention itself is the installed processor's."""

    def __init__(self, dim: int, heads: int, eps: float, processor=None, **fk):
        super().__init__()
        self.heads = heads
        self.to_q = nn.Linear(dim, dim, **fk)
        self.to_k = nn.Linear(dim, dim, **fk)
        self.to_v = nn.Linear(dim, dim, **fk)
        self.norm_q = nn.RMSNorm(dim, eps=eps, **fk)
        self.norm_k = nn.RMSNorm(dim, eps=eps, **fk)
        self.to_out = nn.ModuleList([nn.Linear(dim, dim, **fk), nn.Dropout(0.0)])
        self.add_k_proj = self.add_v_proj = self.norm_added_k = None
        self.processor = processor

    def set_processor(self, processor) -> None:
        self.processor = processor

    def get_processor(self):
        return self.processor

    def forward(self, hidden_states, encoder_hidden_states=None, attention_mask=None, rotary_emb=None):
        return self.processor(self, hidden_states, encoder_hidden_states, attention_mask, rotary_emb)


class DiTBlock(nn.Module):
    def __init__(self, cfg: DiTConfig, **fk):
        super().__init__()
        d = cfg.dim
        f32 = {**fk, "dtype": torch.float32}
        self.norm1 = FP32LayerNorm(d, cfg.eps, elementwise_affine=False, **f32)
        self.attn1 = DiTAttention(d, cfg.heads, cfg.eps, **fk)
        self.norm2 = FP32LayerNorm(d, cfg.eps, elementwise_affine=True, **f32)
        self.attn2 = DiTAttention(d, cfg.heads, cfg.eps, **fk)
        self.ffn = nn.Sequential(nn.Linear(d, cfg.ffn_dim, **fk), nn.GELU(approximate="tanh"),
                                 nn.Linear(cfg.ffn_dim, d, **fk))
        self.norm3 = FP32LayerNorm(d, cfg.eps, elementwise_affine=False, **f32)
        self.scale_shift_table = nn.Parameter(torch.zeros(1, 6, d, **f32))

    # On the GPU the layer norms with their modulation and the gated residuals
    # run as one fused pass each (dfs_adaln_modulate, dfs_gated_residual)
    # instead of torch's chain of dtype copies and broadcast ops, and the FFN's
    # GELU runs in the first GEMM's epilogue (hipBLASLt, through torch's
    # _addmm_activation: 8.2 -> 7.5 ms per call at 75,600 x 5,120 x 13,824; the
    # activation is applied before the bf16 rounding instead of after it).
    fused_elementwise: bool = True

    def _ffn_fused(self, h: torch.Tensor) -> torch.Tensor:
        lin1, act, lin2 = self.ffn
        if lin1.bias is None or not hasattr(torch, "_addmm_activation"):
            return self.ffn(h)
        a = torch._addmm_activation(lin1.bias, h.reshape(-1, h.shape[-1]), lin1.weight.t(), use_gelu=True)
        return lin2(a).reshape(*h.shape[:-1], -1)

    def forward(self, x: torch.Tensor, context: torch.Tensor, temb: torch.Tensor,
                rotary_emb: torch.Tensor) -> torch.Tensor:
        shift_msa, scale_msa, gate_msa, c_shift, c_scale, c_gate = (self.scale_shift_table + temb.float()).chunk(6, 1)
        if self.fused_elementwise and x.is_cuda and x.shape[0] == 1:
            from . import ops

            h = ops.adaln_modulate(x, self.norm1.eps, scale=scale_msa, shift=shift_msa)
            x = ops.gated_residual(x, self.attn1(h, None, None, rotary_emb), gate_msa)
            h = ops.adaln_modulate(x, self.norm2.eps, weight=self.norm2.weight.float(), bias=self.norm2.bias.float())
            x = x + self.attn2(h, context)
            h = ops.adaln_modulate(x, self.norm3.eps, scale=c_scale, shift=c_shift)
            return ops.gated_residual(x, self._ffn_fused(h), c_gate)
        h = (self.norm1(x.float()) * (1 + scale_msa) + shift_msa).type_as(x)
        x = (x.float() + self.attn1(h, None, None, rotary_emb) * gate_msa).type_as(x)
        h = self.norm2(x.float()).type_as(x)
        x = x + self.attn2(h, context)
        h = (self.norm3(x.float()) * (1 + c_scale) + c_shift).type_as(x)
        return (x.float() + self.ffn(h).float() * c_gate).type_as(x)


class WanLikeDiT(nn.Module):
    """Patch embedding, conditioning, ``cfg.layers`` blocks and the output head."""

    def __init__(self, cfg: DiTConfig, device=None, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.cfg = cfg
        fk = {"device": device, "dtype": dtype}
        f32 = {"device": device, "dtype": torch.float32}
        d, p_in = cfg.dim, cfg.in_channels * math.prod(cfg.patch)
        self.patch_embedding = nn.Linear(p_in, d, **fk)  # the stride = kernel Conv3d as a GEMM over patches
        self.text_embedder = nn.Sequential(nn.Linear(cfg.text_dim, d, **fk), nn.GELU(approximate="tanh"),
                                           nn.Linear(d, d, **fk))
        self.time_embedder = nn.Sequential(nn.Linear(cfg.freq_dim, d, **f32), nn.SiLU(), nn.Linear(d, d, **f32))
        self.time_proj = nn.Sequential(nn.SiLU(), nn.Linear(d, 6 * d, **fk))
        self.blocks = nn.ModuleList(DiTBlock(cfg, **fk) for _ in range(cfg.layers))
        self.norm_out = FP32LayerNorm(d, cfg.eps, elementwise_affine=False, **f32)
        self.proj_out = nn.Linear(d, p_in, **fk)
        self.scale_shift_table = nn.Parameter(torch.zeros(1, 2, d, **f32))
        self.register_buffer("rotary_emb", wan_rope_freqs(cfg.grid, cfg.head_dim, cfg.theta).to(device),
                             persistent=False)

    def attention_modules(self) -> List[Tuple[str, DiTAttention]]:
        """(name, module) in the order diffusers' attn_processors lists them."""
        return [(n, m) for n, m in self.named_modules() if isinstance(m, DiTAttention)]

    def patchify(self, latent: torch.Tensor) -> torch.Tensor:
        b, c, f, h, w = latent.shape
        pf, ph, pw = self.cfg.patch
        x = latent.reshape(b, c, f // pf, pf, h // ph, ph, w // pw, pw)
        x = x.permute(0, 2, 4, 6, 1, 3, 5, 7)  # tokens (f, h, w) row-major, channels (c, pf, ph, pw)
        return x.reshape(b, (f // pf) * (h // ph) * (w // pw), c * pf * ph * pw)

    def unpatchify(self, tokens: torch.Tensor) -> torch.Tensor:
        b = tokens.shape[0]
        f, h, w = self.cfg.grid
        pf, ph, pw = self.cfg.patch
        c = self.cfg.in_channels
        x = tokens.reshape(b, f, h, w, c, pf, ph, pw).permute(0, 4, 1, 5, 2, 6, 3, 7)
        return x.reshape(b, c, f * pf, h * ph, w * pw)

    def forward(self, latent: torch.Tensor, timestep: torch.Tensor, context: torch.Tensor) -> torch.Tensor:
        x = self.patch_embedding(self.patchify(latent).to(self.patch_embedding.weight.dtype))
        temb = self.time_embedder(timestep_embedding(timestep, self.cfg.freq_dim))
        tproj = self.time_proj(temb.to(self.time_proj[1].weight.dtype)).unflatten(1, (6, -1))
        ctx = self.text_embedder(context.to(self.text_embedder[0].weight.dtype))
        for block in self.blocks:
            x = block(x, ctx, tproj, self.rotary_emb)
        shift, scale = (self.scale_shift_table + temb.unsqueeze(1)).chunk(2, dim=1)
        x = (self.norm_out(x.float()) * (1 + scale) + shift).type_as(x)
        return self.unpatchify(self.proj_out(x))


@torch.no_grad()
def init_weights(model: nn.Module, std: float, seed: int) -> None:
    """Every weight, bias and modulation table from N(0, std); norm affine
    weights at one and biases at zero."""
    gen = None
    for name, p in model.named_parameters():
        if gen is None or gen.device != p.device:
            gen = torch.Generator(device=p.device)
            gen.manual_seed(seed)
        if ".norm" in f".{name}" and (name.endswith("weight") or name.endswith("bias")):
            p.fill_(1.0 if name.endswith("weight") else 0.0)
        else:
            p.normal_(0.0, std, generator=gen)


def build_model(cfg: DiTConfig, device, dtype: torch.dtype = torch.bfloat16) -> WanLikeDiT:
    model = WanLikeDiT(cfg, device=device, dtype=dtype).eval()
    init_weights(model, cfg.init_std, cfg.seed)
    return model


def synth_inputs(cfg: DiTConfig, device, seed: Optional[int] = None):
    """(latent [1, C, F*pf, H*ph, W*pw], text context [1, text_len, text_dim],
    negative context) from N(0, 1), generated on the host."""
    gen = torch.Generator().manual_seed(cfg.seed + 1 if seed is None else seed)
    latent = torch.randn(cfg.latent_shape, generator=gen)
    ctx = torch.randn(1, cfg.text_len, cfg.text_dim, generator=gen)
    neg = torch.randn(1, cfg.text_len, cfg.text_dim, generator=gen)
    return latent.to(device), ctx.to(device), neg.to(device)


def install_dfs_processors(model: WanLikeDiT, mode: str = "dfs", sparsity: float = 0.3, tile_size: int = 16,
                           block_size: int = 128, video_perm: Optional[torch.Tensor] = None,
                           skip_layers: Sequence[int] = (), skip_steps: int = 12, cache_interval: int = 12,
                           sparsity_dcrt: float = 0.0, cache_flag: bool = True) -> list:
    """One Wan_DFSAttn_Processor2_0 per attention module, built as the Wan
    driver builds them (wan21_t2v_inference.py:150-173): processor_id is the
    module's index, cross_flag marks the attn2 (text) modules."""
    from .replace_wan import Wan_DFSAttn_Processor2_0

    procs = []
    for i, (name, module) in enumerate(model.attention_modules()):
        proc = Wan_DFSAttn_Processor2_0(mode, sparsity, tile_size, block_size, video_perm, i, list(skip_layers),
                                        skip_steps, cache_interval, sparsity_dcrt, cache_flag, "attn2" in name)
        module.set_processor(proc)
        procs.append(proc)
    return procs


def set_step(procs: Sequence, step_idx: int) -> None:
    """Puts every processor at CFG-pass counter ``step_idx`` (2 per step)."""
    for p in procs:
        p.step_idx = step_idx


@torch.inference_mode()
def denoise_step(model: WanLikeDiT, latent: torch.Tensor, timestep: torch.Tensor, context: torch.Tensor,
                 negative: Optional[torch.Tensor] = None, guidance: float = 5.0) -> torch.Tensor:
    """One denoising step's noise prediction: the conditional pass and, with
    ``negative``, the unconditional pass combined by classifier-free
    guidance (the reference's Wan pipeline runs both; its processors count
    the two passes)."""
    cond = model(latent, timestep, context)
    if negative is None:
        return cond
    uncond = model(latent, timestep, negative)
    return uncond + guidance * (cond - uncond)

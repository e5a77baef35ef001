"""Host-side checks of the DiT harness: parameter count, RoPE frequency
table, patch layout and a CPU forward of the small model (torch path)."""
import math

import pytest
import torch

from dfsattn_amd import dit


def test_param_count_formula():
    cfg = dit.DIT_CONFIGS["tiny"]
    model = dit.WanLikeDiT(cfg, device="cpu", dtype=torch.float32)
    assert cfg.params() == sum(p.numel() for p in model.parameters())
    assert abs(dit.DIT_CONFIGS["cfg4"].params() / 1e9 - 14.29) < 0.01  # the Wan 2.1 14B size


def test_wan_rope_freqs_closed_form():
    grid, d = (4, 6, 10), 128
    freqs = dit.wan_rope_freqs(grid, d)
    assert freqs.shape == (1, 1, 240, 64) and freqs.dtype == torch.complex128
    hw = 2 * (d // 6)  # 42 channels -> 21 frequencies for h and for w
    t_dim = d - 2 * hw  # 44 -> 22 for frames
    f, y, x = 3, 5, 7
    row = freqs[0, 0, f * 60 + y * 10 + x]
    for i in range(22):
        assert abs(row[i] - complex(math.cos(f * 10000 ** (-2 * i / t_dim)), math.sin(f * 10000 ** (-2 * i / t_dim)))) < 1e-12
    for j in range(21):
        a = y * 10000 ** (-2 * j / hw)
        b = x * 10000 ** (-2 * j / hw)
        assert abs(row[22 + j] - complex(math.cos(a), math.sin(a))) < 1e-12
        assert abs(row[43 + j] - complex(math.cos(b), math.sin(b))) < 1e-12


def test_patchify_round_trip():
    cfg = dit.DIT_CONFIGS["tiny"]
    model = dit.WanLikeDiT(cfg, device="cpu", dtype=torch.float32)
    latent = torch.randn(cfg.latent_shape, generator=torch.Generator().manual_seed(0))
    tokens = model.patchify(latent)
    assert tokens.shape == (1, cfg.seq_len, cfg.in_channels * 4)
    assert torch.equal(model.unpatchify(tokens), latent)
    # token (f, y, x) holds the 2x2 pixels of its patch, channel-major
    f, y, x = 1, 3, 5
    tok = tokens[0, f * 256 + y * 16 + x].view(cfg.in_channels, 1, 2, 2)
    assert torch.equal(tok[:, 0], latent[0, :, f, 2 * y:2 * y + 2, 2 * x:2 * x + 2])


@torch.no_grad()
def test_tiny_forward_on_cpu_runs_the_torch_path():
    cfg = dit.DIT_CONFIGS["tiny"]
    model = dit.build_model(cfg, "cpu", torch.float32)
    procs = dit.install_dfs_processors(model, "flash")
    assert len(procs) == 2 * cfg.layers and [p.cross_flag for p in procs[:2]] == [False, True]
    latent, ctx, neg = dit.synth_inputs(cfg, "cpu")
    out = dit.denoise_step(model, latent, torch.tensor([500.0]), ctx, neg)
    assert out.shape == latent.shape and bool(torch.isfinite(out).all())
    assert [p.step_idx for p in procs] == [2] * len(procs)  # both CFG passes counted

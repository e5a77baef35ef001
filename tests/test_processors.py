"""Processors, their dense/sparse branch schedule and installation on a model
(replace_wan.py:135-324, replace_hyvideo.py:230-464, attn_processor.py).

CPU: the branch taken on every call of a denoising run is checked against
schedules worked out by hand from the reference's rules (warm-up steps,
skip layers, CFG step counting, periodic dense steps, rest phases), with the
attention functions replaced by recorders. GPU tests live in
test_gpu_processors.py.
"""
import math

import pytest
import torch
import torch.nn as nn

from dfsattn_amd import replace_hyvideo as hy
from dfsattn_amd import replace_wan as wan
from dfsattn_amd.attn_processor import get_attn_processors, set_attn_processor
from stubs import StubAttention


class Recorder:
    def __init__(self):
        self.calls = []

    def dfs(self, q, k, v, **kw):
        self.calls.append(("dfs", kw["step_idx"]))
        return torch.zeros_like(q)

    def full(self, q, k, v, mode="flash", **kw):
        self.calls.append(("dense", mode))
        return torch.zeros_like(q)


@pytest.fixture
def rec(monkeypatch):
    r = Recorder()
    monkeypatch.setattr(wan, "dfs_attention", r.dfs)
    monkeypatch.setattr(wan, "full_attention", r.full)
    monkeypatch.setattr(hy, "dfs_attention", r.dfs)
    monkeypatch.setattr(hy, "full_attention", r.full)
    return r


def _wan_proc(layer=3, skip_layers=(), skip_steps=12, cross=False, **kw):
    return wan.Wan_DFSAttn_Processor2_0("dfs", 0.3, 16, 128, torch.arange(32), layer, list(skip_layers), skip_steps,
                                        12, 0.1, True, cross, **kw)


def _run_wan(proc, calls, seq=32, dim=64):
    attn = StubAttention(dim=dim)
    x = torch.randn(1, seq, dim)
    for _ in range(calls):
        out = proc(attn, x)
        assert out.shape == x.shape


def _kinds(rec):
    return [c[0] for c in rec.calls]


def test_wan_warmup_then_sparse(rec):
    """skip_steps 12 real steps = 24 calls (cond + uncond per step)."""
    _run_wan(_wan_proc(), 100)
    kinds = _kinds(rec)
    assert kinds[:24] == ["dense"] * 24 and kinds[24:] == ["dfs"] * 76
    assert [c[1] for c in rec.calls[24:27]] == [24, 25, 26]  # dfs sees the raw call counter


def test_wan_skip_layer_and_cross_attention_stay_dense(rec):
    _run_wan(_wan_proc(layer=5, skip_layers=(5,)), 60)
    _run_wan(_wan_proc(cross=True), 60)
    assert set(_kinds(rec)) == {"dense"}


def test_wan_counter_wraps_after_fifty_steps(rec):
    proc = _wan_proc()
    _run_wan(proc, 100)
    assert proc.step_idx == 0
    _run_wan(proc, 1)
    assert rec.calls[-1][0] == "dense"  # warm-up again


def test_wan_periodic_dense_and_dense_step(rec):
    # dense_interval 5: real steps with (s - 12 + 1) % 5 == 0 -> 16, 21, 26, ...
    _run_wan(_wan_proc(dense_interval=5, dense_step_idx=60), 100)
    kinds = _kinds(rec)
    dense_real = sorted({i // 2 for i, k in enumerate(kinds) if k == "dense" and i >= 24})
    assert dense_real == [16, 21, 26, 30, 31, 36, 41, 46]  # 30: call 60 (dense_step_idx)
    assert kinds[60] == "dense" and kinds[61] == "dfs"


def test_wan_rest_phase(rec):
    # sparse for real steps 12..21, dense 22..26, sparse from 27
    _run_wan(_wan_proc(rest_steps=10, skip_steps2=5), 100)
    kinds = _kinds(rec)
    per_step = [kinds[2 * s] for s in range(50)]
    assert per_step[:12] == ["dense"] * 12
    assert per_step[12:22] == ["dfs"] * 10
    assert per_step[22:27] == ["dense"] * 5
    assert per_step[27:] == ["dfs"] * 23


def test_wan_projection_path_and_i2v_branch(rec):
    """Output = to_out(attention(...)) + image-context attention (zero
    attention from the recorder leaves to_out's bias, plus SDPA of the image
    context for I2V)."""
    torch.manual_seed(0)
    attn = StubAttention(dim=64, added_kv=True)
    proc = _wan_proc()
    x = torch.randn(1, 32, 64)
    ctx = torch.randn(1, 257 + 512, 64)  # 257 image tokens, then 512 text tokens
    out = proc(attn, x, encoder_hidden_states=ctx)
    q = attn.norm_q(attn.to_q(x)).unflatten(2, (2, -1)).transpose(1, 2)
    k_img = attn.norm_added_k(attn.add_k_proj(ctx[:, :257])).unflatten(2, (2, -1)).transpose(1, 2)
    v_img = attn.add_v_proj(ctx[:, :257]).unflatten(2, (2, -1)).transpose(1, 2)
    img = torch.softmax(q @ k_img.transpose(-1, -2) / math.sqrt(32), -1) @ v_img
    expect = attn.to_out[0](img.transpose(1, 2).flatten(2, 3))
    assert torch.allclose(out, expect, atol=1e-5)


def test_rotary_complex_matches_pairwise_rotation():
    torch.manual_seed(1)
    x = torch.randn(1, 2, 5, 8)
    theta = torch.randn(5, 4)
    freqs = torch.polar(torch.ones_like(theta), theta).to(torch.complex128)
    got = wan.apply_rotary_emb_complex(x, freqs)
    a, b = x[..., 0::2].double(), x[..., 1::2].double()
    c, s = torch.cos(theta).double(), torch.sin(theta).double()
    expect = torch.stack([a * c - b * s, a * s + b * c], dim=-1).flatten(3)
    assert torch.allclose(got.double(), expect, atol=1e-6)
    # the real (cos, sin) form used by HunyuanVideo gives the same rotation
    got_hy = hy.apply_rotary_emb(x, (c.float().repeat_interleave(2, -1), s.float().repeat_interleave(2, -1)))
    assert torch.allclose(got_hy.double(), expect, atol=1e-5)


def _hy_proc(layer=0, skip_layers=(), **kw):
    return hy.HunyuanVideo_DFSAttn_Processor2_0("dfs", 0.3, 16, 128, 24, torch.arange(24), layer,
                                               list(skip_layers), 12, 12, 0.1, True, **kw)


def test_hunyuan_schedule_and_wrap(rec):
    proc = _hy_proc(dense_interval=4)
    attn = StubAttention(dim=64, norm_shape=32)  # HunyuanVideo normalises per head
    x, txt = torch.randn(1, 24, 64), torch.randn(1, 8, 64)
    mask = torch.ones(32, dtype=torch.bool)
    for _ in range(50):
        hs, enc = proc(attn, x, encoder_hidden_states=txt, attention_mask=mask)
        assert hs.shape == (1, 24, 64) and enc.shape == (1, 8, 64)
    kinds = _kinds(rec)
    # Hunyuan counts real steps; periodic dense at (s - 12 + 1) % 4 == 0: 15, 19, ...
    assert kinds[:12] == ["dense"] * 12
    assert [s for s in range(12, 50) if kinds[s] == "dense"] == [15, 19, 23, 27, 31, 35, 39, 43, 47]
    assert proc.step_idx == 0


def test_hunyuan_full_attention_modes(rec):
    for mode in ("flash", "torch", "vanilla"):
        proc = hy.HunyuanVideo_DFSAttn_Processor2_0(mode, 0.3, 16, 128, 24, None, 0, [], 12, 12, 0.1, True)
        proc(StubAttention(dim=64, norm_shape=32), torch.randn(1, 24, 64), encoder_hidden_states=torch.randn(1, 8, 64),
             attention_mask=torch.ones(32, dtype=torch.bool))
    assert rec.calls == [("dense", "flash"), ("dense", "torch"), ("dense", "vanilla")]


def test_hunyuan_double_stream_concatenates_text(rec, monkeypatch):
    seen = {}

    def full(q, k, v, mode="flash", **kw):
        seen["shape"] = tuple(q.shape)
        return torch.zeros_like(q)

    monkeypatch.setattr(hy, "full_attention", full)
    proc = hy.HunyuanVideo_DFSAttn_Processor2_0("flash", 0.3, 16, 128, 24, None, 0, [], 12, 12, 0.1, True)
    attn = StubAttention(dim=64, added_q=True, norm_shape=32)
    hs, enc = proc(attn, torch.randn(1, 24, 64), encoder_hidden_states=torch.randn(1, 8, 64),
                   attention_mask=torch.ones(32, dtype=torch.bool))
    assert seen["shape"] == (1, 2, 32, 32)
    assert hs.shape == (1, 24, 64) and enc.shape == (1, 8, 64)


def test_hunyuan_debug_steps_validation():
    with pytest.raises(ValueError):
        _hy_proc(attention_debug_steps=[-1])
    p = _hy_proc(attention_debug_step=-1)
    assert p.attention_debug_steps == (12,)


def test_set_and_get_attn_processors():
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Module() for _ in range(3)])
    for b in model.blocks:
        b.attn1 = StubAttention()
        b.attn2 = StubAttention()
    procs = get_attn_processors(model)
    assert sorted(procs) == sorted(f"blocks.{i}.attn{j}.processor" for i in range(3) for j in (1, 2))
    set_attn_processor(model, "shared")
    assert all(p == "shared" for p in get_attn_processors(model).values())
    per_layer = {k: i for i, k in enumerate(procs)}
    set_attn_processor(model, dict(per_layer))
    assert get_attn_processors(model) == per_layer
    with pytest.raises(ValueError):
        set_attn_processor(model, {"blocks.0.attn1.processor": 1})

"""GPU parity of the dense path (full_attention) and of whole processor calls
against fp32 references on the host."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import dfs_oracle as orc

pytestmark = pytest.mark.gpu


def _rel(out, ref):
    return float((out.double() - ref.double()).abs().mean() / ref.double().abs().mean())


def _sdpa32(q, k, v):
    """fp32 host reference (math backend, contiguous operands)."""
    s = (q.float() @ k.float().transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
    return torch.softmax(s, -1) @ v.float()


@pytest.fixture(autouse=True)
def _clean():
    from dfsattn_amd import attention_hyvideo as hyat
    from dfsattn_amd import attention_wan as wat
    for mod in (wat, hyat):
        mod.DFS_Attention.clear_cache()
        mod._dfs_attention_instances.clear()
    yield


@pytest.mark.parametrize("length,d", [(1000, 128), (300, 64)])
def test_full_attention_flash_self_matches_dense(dev, length, d):
    from dfsattn_amd.fullattention import full_attention
    g = torch.Generator().manual_seed(length)
    q, k, v = (torch.randn(1, 2, length, d, generator=g).to(torch.bfloat16) for _ in range(3))
    cu = torch.tensor([0, length, length], dtype=torch.int32, device=dev)
    out = full_attention(q.to(dev), k.to(dev), v.to(dev), mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu,
                         max_seqlen_q=length, max_seqlen_kv=length)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    ref = _sdpa32(q, k, v)
    assert _rel(out.cpu(), ref) < 4e-3 and float((out.cpu().float() - ref).abs().max()) < 2e-2


def test_full_attention_flash_segments_and_cross(dev):
    """[0, valid, L]: the valid tokens attend among themselves, the padding
    segment among itself; a rectangular (cross-attention) call runs too."""
    from dfsattn_amd.fullattention import full_attention
    g = torch.Generator().manual_seed(5)
    L, valid = 600, 530
    q, k, v = (torch.randn(1, 2, L, 128, generator=g).to(torch.bfloat16) for _ in range(3))
    cu = torch.tensor([0, valid, L], dtype=torch.int32, device=dev)
    out = full_attention(q.to(dev), k.to(dev), v.to(dev), mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu,
                         max_seqlen_q=L, max_seqlen_kv=L).cpu()
    ref = torch.cat([_sdpa32(q[:, :, :valid], k[:, :, :valid], v[:, :, :valid]),
                     _sdpa32(q[:, :, valid:], k[:, :, valid:], v[:, :, valid:])], dim=2)
    assert _rel(out, ref) < 4e-3
    kc, vc = (torch.randn(1, 2, 96, 128, generator=g).to(torch.bfloat16) for _ in range(2))
    cq = torch.tensor([0, L, L], dtype=torch.int32, device=dev)
    ck = torch.tensor([0, 96, 96], dtype=torch.int32, device=dev)
    out = full_attention(q.to(dev), kc.to(dev), vc.to(dev), mode="flash", cu_seqlens_q=cq, cu_seqlens_kv=ck,
                         max_seqlen_q=L, max_seqlen_kv=96).cpu()
    assert _rel(out, _sdpa32(q, kc, vc)) < 4e-3


def test_full_attention_flash_many_host_segments(dev):
    """Host cu_seqlens of more than two segments (beyond the device varlen
    path) run segment by segment, each square segment on the native kernel."""
    from dfsattn_amd.fullattention import full_attention
    g = torch.Generator().manual_seed(6)
    L = 700
    bounds = [0, 200, 201, 530, L]
    q, k, v = (torch.randn(1, 2, L, 128, generator=g).to(torch.bfloat16) for _ in range(3))
    cu = torch.tensor(bounds, dtype=torch.int32)
    out = full_attention(q.to(dev), k.to(dev), v.to(dev), mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu,
                         max_seqlen_q=L, max_seqlen_kv=L).cpu()
    ref = torch.cat([_sdpa32(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b]) for a, b in zip(bounds, bounds[1:])], dim=2)
    assert _rel(out, ref) < 4e-3 and float((out.float() - ref).abs().max()) < 2e-2


def _stub(dim, heads, dev, norm_shape=None, added_q=False):
    from stubs import StubAttention
    torch.manual_seed(3)
    m = StubAttention(dim=dim, heads=heads, norm_shape=norm_shape, added_q=added_q)
    return m.to(dev, torch.bfloat16).eval()


@torch.no_grad()
def test_wan_processor_sparse_step_matches_reference(dev):
    """One DFS step of the Wan processor (1,024 tokens, 2 heads of 64):
    output = to_out(attention) with the attention recomputed in fp32 on the
    host over the mask the GPU selected."""
    from dfsattn_amd.attention_wan import DFS_Attention
    from dfsattn_amd.replace_wan import Wan_DFSAttn_Processor2_0
    from dfsattn_amd.utils.order import hilbert3d_perm
    grid, heads, dim = (4, 16, 16), 2, 128
    perm = hilbert3d_perm(*grid)
    attn = _stub(dim, heads, dev)
    proc = Wan_DFSAttn_Processor2_0("dfs", 0.3, 16, 128, perm, 0, [], 12, 12, 0.1, True, False)
    proc.step_idx = 24  # first sparse call (real step 12)
    x = torch.randn(1, 1024, dim, generator=torch.Generator().manual_seed(7)).to(dev, torch.bfloat16)
    out = proc(attn, x)
    q = attn.norm_q(attn.to_q(x)).unflatten(2, (heads, -1)).transpose(1, 2).cpu().float()
    k = attn.norm_k(attn.to_k(x)).unflatten(2, (heads, -1)).transpose(1, 2).cpu().float()
    v = attn.to_v(x).unflatten(2, (heads, -1)).transpose(1, 2).cpu().float()
    mask = DFS_Attention._cached_metadata[(0, "native", 128, 16, 16)]["block_mask"].cpu()
    p, inv = orc.full_permutation(perm, 1024)
    ref = orc.masked_attention(*(orc.apply_permutation(t, p) for t in (q, k, v)), mask)[:, :, inv]
    expect = attn.to_out[0](ref.transpose(1, 2).flatten(2, 3).to(dev, torch.bfloat16))
    assert _rel(out.cpu(), expect.cpu()) < 1e-2


@pytest.mark.parametrize("n_pad", [0, 30])
@torch.no_grad()
def test_hunyuan_processor_sparse_step_with_text(dev, n_pad):
    """n_pad trailing text tokens masked out by attention_mask: the processor
    passes cu_seqlens [0, valid, L] and the valid length, so valid tokens and
    padding attend as two sequences (attention_hyvideo.py:1054-1082)."""
    from dfsattn_amd.attention_hyvideo import DFS_Attention
    from dfsattn_amd.replace_hyvideo import HunyuanVideo_DFSAttn_Processor2_0
    from dfsattn_amd.utils.order import hilbert3d_perm
    grid, heads, dim, n_text = (3, 16, 20), 2, 256, 100
    video_len = grid[0] * grid[1] * grid[2]
    perm = hilbert3d_perm(*grid)
    attn = _stub(dim, heads, dev, norm_shape=128)
    proc = HunyuanVideo_DFSAttn_Processor2_0("dfs", 0.5, 16, 128, video_len, perm, 0, [], 12, 12, 0.1, True)
    proc.step_idx = 12
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, video_len, dim, generator=g).to(dev, torch.bfloat16)
    txt = torch.randn(1, n_text, dim, generator=g).to(dev, torch.bfloat16)
    mask = torch.ones(video_len + n_text, dtype=torch.bool, device=dev)
    if n_pad:
        mask[-n_pad:] = False
    hs, enc = proc(attn, x, encoder_hidden_states=txt, attention_mask=mask)
    joint = torch.cat([x, txt], dim=1)
    q = attn.norm_q(attn.to_q(joint).unflatten(2, (heads, -1)).transpose(1, 2)).cpu().float()
    k = attn.norm_k(attn.to_k(joint).unflatten(2, (heads, -1)).transpose(1, 2)).cpu().float()
    v = attn.to_v(joint).unflatten(2, (heads, -1)).transpose(1, 2).cpu().float()
    key = next(iter(DFS_Attention._cached_metadata))
    bmask = DFS_Attention._cached_metadata[key]["block_mask"].cpu()
    p, inv = orc.full_permutation(perm, video_len + n_text)
    L = video_len + n_text
    ref = orc.segment_attention(*(orc.apply_permutation(t, p) for t in (q, k, v)), bmask, [0, L - n_pad, L])
    ref = ref[:, :, inv].transpose(1, 2).flatten(2, 3).to(dev, torch.bfloat16)
    exp_hs = attn.to_out[0](ref[:, :video_len])
    exp_enc = ref[:, video_len:]
    assert _rel(hs.cpu(), exp_hs.cpu()) < 1e-2
    assert _rel(enc.cpu(), exp_enc.cpu()) < 1e-2

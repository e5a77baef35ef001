"""The reference-side bindings that the repository's integration guide
prints, run exactly as printed (the Python blocks are read from the guide
at DOC; only the library path placeholder is pointed at this build): the
ctypes replacement of block_sparse_attn_func (attention_wan.py:335-391) and
the RoPE / RMSNorm shims of replace_wan.py:24-66, against the oracle."""
import math
import os
import re

import pytest
import torch

from dfsattn_amd import _lib
from oracle import dfs_oracle as orc

pytestmark = pytest.mark.gpu

DOC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")


def _rel(out, ref):
    return float((out.double() - ref.double()).abs().mean() / ref.double().abs().mean())


def _printed_bindings():
    """Namespace after executing the document's ctypes blocks in order."""
    text = open(DOC, encoding="utf-8").read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    stub = [b for b in blocks if "def amd_block_sparse_attention" in b]
    shims = [b for b in blocks if "def triton_rmsnorm_forward" in b]
    assert len(stub) == 1 and len(shims) == 1
    ns = {}
    code = stub[0].replace("/path/to/dfsattn_amd/_lib/libdfsattn_amd.so", _lib.LIB_PATH)
    exec(compile(code, "INTEGRATION.md:stub", "exec"), ns)
    exec(compile(shims[0], "INTEGRATION.md:shims", "exec"), ns)
    return ns


@pytest.mark.parametrize("heads,length,big_v", [(3, 1000, False), (2, 777, True)])
def test_printed_block_sparse_stub(dev, heads, length, big_v):
    """amd_block_sparse_attention on permuted bf16 inputs and a bool block
    mask, as _run_block_sparse_attention would call it, against fp32 masked
    attention (bf16 output); with V beyond the f16 range in one head."""
    ns = _printed_bindings()
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    cfg = DfsConfig("stub", (1, 1, length), heads, 128, torch.bfloat16, seed=41)
    q, k, v = (x.clone() for x in synth_qkv(cfg))
    if big_v:
        v[:, 1] = (v[:, 1].float() * 2.0e5).to(torch.bfloat16)
    nb = math.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=torch.Generator().manual_seed(42)) < 0.4
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    out = ns["amd_block_sparse_attention"](q.to(dev), k.to(dev), v.to(dev), mask.to(dev))
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    ref = orc.masked_attention(q, k, v, mask)
    got = out.cpu().float()
    assert bool(torch.isfinite(got).all())
    for h in range(heads):
        assert _rel(got[:, h], ref[:, h]) < 4e-3, h


def test_printed_rope_and_rmsnorm_shims(dev):
    """The printed apply_qk_rope_inplace_cossin_complex (in place on [B, H, S,
    D], the first len_text_prompt rows left) and triton_rmsnorm_forward
    (over the last axis) against the oracle's restatements."""
    ns = _printed_bindings()
    g = torch.Generator().manual_seed(43)
    B, H, S, D, skip = 1, 4, 200, 128, 16
    q = (torch.randn(B, H, S, D, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(B, H, S, D, generator=g) * 2).to(torch.bfloat16)
    ang = torch.rand(S - skip, D // 2, generator=g, dtype=torch.float64) * 20
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    qd, kd = q.to(dev), k.to(dev)
    ns["apply_qk_rope_inplace_cossin_complex"](qd, kd, cos.to(dev), sin.to(dev), skip)
    for got, x in ((qd, q), (kd, k)):
        ref = x.clone()
        ref[:, :, skip:] = orc.rope_complex_pairs(x[:, :, skip:], cos, sin)
        assert torch.equal(got.cpu(), ref)  # the rotation alone is bit-exact
    x = (torch.randn(3, 50, 5120, generator=g) * 3).to(torch.bfloat16)
    w = (torch.rand(5120, generator=g) + 0.5).to(torch.bfloat16)
    y = ns["triton_rmsnorm_forward"](x.to(dev), w.to(dev), 1e-6).cpu()
    ref = orc.rmsnorm_rows(x, w, 1e-6)
    assert y.shape == x.shape and y.dtype == x.dtype
    torch.testing.assert_close(y.float(), ref.float(), rtol=2.0 ** -7, atol=1e-5)
    assert float((y == ref).float().mean()) > 0.99

"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the synthetic generator and the oracle still reproduce the fixtures, and
the fixtures satisfy what the mathematics fixes independently of the oracle
(softmax rows of the block scores sum to block/tile, the selection keeps
exactly k columns per row under each policy, text query rows equal dense
attention, the Hilbert permutation equals the C library's).
GPU: the HIP path against the fixtures: fp32 block scores within 2e-3,
selection from the fixture's own scores bit-exact, block-sparse attention
(fp32 output) within max-abs 2e-2 and mean-rel 1e-3 of the fixture output.
"""
import math
import os

import numpy as np
import pytest
import torch

from dfsattn_amd.layout import ScoringLayout, hunyuan_policy, topk_count, wan_policy
from dfsattn_amd.workloads import CONFIGS, DfsConfig, synth_qkv
from oracle import dfs_oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ("cfg0", "hytext", "tail")
SPECS = {
    "cfg0": CONFIGS[0],
    "hytext": DfsConfig("hytext", (4, 8, 16), 2, 64, torch.bfloat16, text_len=40, seed=7),
    "tail": DfsConfig("tail", (3, 7, 9), 1, 64, torch.bfloat16, seed=11),
}


def load(name):
    d = np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False)
    return {k: d[k] for k in d.files}


def as_f32(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float()


def layout_policy(g):
    L = g["q"].shape[2]
    vl = int(g["video_len"])
    lay = ScoringLayout(L, vl, int(g["tile"]))
    pol = hunyuan_policy(lay, float(g["sparsity"])) if bool(g["hunyuan"]) else wan_policy(lay, float(g["sparsity"]))
    return lay, pol


@pytest.mark.parametrize("name", CASES)
def test_generator_reproduces_inputs(name):
    g = load(name)
    q, k, v = synth_qkv(SPECS[name], dtype=torch.float32)
    for x, key in ((q, "q"), (k, "k"), (v, "v")):
        bits = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(bits, g[key]), key


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    g = load(name)
    q, k, v = (as_f32(g[x]) for x in "qkv")
    vl = int(g["video_len"]) if bool(g["hunyuan"]) else None
    out, mask, scores = orc.dfs_attention_reference(q, k, v, torch.from_numpy(g["perm"]), float(g["sparsity"]),
                                                    int(g["tile"]), video_len=vl)
    assert np.array_equal(mask.numpy(), g["mask"])
    np.testing.assert_allclose(scores.numpy(), g["scores"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(out.numpy(), g["out"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", CASES)
def test_fixture_invariants(name):
    """Properties fixed by the definitions, independent of the oracle code."""
    g = load(name)
    heads, L = g["q"].shape[1], g["q"].shape[2]
    vl, tile = int(g["video_len"]), int(g["tile"])
    kb = math.ceil(L / 128)
    # every scored row is a sum of 8 x 8 tile-softmax rows: 128 / 16 = 8
    np.testing.assert_allclose(g["scores"].sum(-1), 128 / tile, rtol=1e-5)
    mask = g["mask"]
    assert mask.shape == (heads, kb, kb)
    k = topk_count(float(g["sparsity"]), kb)
    if bool(g["hunyuan"]):
        ds = vl // 128
        assert mask[:, :, ds:].all() and mask[:, ds:, :].all()
        assert (mask[:, :ds].sum(-1) == k).all()
    else:
        assert (mask.sum(-1) == k).all()
        # kept columns are the k largest scores of the row (no ties in these fixtures)
        for h in range(heads):
            for i in range(kb):
                top = set(np.argsort(-g["scores"][h, i], kind="stable")[:k].tolist())
                assert top == set(np.nonzero(mask[h, i])[0].tolist())
    # Hilbert permutation: a bijection of the video tokens, equal to the C library's
    from dfsattn_amd import ops
    perm = g["perm"]
    assert np.array_equal(np.sort(perm), np.arange(vl))
    assert np.array_equal(ops.hilbert3d_perm(*g["grid"].tolist()).numpy(), perm)
    # text query rows see every key: dense softmax attention closed form
    if bool(g["hunyuan"]):
        q, k_, v = (as_f32(g[x]) for x in "qkv")
        s = (q[:, :, vl:] @ k_.transpose(-1, -2)) / math.sqrt(q.shape[-1])
        ref = torch.softmax(s, dim=-1) @ v
        np.testing.assert_allclose(g["out"][:, :, vl:], ref.numpy(), rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_gpu_matches_fixture(name, dev):
    from dfsattn_amd import ops

    g = load(name)
    lay, pol = layout_policy(g)
    q, k, v = (torch.from_numpy(g[x].view(np.int16).copy()).view(torch.bfloat16).to(dev) for x in "qkv")
    full, _ = orc.full_permutation(torch.from_numpy(g["perm"]), q.shape[2])
    perm_d = ops.device_perm(full, dev)
    row_ptr = torch.from_numpy(pol.row_ptr(q.shape[1])).to(dev)
    prep = ops.prepare_qkv(q, k, v, perm_d, lay)
    # scoring: fp32 block scores of the GPU against the fixture
    _, scores, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True)
    np.testing.assert_allclose(scores.cpu().numpy(), g["scores"], rtol=1e-5, atol=1e-10)
    # selection from the fixture's own fp32 scores: bit-exact mask
    col_idx, mask = ops.topk_from_scores(torch.from_numpy(g["scores"]).to(dev), pol, row_ptr, want_mask=True)
    assert np.array_equal(mask.cpu().numpy().astype(bool), g["mask"])
    # attention over the fixture mask, fp32 output in the original order
    out = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=torch.float32, out_perm=perm_d)
    torch.cuda.synchronize()
    ref = torch.from_numpy(g["out"]).double()
    err = (out.cpu().double() - ref).abs()
    assert float(err.max()) <= 2e-2
    assert float(err.mean() / ref.abs().mean()) <= 1e-3

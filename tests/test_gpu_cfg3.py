"""the mask-cache regime at the 75.6k-token Wan shape. 50
sequential denoising calls with Q_t = Q_{t-1} + N(0, 0.02) (likewise K):
the first 12 real steps dense, then dfs_attention with skip 12, interval 12
and the step counter counting CFG passes (attention_wan.py:41-66, 432-470,
792-800). Checks the refresh steps and their top-k sizes for sparsity 0.3
with the reference's default decay 0.1 and without decay, and for sparsity
0.5 (the sweep's largest point) without decay, that cached calls
reuse the refreshed columns bit for bit, the fresh selection (bit-exact
from the GPU's own fp32 scores, and against the oracle's fp32 scores up to
near-ties), and sampled query blocks of one refresh call and one
cached call against fp32 masked attention (fp32 output, 1e-3 mean-rel)."""
import pytest
import torch

from oracle import dfs_oracle as orc

pytestmark = pytest.mark.gpu


def _rel(out, ref):
    return float((out.double() - ref.double()).abs().mean() / ref.double().abs().mean())


def _check_output(dev, entry, q, k, v, full, perm_d, lay, out_bf16, label):
    """fp32 output of the call's operands and cached mask, on sampled query
    blocks of two heads, against fp32 masked attention."""
    from dfsattn_amd import ops
    H, L = q.shape[1], q.shape[2]
    heads = [0, H - 1]
    qbs = [0, lay.q_blocks // 2, lay.q_blocks - 1]
    mask = entry["block_mask"].cpu()
    sub = [orc.apply_permutation(t[:, heads].float().cpu(), full) for t in (q, k, v)]
    ref = orc.masked_attention(*sub, mask[heads], 128, q_blocks=qbs)
    rows = torch.cat([torch.arange(b * 128, min((b + 1) * 128, L)) for b in qbs])
    prep = ops.prepare_qkv(q, k, v, perm_d, lay, pool=False)
    out32 = ops.bsa_fwd(prep, entry["row_ptr"], entry["col_idx"], out_dtype=torch.float32)
    g32, r = out32[:, heads].cpu()[:, :, rows], ref[:, :, rows]
    max_abs, mr = float((g32 - r).abs().max()), _rel(g32, r)
    print(f"{label}: fp32 output max-abs {max_abs:.2e}, mean-rel {mr:.2e}", flush=True)
    assert max_abs <= 2e-2 and mr <= 1e-3
    # the call's own (bf16) output is the same computation, rounded
    got = out_bf16[:, heads].cpu()[:, :, full][:, :, rows].float()
    assert _rel(got, g32) < 4e-3


def _check_selection(dev, entry, q, k, v, full, perm_d, lay, kpick, label):
    """Head 0 of a refresh: the cached mask is the top-k of the GPU's own fp32
    block scores (bit-exact), and every row that selects differently from the
    oracle's fp32 scores has its k-th and (k+1)-th oracle scores closer than
    twice the measured score error."""
    from dfsattn_amd import ops
    from dfsattn_amd.layout import TopkPolicy
    Kb = lay.k_blocks
    pol = TopkPolicy(lay.q_blocks, Kb, lay.q_blocks, Kb, kpick, Kb, lay.q_blocks)
    prep = ops.prepare_qkv(q[:, :1], k[:, :1], v[:, :1], perm_d, lay)
    row_ptr = torch.from_numpy(pol.row_ptr(1)).to(dev)
    _, scores, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True)
    got = scores.cpu()
    mask = entry["block_mask"][:1].cpu()
    assert torch.equal(mask, orc.select_topk(got, kpick))
    qp = orc.apply_permutation(q[:, :1].float().cpu(), full)
    kp = orc.apply_permutation(k[:, :1].float().cpu(), full)
    ref_scores = orc.block_scores(qp, kp, lay.tile, 128, None, head_chunk=1)
    ref_sel = orc.select_topk(ref_scores, kpick)
    err = float((got - ref_scores).abs().max())
    gaps = []
    for r in range(ref_scores.shape[1]):
        if not torch.equal(mask[0, r], ref_sel[0, r]):
            top = torch.sort(ref_scores[0, r], descending=True).values
            gaps.append(float(top[kpick - 1] - top[kpick]))
    print(f"{label}: {len(gaps)} of {ref_scores.shape[1]} rows select differently from the oracle's fp32 scores; "
          f"max score error {err:.2e}, largest gap among them {max(gaps, default=0.0):.2e}", flush=True)
    assert all(g <= 2 * err for g in gaps), (gaps, err)


@pytest.mark.parametrize("sparsity,dcrt,expect", [(0.3, 0.1, {12: 177, 24: 118, 36: 59}),
                                                  (0.3, 0.0, {12: 177, 24: 177, 36: 177, 48: 177}),
                                                  (0.5, 0.0, {12: 295, 24: 295, 36: 295, 48: 295})])
def test_mask_cache_regime_at_cfg1_shape(dev, sparsity, dcrt, expect):
    from dfsattn_amd import ops
    from dfsattn_amd.attention_wan import DFS_Attention, _dfs_attention_instances, dfs_attention
    from dfsattn_amd.fullattention import full_attention
    from dfsattn_amd.layout import ScoringLayout
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[1]
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()
    q, k, v = synth_qkv(cfg, device=dev)
    perm = hilbert3d_perm(*cfg.grid)
    L = cfg.seq_len
    full, _ = orc.full_permutation(perm, L)
    perm_d = ops.device_perm(full, dev)
    lay = ScoringLayout(L, L, cfg.tile)
    gen = torch.Generator(device=dev).manual_seed(33)
    key = (0, "native", 128, 16, 16)
    refreshes, kept_cols, prev = {}, None, None
    for t in range(50):
        if t > 0:  # the drift of the configuration: N(0, 0.02) per step on Q and K
            q = (q.float() + 0.02 * torch.randn(q.shape, generator=gen, device=dev)).to(q.dtype)
            k = (k.float() + 0.02 * torch.randn(k.shape, generator=gen, device=dev)).to(k.dtype)
        if t < 12:  # dense warm-up steps (replace_wan.py:252-302)
            if t in (0, 11):
                dense = full_attention(q, k, v, mode="flash")
                assert bool(torch.isfinite(dense).all())
            continue
        out = dfs_attention(q, k, v, step_idx=2 * t, skip_steps=12, cache_interval=12, layer_idx=0,
                            sparsity=sparsity, sparsity_dcrt=dcrt, tile_size=cfg.tile, video_perm=perm,
                            cache_flag=True)
        entry = DFS_Attention._cached_metadata[key]
        if entry is not prev:  # a refresh stored a new entry
            kpick = int((entry["row_ptr"][1] - entry["row_ptr"][0]).item())
            refreshes[t] = kpick
            kept_cols = entry["col_idx"].clone()
            if t == 24:  # the fresh selection of head 0 against the oracle's fp32 scores
                _check_selection(dev, entry, q, k, v, full, perm_d, lay, kpick, f"s {sparsity} dcrt {dcrt} step {t}")
            if t == 12:
                _check_output(dev, entry, q, k, v, full, perm_d, lay, out, f"s {sparsity} dcrt {dcrt} refresh step {t}")
        else:
            assert torch.equal(entry["col_idx"], kept_cols)  # the cached columns, bit for bit
            if t == 13:
                _check_output(dev, entry, q, k, v, full, perm_d, lay, out, f"s {sparsity} dcrt {dcrt} cached step {t}")
        prev = entry
    print(f"s {sparsity} dcrt {dcrt}: refreshes at real steps {refreshes}", flush=True)
    assert refreshes == expect
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()

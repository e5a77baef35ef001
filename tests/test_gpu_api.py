"""End-to-end parity of the reference-compatible API on the GPU:
dfs_attention (Wan and HunyuanVideo variants) against the CPU oracle's whole
call on the same (bf16-rounded) inputs, and the mask cache behaviour."""
import math

import pytest
import torch

from oracle import dfs_oracle as orc

pytestmark = pytest.mark.gpu


def _rel(out, ref):
    return float((out.double() - ref.double()).abs().mean() / ref.double().abs().mean())


def _assert_selection(mask, q, k, v, perm, sparsity, tile, ref_scores, dev, video_len=None):
    """The cached mask is the oracle's selection rule applied to the GPU's own
    fp32 block scores, bit-exact; and every row where it differs from the
    selection over the oracle's fp32 scores is one whose k-th and (k+1)-th
    oracle candidate scores lie closer than twice the measured score error
    (two scores each off by at most that much can swap)."""
    from dfsattn_amd import ops
    from dfsattn_amd.layout import ScoringLayout, hunyuan_policy, wan_policy

    L, H = q.shape[2], q.shape[1]
    full, _ = orc.full_permutation(perm, L)
    lay = ScoringLayout(L, video_len or L, tile)
    pol = hunyuan_policy(lay, sparsity) if video_len else wan_policy(lay, sparsity)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ops.device_perm(full, dev), lay)
    row_ptr = torch.from_numpy(pol.row_ptr(H)).to(dev)
    _, scores, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True)
    got = scores.cpu()

    def pick(s):
        return (orc.mask_from_scores_hunyuan(s, sparsity, L, video_len) if video_len
                else orc.mask_from_scores_wan(s, sparsity))

    assert torch.equal(mask, pick(got))
    ref_sel = pick(ref_scores)
    err = float((got - ref_scores).abs().max())
    differ = [(h, r) for h in range(H) for r in range(ref_scores.shape[1]) if not torch.equal(mask[h, r], ref_sel[h, r])]
    gaps = []
    for h, r in differ:
        assert pol.k_pick < pol.n_cand, (h, r)  # every candidate kept: nothing can swap
        top = torch.sort(ref_scores[h, r, :pol.n_cand], descending=True).values
        gaps.append(float(top[pol.k_pick - 1] - top[pol.k_pick]))
    print(f"{len(differ)} of {H * ref_scores.shape[1]} rows select differently from the oracle's fp32 scores; "
          f"max score error {err:.2e}, largest k-th/(k+1)-th gap among them {max(gaps, default=0.0):.2e}",
          flush=True)
    assert all(g <= 2 * err for g in gaps), (gaps, err)


@pytest.fixture(autouse=True)
def _clean():
    from dfsattn_amd import attention_hyvideo as hy
    from dfsattn_amd import attention_wan as wan
    for mod in (wan, hy):
        mod.DFS_Attention.clear_cache()
        mod._dfs_attention_instances.clear()
    yield


def test_wan_cfg0_shape_matches_oracle(dev):
    """configs[0] shape (1,024 tokens, 2 heads, d64, tile 16, sparsity 0.3),
    run in bf16 on the GPU (the native kernel takes bf16/f16, like
    block_sparse_attn); the oracle runs fp32 on the same bf16 values."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[0]
    q, k, v = synth_qkv(cfg, dtype=torch.bfloat16)
    perm = hilbert3d_perm(*cfg.grid)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=24, skip_steps=12, cache_interval=12,
                        layer_idx=3, sparsity=0.3, sparsity_dcrt=0.1, tile_size=16, video_perm=perm)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    ref, ref_mask, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, 0.3, 16)
    entry = DFS_Attention._cached_metadata[(3, "native", 128, 16, 16)]
    mask = entry["block_mask"].cpu()
    assert mask.shape == ref_mask.shape
    _assert_selection(mask, q, k, v, perm, 0.3, 16, ref_scores, dev)
    # output against the oracle attention on the GPU's own mask (fp32 reference)
    p, inv = orc.full_permutation(perm, q.shape[2])
    ref_own = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(out.cpu(), ref_own) < 4e-3  # includes the bf16 rounding of the output (~1.4e-3)
    assert float((out.cpu().float() - ref_own).abs().max()) < 2e-2


def test_wan_cache_reuses_mask_across_steps(dev):
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[0]
    q, k, v = (x.to(dev) for x in synth_qkv(cfg, dtype=torch.bfloat16))
    perm = hilbert3d_perm(*cfg.grid)
    kw = dict(skip_steps=12, cache_interval=12, layer_idx=1, sparsity=0.3, sparsity_dcrt=0.1, tile_size=16,
              video_perm=perm)
    dfs_attention(q, k, v, step_idx=24, **kw)  # refresh (real step 12)
    key = (1, "native", 128, 16, 16)
    first = DFS_Attention._cached_metadata[key]["col_idx"].clone()
    # uncond pass + later steps reuse the cached mask even for different inputs
    q2 = torch.flip(q, dims=[2])
    out_cached = dfs_attention(q2, k, v, step_idx=25, **kw)
    assert torch.equal(DFS_Attention._cached_metadata[key]["col_idx"], first)
    from dfsattn_amd import ops
    from dfsattn_amd.layout import ScoringLayout
    lay = ScoringLayout(q.shape[2], q.shape[2], 16)
    pd = ops.device_perm(perm, dev)
    prep = ops.prepare_qkv(q2, k, v, pd, lay, pool=False)
    ent = DFS_Attention._cached_metadata[key]
    direct = ops.bsa_fwd(prep, ent["row_ptr"], ent["col_idx"], out_perm=pd)
    assert torch.equal(out_cached, direct)
    # the next refresh (real step 24) recomputes with sparsity 0.2
    dfs_attention(q2, k, v, step_idx=48, **kw)
    assert DFS_Attention._cached_metadata[key]["policy"].k_pick == max(1, int(0.2 * 8))


def test_hunyuan_with_text_matches_oracle(dev):
    from dfsattn_amd.attention_hyvideo import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("hy-small", (3, 16, 20), 2, 128, torch.bfloat16, text_len=100, seed=9)
    q, k, v = synth_qkv(cfg)
    perm = hilbert3d_perm(*cfg.grid)
    L, vl = cfg.seq_len, cfg.video_len
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=12, skip_steps=12, cache_interval=12,
                        layer_idx=0, sparsity=0.5, sparsity_dcrt=0.1, tile_size=16, video_len=vl,
                        video_perm=perm)
    ref, ref_mask, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, 0.5, 16,
                                                            video_len=vl)
    key = next(iter(DFS_Attention._cached_metadata))
    mask = DFS_Attention._cached_metadata[key]["block_mask"].cpu()
    assert mask[:, :, vl // 128:].all() and mask[:, vl // 128:].all()
    _assert_selection(mask, q, k, v, perm, 0.5, 16, ref_scores, dev, video_len=vl)
    p, inv = orc.full_permutation(perm, L)
    ref_own = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(out.cpu(), ref_own) < 4e-3
    # text query rows attend to everything: equal to dense attention there
    dense = orc.dense_attention(q.float(), k.float(), v.float())
    text_rows = out.cpu()[:, :, vl:].float()
    assert _rel(text_rows, dense[:, :, vl:]) < 4e-3


def test_api_rejects_what_the_native_path_cannot_run(dev):
    from dfsattn_amd.attention_hyvideo import dfs_attention as hy_dfs
    from dfsattn_amd.attention_wan import dfs_attention

    q = torch.randn(1, 2, 256, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        dfs_attention(q, q, q, step_idx=100, sparse_execution="hybrid", tile_size=16)
    with pytest.raises(ValueError):
        dfs_attention(q, q, q, step_idx=100, sparse_execution="flashinfer64")
    with pytest.raises(RuntimeError):
        dfs_attention(q.float(), q.float(), q.float(), step_idx=100, layer_idx=7, tile_size=16)
    with pytest.raises(ValueError):
        hy_dfs(q, q, q, step_idx=30, layer_idx=2, tile_size=16, video_len=200, block_top_p=0.9)
    cu = torch.tensor([0, 100, 200, 256], dtype=torch.int32)
    with pytest.raises(NotImplementedError):  # more than two sequences
        hy_dfs(q, q, q, step_idx=30, layer_idx=4, tile_size=16, video_len=200, cu_seqlens_q=cu, cu_seqlens_kv=cu)
    with pytest.raises(NotImplementedError):  # ... also on the device (only the entry count is checked there)
        hy_dfs(q, q, q, step_idx=30, layer_idx=4, tile_size=16, video_len=200, cu_seqlens_q=cu.to(dev),
               cu_seqlens_kv=cu.to(dev))
    with pytest.raises(ValueError):  # different sequence counts for queries and keys
        hy_dfs(q, q, q, step_idx=30, layer_idx=4, tile_size=16, video_len=200,
               cu_seqlens_q=torch.tensor([0, 100, 256], dtype=torch.int32, device=dev),
               cu_seqlens_kv=torch.tensor([0, 256], dtype=torch.int32, device=dev) + 0)


@pytest.mark.parametrize("grid,text_len,pad,via", [((3, 16, 20), 100, 40, "valid"), ((4, 16, 16), 300, 230, "cu"),
                                                    ((4, 16, 16), 300, 172, "valid"), ((3, 16, 20), 100, 40, "device"),
                                                    ((4, 16, 16), 300, 230, "device"),
                                                    ((3, 16, 20), 100, 400, "device")])
def test_hunyuan_padding_segment_matches_oracle(dev, grid, text_len, pad, via):
    """cu_seqlens [0, valid, L] (text padding, replace_hyvideo.py:221-228):
    the mask is selected over the whole sequence, then the valid tokens and
    the padding tokens attend as two sequences under the same mask indexed
    from each one's start (attention_hyvideo.py:1054-1082). The valid length
    comes from flashinfer64_valid_sequence (as the processor passes it) or
    from host cu_seqlens."""
    from dfsattn_amd.attention_hyvideo import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("hy-pad", grid, 2, 128, torch.bfloat16, text_len=text_len, seed=11)
    q, k, v = synth_qkv(cfg)
    perm = hilbert3d_perm(*cfg.grid)
    L, vl = cfg.seq_len, cfg.video_len
    valid = L - pad
    cu = torch.tensor([0, valid, L], dtype=torch.int32)
    if via == "valid":  # the host valid length alone (no cu_seqlens)
        kw = dict(flashinfer64_valid_sequence=valid)
    elif via == "device":  # device cu_seqlens only: the split stays on the device
        kw = dict(cu_seqlens_q=cu.to(dev), cu_seqlens_kv=cu.to(dev))
    else:
        kw = dict(cu_seqlens_q=cu, cu_seqlens_kv=cu)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=12, skip_steps=12, cache_interval=12,
                        layer_idx=0, sparsity=0.5, sparsity_dcrt=0.1, tile_size=16, video_len=vl,
                        video_perm=perm, max_seqlen_q=valid, max_seqlen_kv=valid, **kw)
    key = next(iter(DFS_Attention._cached_metadata))
    mask = DFS_Attention._cached_metadata[key]["block_mask"].cpu()
    _, _, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, 0.5, 16, video_len=vl,
                                                   valid=valid)
    _assert_selection(mask, q, k, v, perm, 0.5, 16, ref_scores, dev, video_len=vl)
    p, inv = orc.full_permutation(perm, L)
    ref = orc.segment_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask, [0, valid, L])
    ref = ref[:, :, inv]
    got = out.cpu().float()
    assert _rel(got[:, :, :valid], ref[:, :, :valid]) < 4e-3
    assert _rel(got[:, :, valid:], ref[:, :, valid:]) < 4e-3
    assert float((got - ref).abs().max()) < 2e-2
    # the padding rows differ from what the single-sequence call gives them
    whole = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(got[:, :, valid:], whole[:, :, valid:]) > 0.05


@pytest.mark.parametrize("order", ["org", "morton", "blk", "hwf", "fwh", "hilbert2d"])
def test_wan_other_token_orders_match_oracle(dev, order):
    """Every --order of the drivers (wan21_t2v_inference.py:133-144,
    hyvideo_t2v_inference.py:243-254) through the same native path: the
    mask and output follow the oracle's whole call under that permutation
    ("org" passes no permutation)."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import video_perm_for
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("orders", (3, 16, 20), 2, 128, torch.bfloat16, seed=13)
    q, k, v = synth_qkv(cfg)
    perm = video_perm_for(order, *cfg.grid)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=24, skip_steps=12, cache_interval=12,
                        layer_idx=0, sparsity=0.3, sparsity_dcrt=0.1, tile_size=16, video_perm=perm)
    ref_perm = torch.arange(cfg.seq_len) if perm is None else perm
    _, _, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), ref_perm, 0.3, 16)
    mask = DFS_Attention._cached_metadata[(0, "native", 128, 16, 16)]["block_mask"].cpu()
    _assert_selection(mask, q, k, v, ref_perm, 0.3, 16, ref_scores, dev)
    p, inv = orc.full_permutation(ref_perm, cfg.seq_len)
    ref = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(out.cpu(), ref) < 4e-3
    assert float((out.cpu().float() - ref).abs().max()) < 2e-2


def test_records_and_mask_export_from_a_call(dev, tmp_path):
    """record_density, record_timing and configure_mask_export around one
    refresh call: the density is the kept fraction of the cached mask, the
    exported npy equals it, and the timing CSV counts one selection and one
    execution."""
    import csv

    import numpy as np
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[0]
    q, k, v = (x.to(dev) for x in synth_qkv(cfg, dtype=torch.bfloat16))
    DFS_Attention.configure_mask_export(str(tmp_path / "masks"), head_indices=(1,), layer_interval=3, save_bool=True)
    DFS_Attention.set_record_timing(True)
    try:
        dfs_attention(q, k, v, step_idx=24, skip_steps=12, cache_interval=12, layer_idx=3, sparsity=0.3,
                      sparsity_dcrt=0.1, tile_size=16, video_perm=hilbert3d_perm(*cfg.grid), record_density=True)
        mask = DFS_Attention._cached_metadata[(3, "native", 128, 16, 16)]["block_mask"].cpu()
        assert DFS_Attention.get_density_records()[24][3] == pytest.approx(float(mask.float().mean()))
        layer = tmp_path / "masks" / "step_024" / "layer_03"
        assert np.array_equal(np.load(layer / "block_mask.npy"), mask.numpy())
        assert (layer / "head_01_block_mask.png").exists()
        DFS_Attention.dump_timing_records(str(tmp_path / "timing.csv"))
        rows = {r["phase"]: r for r in csv.DictReader(open(tmp_path / "timing.csv"))}
        assert rows["top_k_selection"]["calls"] == "1" and rows["attention_execution"]["calls"] == "1"
        assert float(rows["attention_execution"]["total_ms"]) > 0
    finally:
        DFS_Attention.configure_mask_export(None)
        DFS_Attention.set_record_timing(False)
        DFS_Attention.set_record_density(False)


def test_default_path_keeps_inputs_beyond_f16(dev):
    """Default settings (f16 operands) with |v| and |q| far beyond the f16
    range in some heads: every finite bf16 input is carried (per-head powers
    of two, decided on the device), and the call matches the oracle's whole
    call on the same inputs."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("big", (4, 16, 16), 4, 128, torch.bfloat16, seed=5)
    q, k, v = (x.clone() for x in synth_qkv(cfg))
    v[:, 0] = (v[:, 0].float() * 2.0e5).to(torch.bfloat16)
    q[:, 1] = (q[:, 1].float() * 1.0e5).to(torch.bfloat16)
    v[:, 2, 100:140] = 7.0e4  # a few rows just past the f16 maximum
    q[:, 3] = (q[:, 3].float() * 3.0e5).to(torch.bfloat16)
    v[:, 3] = (v[:, 3].float() * 1.0e6).to(torch.bfloat16)
    perm = hilbert3d_perm(*cfg.grid)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=24, skip_steps=12, cache_interval=12,
                        layer_idx=5, sparsity=0.3, sparsity_dcrt=0.1, tile_size=16, video_perm=perm)
    assert bool(torch.isfinite(out).all())
    mask = DFS_Attention._cached_metadata[(5, "native", 128, 16, 16)]["block_mask"].cpu()
    _, _, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, 0.3, 16)
    _assert_selection(mask, q, k, v, perm, 0.3, 16, ref_scores, dev)
    p, inv = orc.full_permutation(perm, q.shape[2])
    ref = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    for h in range(4):
        assert _rel(out.cpu()[:, h], ref[:, h]) < 4e-3, h  # bf16 output


def test_wan_key_split_on_the_device(dev):
    """Wan's cu_seqlens_q [0, S, S] with cu_seqlens_kv [0, s_k, S] (the
    processor's form with an attention mask, replace_wan.py:246-250) as device
    tensors: every query attends only the first s_k keys (execution order)
    under the selected mask; no host read of the split."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("wan-split", (3, 16, 20), 2, 128, torch.bfloat16, seed=8)
    q, k, v = synth_qkv(cfg)
    S, s_k = cfg.seq_len, 700
    perm = hilbert3d_perm(*cfg.grid)
    cq = torch.tensor([0, S, S], dtype=torch.int32, device=dev)
    ck = torch.tensor([0, s_k, S], dtype=torch.int32, device=dev)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=24, skip_steps=12, cache_interval=12,
                        layer_idx=9, sparsity=0.5, sparsity_dcrt=0.0, tile_size=16, video_perm=perm,
                        cu_seqlens_q=cq, cu_seqlens_kv=ck, max_seqlen_q=S, max_seqlen_kv=S)
    mask = DFS_Attention._cached_metadata[(9, "native", 128, 16, 16)]["block_mask"].cpu()
    p, inv = orc.full_permutation(perm, S)
    ref = orc.varlen_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask,
                               [0, S, S], [0, s_k, S])[:, :, inv]
    got = out.cpu().float()
    assert _rel(got, ref) < 4e-3 and float((got - ref).abs().max()) < 2e-2
    whole = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(got, whole) > 0.05  # the key split changes the result


def test_dense_path_device_split_and_range(dev):
    """full_attention("flash") with device cu_seqlens [0, valid, L] and V
    beyond the f16 range: no host read of the split, the dense kernel keeps
    every finite input, and both sequences match fp32 attention."""
    from dfsattn_amd.fullattention import full_attention

    torch.manual_seed(12)
    L, valid = 700, 520
    q, k, v = (torch.randn(1, 2, L, 128) for _ in range(3))
    v[:, 1] *= 3.0e5
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    cu = torch.tensor([0, valid, L], dtype=torch.int32, device=dev)
    out = full_attention(q.to(dev), k.to(dev), v.to(dev), mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu)
    nb = math.ceil(L / 128)
    ref = orc.segment_attention(q.float(), k.float(), v.float(), torch.ones(2, nb, nb, dtype=torch.bool),
                                [0, valid, L])
    assert bool(torch.isfinite(out).all())
    for h in range(2):
        assert _rel(out.cpu()[:, h], ref[:, h]) < 4e-3, h


@pytest.mark.parametrize("grid,heads,d,dtype,sparsity", [
    ((1, 10, 10), 1, 64, torch.bfloat16, 0.3),     # 100 tokens: one partial block
    ((1, 3, 43), 2, 128, torch.float16, 0.3),      # 129 tokens: a last block of one token
    ((2, 16, 24), 2, 128, torch.bfloat16, 1.0),    # every block kept
    ((2, 16, 24), 3, 64, torch.bfloat16, 0.01),    # k = max(1, int(s * Kb)) = 1
])
def test_wan_edge_shapes_match_oracle(dev, grid, heads, d, dtype, sparsity):
    """dfs_attention at boundary sizes and sparsities against the oracle's
    whole call (mask from the oracle's fp32 scores, attention on the GPU's
    own mask)."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("edge", grid, heads, d, dtype, seed=11)
    q, k, v = synth_qkv(cfg)
    perm = hilbert3d_perm(*grid)
    print(f"edge case grid={grid} heads={heads} d={d} {dtype} s={sparsity}", flush=True)
    out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), step_idx=24, skip_steps=12, cache_interval=12,
                        layer_idx=7, sparsity=sparsity, sparsity_dcrt=0.0, tile_size=16, video_perm=perm)
    assert out.shape == q.shape and out.dtype == dtype
    mask = DFS_Attention._cached_metadata[(7, "native", 128, 16, 16)]["block_mask"].cpu()
    _, _, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, sparsity, 16)
    _assert_selection(mask, q, k, v, perm, sparsity, 16, ref_scores, dev)
    kb = mask.shape[-1]
    assert bool((mask.sum(-1) == max(1, int(sparsity * kb))).all())
    p, inv = orc.full_permutation(perm, q.shape[2])
    ref = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(out.cpu(), ref) < 4e-3
    assert float((out.cpu().float() - ref).abs().max()) < 2e-2


def test_bf16_operand_setting_through_the_call(dev):
    """DFS_Attention.operand_dtype = bf16 (the reference kernel's operand
    precision): the whole call and the dense path keep Q, K, V and P in
    bf16, select the same mask as the default call, and match fp32 attention
    on that mask within the bf16 operand class (P rounded to bf16: about
    1.5e-3 mean-rel, plus the bf16 output rounding)."""
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention
    from dfsattn_amd.fullattention import full_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    cfg = DfsConfig("bf16ops", (3, 16, 20), 2, 128, torch.bfloat16, seed=17)
    q, k, v = synth_qkv(cfg)
    perm = hilbert3d_perm(*cfg.grid)
    kw = dict(step_idx=24, skip_steps=12, cache_interval=12, sparsity=0.3, sparsity_dcrt=0.0, tile_size=16,
              video_perm=perm)
    default = dfs_attention(q.to(dev), k.to(dev), v.to(dev), layer_idx=0, **kw)
    mask_default = DFS_Attention._cached_metadata[(0, "native", 128, 16, 16)]["block_mask"].cpu()
    DFS_Attention.operand_dtype = torch.bfloat16
    try:
        out = dfs_attention(q.to(dev), k.to(dev), v.to(dev), layer_idx=1, **kw)
        dense = full_attention(q.to(dev), k.to(dev), v.to(dev), mode="flash",
                               operand_dtype=DFS_Attention.operand_dtype)
    finally:
        DFS_Attention.operand_dtype = None
    mask = DFS_Attention._cached_metadata[(1, "native", 128, 16, 16)]["block_mask"].cpu()
    assert torch.equal(mask, mask_default)  # scoring does not depend on the attention operands
    p, inv = orc.full_permutation(perm, q.shape[2])
    ref = orc.masked_attention(*(orc.apply_permutation(x.float(), p) for x in (q, k, v)), mask)[:, :, inv]
    assert out.dtype == torch.bfloat16 and not torch.equal(out, default)
    assert _rel(out.cpu(), ref) < 5e-3 and float((out.cpu().float() - ref).abs().max()) < 2e-2
    ref_dense = orc.dense_attention(q.float(), k.float(), v.float())
    assert _rel(dense.cpu(), ref_dense) < 5e-3


@pytest.mark.parametrize("variant,q_tile,k_tile", [("wan", 8, 64), ("wan", 128, 32), ("hunyuan", 64, 16),
                                                   ("hunyuan", 32, 4)])
def test_dfs_attention_class_with_unequal_tiles(dev, variant, q_tile, k_tile):
    """DFS_Attention with separate q_tile_size / k_tile_size (the class
    arguments, attention_wan.py:94-95, 192-203; attention_hyvideo.py:125-126):
    the cached mask is the oracle's selection over the GPU's fp32 scores, and
    the output matches the oracle's whole call."""
    from dfsattn_amd import ops
    from dfsattn_amd.layout import ScoringLayout, hunyuan_policy, wan_policy
    from dfsattn_amd.workloads import DfsConfig, synth_qkv

    text = 100 if variant == "hunyuan" else 0
    cfg = DfsConfig("t", (4, 16, 40), 2, 128, torch.bfloat16, text_len=text, seed=31)  # 2,560 video tokens
    q, k, v = synth_qkv(cfg)
    L, video = cfg.seq_len, cfg.video_len
    perm = torch.randperm(video, generator=torch.Generator().manual_seed(32))
    if variant == "wan":
        from dfsattn_amd.attention_wan import DFS_Attention
        att = DFS_Attention(step_idx=0, layer_idx=7, sparse_ratio=0.3, cache_flag=True, video_perm=perm,
                            q_tile_size=q_tile, k_tile_size=k_tile)
    else:
        from dfsattn_amd.attention_hyvideo import DFS_Attention
        att = DFS_Attention(step_idx=0, layer_idx=7, sparse_ratio=0.3, cache_flag=True, video_perm=perm,
                            video_len=video, q_tile_size=q_tile, k_tile_size=k_tile)
    out = att.forward(q.to(dev), k.to(dev), v.to(dev))
    ref, _, ref_scores = orc.dfs_attention_reference(q.float(), k.float(), v.float(), perm, 0.3, q_tile,
                                                     video_len=video if text else None, k_tile=k_tile)
    entry = next(iter(type(att)._cached_metadata.values()))
    mask = entry["block_mask"].cpu()
    # the GPU's own scores for this call, and the selection rule over them
    lay = ScoringLayout(L, video, q_tile, k_tile=k_tile)
    pol = hunyuan_policy(lay, 0.3) if text else wan_policy(lay, 0.3)
    full, inv = orc.full_permutation(perm, L)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ops.device_perm(full, dev), lay)
    _, scores, _ = ops.block_score_topk(prep, pol, torch.from_numpy(pol.row_ptr(2)).to(dev), want_scores=True)
    got = scores.cpu()
    assert torch.allclose(got, ref_scores, rtol=1e-5, atol=1e-10)
    sel = (orc.mask_from_scores_hunyuan(got, 0.3, L, video) if text else orc.mask_from_scores_wan(got, 0.3))
    assert torch.equal(mask, sel)
    ref_own = orc.masked_attention(*(orc.apply_permutation(x.float(), full) for x in (q, k, v)), mask)[:, :, inv]
    assert _rel(out.cpu(), ref_own) < 4e-3 and float((out.cpu().float() - ref_own).abs().max()) < 2e-2

"""Kernel-level parity of the HIP path against the CPU oracle (GPU only).

Bit-exact: permute gather/scatter, operand preparation, top-k from identical
fp32 scores. Tolerance: pooled tiles (hi+lo split, rel 2e-5), block scores
(rel 2e-3 against fp32), attention output in fp32 (max-abs 2e-2, mean-rel 1e-3
against fp32 masked-dense attention; mean-rel = mean|out - ref| / mean|ref|).
"""
import math

import numpy as np
import pytest
import torch

from dfsattn_amd import ops
from dfsattn_amd.layout import ScoringLayout, hunyuan_policy, wan_policy, dense_policy
from oracle import dfs_oracle as orc

pytestmark = pytest.mark.gpu


def _swap23(s):
    return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1)


def vt_reference(v_perm_padded: torch.Tensor, dtype) -> torch.Tensor:
    """[H, R, D] (execution order, zero rows past L) -> [H, R/128, D, 128]
    with tokens of each 16-group in swap23 order."""
    h, r, d = v_perm_padded.shape
    idx = torch.tensor([_swap23(s) for s in range(16)])
    x = v_perm_padded.view(h, r // 128, 8, 16, d)[:, :, :, idx, :]
    return x.reshape(h, r // 128, 128, d).transpose(2, 3).to(dtype).contiguous()


def mean_rel(out, ref):
    return float((out.double() - ref.double()).abs().mean() / ref.double().abs().mean())


@pytest.mark.parametrize("dtype,d,length,n", [
    (torch.bfloat16, 128, 67, 61),   # the reference's own Triton-permute test shape
    (torch.float32, 64, 1000, 1000),
    (torch.float16, 3, 257, 200),    # 6-byte rows: 2-byte vector path
])
def test_permute_gather_scatter_bit_exact(dev, dtype, d, length, n):
    torch.manual_seed(40)
    src = torch.randn((1, 3, length, d), dtype=dtype)
    perm = torch.randperm(n)
    perm_d = perm.to(dev, torch.int32)
    out = ops.permute_gather(src.to(dev), perm_d, rows=n + 5).cpu()
    assert torch.equal(out[:, :, :n], src[:, :, perm])
    assert torch.count_nonzero(out[:, :, n:]) == 0
    # inverse permutation: scatter of the gathered rows restores the source rows
    back = torch.zeros_like(src).to(dev)
    ops.permute_scatter(out[:, :, :n].contiguous().to(dev), perm_d, out=back)
    back = back.cpu()
    assert torch.equal(back[:, :, perm], src[:, :, perm])
    untouched = torch.ones(length, dtype=torch.bool)
    untouched[perm] = False
    assert torch.count_nonzero(back[:, :, untouched]) == 0


@pytest.mark.parametrize("case", ["wan_tail", "wan_even", "hunyuan_text", "hunyuan_no_text", "d64_tile32",
                                  "tile8", "d64_tile64", "q8_k64", "q128_k4_text", "d64_q64_k32", "no_q_operand"])
def test_prepare_qkv_matches_oracle(dev, case):
    heads, d, tile, dtype, pv = 2, 128, 16, torch.bfloat16, torch.float16
    k_tile = None
    q_operand = case != "no_q_operand"
    if case == "wan_tail":
        length, video = 1000, 1000
    elif case == "wan_even":
        length, video = 1024, 1024
    elif case == "hunyuan_text":
        length, video = 1000 + 60, 1000
    elif case == "hunyuan_no_text":
        length, video = 1000, 1000
    elif case == "tile8":  # tile sizes the scorer does not take are still prepared
        length, video, tile = 1000 + 40, 1000, 8
    elif case == "d64_tile64":
        length, video, d, tile = 900, 900, 64, 64
    elif case == "q8_k64":  # unequal query and key tiles (attention_wan.py:94-95)
        length, video, tile, k_tile = 1000, 1000, 8, 64
    elif case == "q128_k4_text":
        length, video, tile, k_tile = 1000 + 60, 1000, 128, 4
    elif case == "d64_q64_k32":
        length, video, d, tile, k_tile = 900, 900, 64, 64, 32
    elif case == "no_q_operand":  # Q only pooled (the attention kernel reads it from the input)
        length, video = 1000 + 60, 1000
    else:
        length, video, d, tile, pv = 777, 777, 64, 32, torch.bfloat16
    torch.manual_seed(7)
    q, k, v = (torch.randn((1, heads, length, d)).to(dtype) for _ in range(3))
    vperm = torch.randperm(video)
    perm, _ = orc.full_permutation(vperm, length)
    layout = ScoringLayout(length, video, tile, k_tile=k_tile)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), perm.to(dev, torch.int32), layout, operand_dtype=pv,
                           q_operand=q_operand)
    qp, kp, vp = (orc.apply_permutation(x, perm) for x in (q, k, v))
    R = layout.rows
    pad = lambda x: torch.cat([x[0], x.new_zeros(heads, R - length, d)], dim=1)
    assert prep.k_perm.dtype == pv  # f16 operands: exact bf16 -> f16 rounding
    if q_operand:
        assert prep.q_perm.dtype == pv and torch.equal(prep.q_perm.cpu(), pad(qp).to(pv))
    else:
        assert prep.q_perm is None and prep.q_src is not None
    assert torch.equal(prep.k_perm.cpu(), pad(kp).to(pv))
    assert torch.equal(prep.v_t.cpu(), vt_reference(pad(vp), pv))
    if prep.exps is not None:  # bf16 inputs inside the f16 range: no head is rescaled
        assert int(prep.exps.abs().sum().item()) == 0
    qt, kt = orc.pooled_tiles(qp, kp, tile, 128, video, k_tile=k_tile)
    for hi, lo, ref in ((prep.q_hi, prep.q_lo, qt[0]), (prep.k_hi, prep.k_lo, kt[0])):
        got = hi.cpu().float() + lo.cpu().float()
        assert got.shape == ref.shape
        assert torch.allclose(got, ref, rtol=2e-5, atol=1e-6), float((got - ref).abs().max())


def test_prepare_rescales_heads_beyond_f16(dev):
    """bf16 inputs rounded to f16 operands: a head holding a finite value
    beyond the f16 range is stored as x * 2^-e, e the smallest exponent with
    max|x| * 2^-e < 2^15 (1e6 = 2^19.93 -> e = 5), bit-exactly; every other
    head keeps plain rounding and exponent 0. bf16 operands keep the bits and
    carry no exponents."""
    heads, length, d = 3, 300, 64
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32, device=dev)
    for which in range(3):
        qkv = [torch.randn((1, heads, length, d)).to(torch.bfloat16) for _ in range(3)]
        qkv[which][0, 1, 123, 7] = 1.0e6
        prep = ops.prepare_qkv(*(x.to(dev) for x in qkv), ident, layout, pool=False)
        exps = prep.exps.cpu()
        want = torch.zeros(3, heads, dtype=torch.int32)
        want[which, 1] = 5
        assert torch.equal(exps, want), (which, exps)
        R = layout.rows
        scaled = [x[0].float() for x in qkv]
        scaled[which][1] *= 2.0 ** -5
        for t, got in enumerate((prep.q_perm, prep.k_perm)):
            ref = torch.cat([scaled[t].to(torch.float16), torch.zeros(heads, R - length, d, dtype=torch.float16)], 1)
            assert torch.equal(got.cpu(), ref), (which, t)
        pad = torch.cat([scaled[2], scaled[2].new_zeros(heads, R - length, d)], 1)
        assert torch.equal(prep.v_t.cpu(), vt_reference(pad, torch.float16)), which
        keep = ops.prepare_qkv(*(x.to(dev) for x in qkv), ident, layout, operand_dtype=torch.bfloat16, pool=False)
        assert keep.exps is None
        assert torch.equal(keep.q_perm.cpu()[:, :length], qkv[0][0])


@pytest.mark.parametrize("pv", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("q_operand", [True, False])
def test_bsa_fwd_keeps_inputs_beyond_f16(dev, pv, q_operand):
    """Heads with q, k or v beyond the f16 range (q * scale * log2(e) beyond
    it too, so rows carry their own power of two) against fp32 masked
    attention of the same bf16 inputs."""
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads, d, length = 4, 128, 1000
    cfg = DfsConfig("big", (1, 1, length), heads, d, torch.bfloat16, seed=31)
    q, k, v = (x.clone() for x in synth_qkv(cfg))
    v[:, 0] = (v[:, 0].float() * 3.0e5).to(torch.bfloat16)        # V beyond f16
    k[:, 1] = (k[:, 1].float() * 2.0e5).to(torch.bfloat16)        # K beyond f16
    q[:, 2] = (q[:, 2].float() * 1.0e6).to(torch.bfloat16)        # Q, and Q * c, beyond f16
    q[:, 3, :500] = (q[:, 3, :500].float() * 4.0e5).to(torch.bfloat16)  # only some rows of a head
    k[:, 3] = (k[:, 3].float() * 1.0e2).to(torch.bfloat16)
    g = torch.Generator().manual_seed(32)
    nb = math.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=g) < 0.5
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32, device=dev)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ident, layout, operand_dtype=pv, pool=False,
                           q_operand=q_operand)
    row_ptr, col_idx = ops.mask_to_csr(mask.to(dev))
    got = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=torch.float32).cpu()
    ref = orc.masked_attention(q, k, v, mask)
    assert bool(torch.isfinite(got).all())
    for h in range(heads):
        rel = mean_rel(got[:, h], ref[:, h])
        print(f"head {h} ({pv}): mean-rel {rel:.2e}", flush=True)
        assert rel <= (1e-3 if pv == torch.float16 else 3e-3), h


def _random_scores(heads, rows, cols, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    s = torch.rand((heads, rows, cols), generator=g)
    if ties:
        s = torch.round(s * 8) / 8  # many exact ties, some straddling the k-th place
    return s


@pytest.mark.parametrize("cols,ratio,ties", [(591, 0.3, False), (8, 0.3, False), (100, 0.05, True),
                                             (931, 0.3, True), (2048, 0.5, False)])
def test_topk_from_scores_wan_bit_exact(dev, cols, ratio, ties):
    layout = ScoringLayout(cols * 128 - 7, cols * 128 - 7, 16)
    pol = wan_policy(layout, ratio)
    heads = 3
    scores = _random_scores(heads, pol.scored_rows, pol.k_blocks, cols, ties)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    col_idx, mask = ops.topk_from_scores(scores.to(dev), pol, row_ptr, want_mask=True)
    want = orc.mask_from_scores_wan(scores, ratio)
    assert torch.equal(mask.cpu().bool(), want)
    # CSR lists ascending columns of the same set
    got = ops.csr_to_mask(row_ptr, col_idx, heads, pol.q_blocks, pol.k_blocks).cpu()
    assert torch.equal(got, want)
    cols_np = col_idx.cpu().numpy().reshape(heads * pol.q_blocks, pol.k_pick)
    assert (np.diff(cols_np, axis=1) > 0).all()
    # the reference's literal torch.topk + scatter_ selects the same set on every
    # row where no tie straddles the k-th place
    clean = ~orc.boundary_ties(scores, pol.k_pick)
    assert torch.equal(want[clean], orc.mask_from_scores_torch(scores, pol.k_pick)[clean])


@pytest.mark.parametrize("video,text,ratio", [(118800, 256, 0.3), (1000, 60, 0.5),
                                              (1000, 0, 0.3), (1024, 0, 0.3), (3000, 256, 0.2)])
def test_topk_from_scores_hunyuan_policy(dev, video, text, ratio):
    layout = ScoringLayout(video + text, video, 16)
    pol = hunyuan_policy(layout, ratio)
    heads = 2
    scores = _random_scores(heads, pol.scored_rows, pol.k_blocks, video)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    col_idx, mask = ops.topk_from_scores(scores.to(dev), pol, row_ptr, want_mask=True)
    want = orc.mask_from_scores_hunyuan(scores, ratio, video + text, video)
    assert torch.equal(mask.cpu().bool(), want)
    assert torch.equal(ops.csr_to_mask(row_ptr, col_idx, heads, pol.q_blocks, pol.k_blocks).cpu(), want)


@pytest.mark.parametrize("d,tile,video,text,heads,k_tile", [
    (128, 16, 4 * 16 * 16, 0, 2, None), (128, 16, 3 * 20 * 21, 0, 2, None), (64, 16, 4 * 16 * 16, 0, 2, None),
    (128, 32, 2000, 0, 2, None), (128, 16, 2000, 100, 2, None), (64, 32, 1500, 100, 2, None),
    (128, 16, 20 * 128 + 16, 120, 2, None),  # last scored row dense, alone in its group
    (128, 16, 3000, 0, 8, None), (128, 16, 2000, 100, 16, None),  # heads divisible by 8: whole heads per XCD
    # the generic scorer: every other tile size, equal or not (attention_wan.py:94-95, 227-246)
    (128, 8, 2000, 0, 2, 8), (128, 64, 2000, 0, 2, 64), (128, 128, 2000, 100, 2, 128), (128, 4, 1000, 0, 2, 4),
    (128, 8, 2000, 0, 3, 64), (128, 64, 2000, 0, 2, 8), (128, 16, 2000, 100, 2, 32), (128, 32, 1500, 0, 2, 16),
    (64, 128, 1500, 100, 2, 4), (64, 4, 1000, 0, 2, 128), (128, 16, 2000, 100, 2, 8)])
def test_block_score_topk_matches_oracle(dev, d, tile, video, text, heads, k_tile):
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    cfg = DfsConfig("t", (1, 1, video), heads, d, torch.bfloat16, text_len=text, tile=tile, seed=3)
    q, k, v = synth_qkv(cfg)
    length = video + text
    print(f"scoring case d={d} tiles={tile}/{k_tile} video={video} text={text} heads={heads}", flush=True)
    perm, _ = orc.full_permutation(torch.randperm(video, generator=torch.Generator().manual_seed(5)), length)
    layout = ScoringLayout(length, video, tile, k_tile=k_tile)
    pol = wan_policy(layout, 0.3) if text == 0 else hunyuan_policy(layout, 0.3)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), perm.to(dev, torch.int32), layout)
    col_idx, scores, mask = ops.block_score_topk(prep, pol, row_ptr, want_scores=True, want_mask=True)
    qp, kp = orc.apply_permutation(q, perm), orc.apply_permutation(k, perm)
    ref = orc.block_scores(qp, kp, tile, 128, video if text else None, k_tile=k_tile)
    got = scores.cpu()
    assert got.shape == ref.shape
    err = (got.double() - ref.double()).abs()
    print(f"  score error: max abs {float(err.max()):.3g}, max rel {float((err / ref.double().abs().clamp_min(1e-30)).max()):.3g},"
          f" max rel above 1e-3 {float((err / ref.double().abs())[ref > 1e-3].max()):.3g}", flush=True)
    # measured: at most 4e-7 relative on every entry (hi/lo-split products)
    assert torch.allclose(got, ref, rtol=1e-5, atol=1e-10), float((got - ref).abs().max())
    # every scored row of the block scores sums to block/tile
    assert torch.allclose(got.sum(-1), torch.full_like(got.sum(-1), 128 / tile), rtol=1e-4)
    # the fused top-k equals the oracle's selection on the same fp32 scores
    sel = orc.mask_from_scores_wan(got, 0.3) if text == 0 else \
        orc.mask_from_scores_hunyuan(got, 0.3, length, video)
    assert torch.equal(mask.cpu().bool(), sel)
    assert torch.equal(ops.csr_to_mask(row_ptr, col_idx, heads, pol.q_blocks, pol.k_blocks).cpu(), sel)
    # and agrees with the oracle's own fp32 mask wherever the k-th and
    # (k+1)-th oracle scores of a row are further apart than twice the
    # measured score error
    ref_sel = orc.mask_from_scores_wan(ref, 0.3) if text == 0 else \
        orc.mask_from_scores_hunyuan(ref, 0.3, length, video)
    err = float((got - ref).abs().max())
    for h in range(heads):
        for r in range(ref.shape[1]):
            if not torch.equal(sel[h, r], ref_sel[h, r]):
                top = torch.sort(ref[h, r, :pol.n_cand], descending=True).values
                assert float(top[pol.k_pick - 1] - top[pol.k_pick]) <= 2 * err, (h, r, err)


@pytest.mark.parametrize("video,text", [(4 * 16 * 16 * 4, 0), (2000, 100)])
def test_block_score_topk_lds_sums_path_selects_the_same(dev, video, text):
    """dfs_block_score_topk without a score matrix keeps its block sums in
    LDS; its selection equals the two-pass global-sums path's (the same
    arithmetic), and the one-pass path's scores agree with both to fp32
    rounding."""
    import ctypes
    from dfsattn_amd import _lib
    from dfsattn_amd.ops import _policy_args
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads = 3
    cfg = DfsConfig("t", (1, 1, video), heads, 128, torch.bfloat16, text_len=text, seed=6)
    q, k, v = synth_qkv(cfg)
    length = video + text
    perm, _ = orc.full_permutation(torch.randperm(video, generator=torch.Generator().manual_seed(2)), length)
    layout = ScoringLayout(length, video, 16)
    pol = wan_policy(layout, 0.3) if text == 0 else hunyuan_policy(layout, 0.3)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), perm.to(dev, torch.int32), layout)
    col_global, scores2, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True, one_pass=False)
    col_lds = torch.empty_like(col_global)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.call("dfs_block_score_topk", p(prep.q_hi), p(prep.q_lo), p(prep.k_hi), p(prep.k_lo), heads, 128, 16, 16,
              *_policy_args(pol), p(row_ptr), p(col_lds), None, None, None, 0,
              ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert torch.equal(col_lds.cpu(), col_global.cpu())
    _, scores1, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True, one_pass=True)
    torch.testing.assert_close(scores1.cpu(), scores2.cpu(), rtol=2e-5, atol=1e-7)


def test_block_score_topk_workspace_checks(dev):
    """The one-pass form needs a large enough, aligned workspace; the score
    matrix is optional there, and the selection is the same without it."""
    import ctypes
    from dfsattn_amd import _lib
    from dfsattn_amd.ops import _policy_args, score_workspace_bytes
    heads, length = 2, 1000
    q = torch.randn(1, heads, length, 64).bfloat16().to(dev)
    layout = ScoringLayout(length, length, 16)
    pol = wan_policy(layout, 0.3)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    prep = ops.prepare_qkv(q, q, q, torch.arange(length, dtype=torch.int32, device=dev), layout)
    need = score_workspace_bytes(heads, 16, 16, pol.q_blocks, pol.k_blocks)
    # rows of 16 query blocks per workgroup x 8 tiles, key blocks padded to 32-tile chunks
    assert need == heads * 16 * 8 * 8 * 4
    ws = torch.empty(need // 4 + 4, dtype=torch.float32, device=dev)
    col = torch.empty(pol.nnz(heads), dtype=torch.int32, device=dev)
    scores = torch.empty((heads, pol.scored_rows, pol.k_blocks), dtype=torch.float32, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    args = (p(prep.q_hi), p(prep.q_lo), p(prep.k_hi), p(prep.k_lo), heads, 64, 16, 16, *_policy_args(pol), p(row_ptr),
            p(col))
    for sc, w, nbytes in ((p(scores), p(ws), need - 4), (p(scores), ctypes.c_void_p(ws.data_ptr() + 4), need)):
        with pytest.raises(_lib.DfsKernelError):
            _lib.call("dfs_block_score_topk", *args, sc, None, w, nbytes, stream)
    _lib.call("dfs_block_score_topk", *args, p(scores), None, p(ws), need, stream)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(scores).all())
    with_scores = col.clone()
    col.fill_(-1)
    _lib.call("dfs_block_score_topk", *args, None, None, p(ws), need, stream)
    torch.cuda.synchronize()
    assert torch.equal(col, with_scores)


@pytest.mark.parametrize("heads,length,text", [(2, 3000, 0), (8, 2000, 0), (2, 2000, 100)])
def test_block_score_topk_all_tied_keeps_lowest_columns(dev, heads, length, text):
    """Q = 0 makes every logit 0, so every scored block sums exactly the same
    (its 64 tile pairs of 1/Z each): the top-k is one big tie, and the fused
    selection (one-pass and two-pass forms, whole heads per XCD at 8 heads)
    keeps the lowest candidate columns, as a stable descending sort does."""
    video = length - text
    q = torch.zeros(1, heads, length, 128, dtype=torch.bfloat16, device=dev)
    k = torch.randn(1, heads, length, 128, generator=torch.Generator().manual_seed(4)).bfloat16().to(dev)
    layout = ScoringLayout(length, video, 16)
    pol = wan_policy(layout, 0.3) if text == 0 else hunyuan_policy(layout, 0.3)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    prep = ops.prepare_qkv(q, k, k, torch.arange(length, dtype=torch.int32, device=dev), layout)
    want = torch.zeros((heads, pol.q_blocks, pol.k_blocks), dtype=torch.bool)
    want[:, :pol.dense_row, :pol.k_pick] = True
    want[:, :pol.dense_row, pol.dense_col:] = True
    want[:, pol.dense_row:] = True
    for one_pass in (True, False):
        _, scores, mask = ops.block_score_topk(prep, pol, row_ptr, want_scores=True, want_mask=True,
                                               one_pass=one_pass)
        got = scores.cpu()[:, :min(pol.scored_rows, pol.dense_row), :pol.n_cand]
        assert bool((got == got[0, 0, 0]).all())  # one tie over every candidate
        assert torch.equal(mask.cpu().bool(), want), one_pass


@pytest.mark.parametrize("direction", ["rising", "falling"])
@pytest.mark.parametrize("tile,one_pass", [(16, True), (32, True), (16, False), (32, False)])
def test_block_scores_with_far_apart_logits(dev, direction, tile, one_pass):
    """Key tiles whose logits rise (or fall) by ~130 log2 units across the
    row: the scoring pass's reference (the first chunk's maximum) has to
    move for rising logits (in the one-pass form, rescaling the block sums
    already stored) and stays for falling ones; every form matches the fp32
    softmax of the oracle."""
    length, d = 2048, 128
    ramp = torch.linspace(0.0, 8.0, length)
    if direction == "falling":
        ramp = ramp.flip(0)
    q = torch.ones(1, 1, length, d).bfloat16()
    k = (ramp[None, None, :, None] * torch.ones(1, 1, length, d)).bfloat16()
    v = torch.zeros_like(q)
    layout = ScoringLayout(length, length, tile)
    pol = wan_policy(layout, 0.3)
    row_ptr = torch.from_numpy(pol.row_ptr(1)).to(dev)
    ident = torch.arange(length, dtype=torch.int32)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ident.to(dev), layout)
    _, scores, _ = ops.block_score_topk(prep, pol, row_ptr, want_scores=True, one_pass=one_pass)
    ref = orc.block_scores(q.float(), k.float(), tile, 128, None)
    got = scores.cpu()
    assert bool(torch.isfinite(got).all())
    err = (got.double() - ref.double()).abs()
    print(f"far-apart logits {direction} tile={tile} one_pass={one_pass}: max abs {float(err.max()):.3g}, "
          f"max rel above 1e-6 {float((err / ref.double().abs())[ref > 1e-6].max()):.3g}", flush=True)
    assert torch.allclose(got, ref, rtol=1e-4, atol=1e-9), float((got - ref).abs().max())


def _run_bsa(dev, q, k, v, mask_bool, pv, out_dtype, perm=None, scale=None):
    heads, length, d = q.shape[1], q.shape[2], q.shape[3]
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ident.to(dev), layout, operand_dtype=pv, pool=False)
    row_ptr, col_idx = ops.mask_to_csr(mask_bool.to(dev))
    out = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=out_dtype, scale=scale,
                      out_perm=None if perm is None else perm.to(dev, torch.int32))
    return out.cpu()


SCALES = (None, 0.6)  # the softmax scale: default D^-1/2, and one that sends every head to the scaled instance


@pytest.mark.parametrize("scale", SCALES)
@pytest.mark.parametrize("d,length,density,pv", [
    (128, 1000, 0.3, torch.float16), (128, 1024, 0.5, torch.float16), (64, 1000, 0.3, torch.float16),
    (128, 3000, 0.3, torch.float16), (128, 1000, 1.0, torch.float16), (128, 1000, 0.3, torch.bfloat16),
    (64, 130, 1.0, torch.float16), (128, 1100, 0.3, torch.float16), (64, 1400, 0.2, torch.bfloat16)])
def test_bsa_fwd_matches_masked_dense(dev, scale, d, length, density, pv):
    """The attention kernel against fp32 masked attention, at the default
    softmax scale and at one large enough that every head runs in the scaled
    instance (rows carrying their own powers of two)."""
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads = 2
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.bfloat16, seed=11)
    q, k, v = synth_qkv(cfg)
    nb = math.ceil(length / 128)
    g = torch.Generator().manual_seed(12)
    mask = torch.rand((heads, nb, nb), generator=g) < density
    mask[:, torch.arange(nb), torch.arange(nb)] = True  # no empty rows
    out = _run_bsa(dev, q, k, v, mask, pv, torch.float32, scale=scale)
    ref = orc.masked_attention(q, k, v, mask, scale=scale)
    max_abs = float((out - ref).abs().max())
    mr = mean_rel(out, ref)
    tol = 1e-3 if pv == torch.float16 else 3e-3  # bf16 P: reference-kernel precision class
    assert max_abs <= 2e-2 and mr <= tol, (max_abs, mr)
    if density == 1.0:
        dense = orc.dense_attention(q, k, v, scale=scale)
        assert mean_rel(out, dense) <= tol


@pytest.mark.parametrize("length", [127, 129, 255, 257, 383, 641])
@pytest.mark.parametrize("heads,d", [(1, 128), (3, 64), (5, 128)])
def test_bsa_fwd_ragged_lengths(dev, length, heads, d):
    """Lengths just under and over multiples of the 128-token block (the
    last block's keys masked, its rows dropped) with odd head counts, at the
    output contract on fp32 output."""
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.bfloat16, seed=length + heads)
    q, k, v = synth_qkv(cfg)
    nb = math.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=torch.Generator().manual_seed(length)) < 0.5
    mask[:, :, nb - 1] = True  # every row sees the partial block
    out = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32)
    ref = orc.masked_attention(q, k, v, mask)
    assert out.shape == ref.shape
    assert float((out - ref).abs().max()) <= 2e-2 and mean_rel(out, ref) <= 1e-3


def test_bsa_fwd_bf16_out_and_fused_unpermute(dev):
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads, d, length = 2, 128, 1000
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.bfloat16, seed=13)
    q, k, v = synth_qkv(cfg)
    nb = math.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=torch.Generator().manual_seed(2)) < 0.4
    mask[:, :, 0] = True
    perm = torch.randperm(length, generator=torch.Generator().manual_seed(3))
    out32 = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32)
    out16 = _run_bsa(dev, q, k, v, mask, torch.float16, torch.bfloat16)
    assert torch.equal(out16, out32.to(torch.bfloat16))
    scat = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32, perm=perm)
    assert torch.equal(scat[:, :, perm], out32)


@pytest.mark.parametrize("scale", SCALES)
def test_empty_rows_give_zero(dev, scale):
    heads, d, length = 1, 128, 512
    q, k, v = (torch.randn((1, heads, length, d)).to(torch.bfloat16) for _ in range(3))
    mask = torch.zeros((heads, 4, 4), dtype=torch.bool)
    mask[0, 0, 1] = True
    out = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32, scale=scale)
    assert torch.count_nonzero(out[:, :, 128:]) == 0
    ref = orc.masked_attention(q, k, v, mask, scale=scale)
    assert mean_rel(out[:, :, :128], ref[:, :, :128]) < 1e-3


@pytest.mark.parametrize("scale", SCALES)
def test_rows_keeping_only_a_short_tail_block(dev, scale):
    """The last block holds 26 keys: a wave whose keys of that block are all
    masked, and which has seen no other key, must contribute nothing."""
    heads, d, length = 2, 128, 1050
    q, k, v = (torch.randn((1, heads, length, d), generator=torch.Generator().manual_seed(s)).to(torch.bfloat16)
               for s in (21, 22, 23))
    nb = math.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=torch.Generator().manual_seed(24)) < 0.3
    mask[:, 0] = False
    mask[:, 0, nb - 1] = True   # only the tail block
    mask[:, 1] = False
    mask[:, 1, 3] = True
    mask[:, 1, nb - 1] = True
    mask[:, nb - 1] = False
    mask[:, nb - 1, nb - 1] = True
    out = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32, scale=scale)
    assert torch.isfinite(out).all()
    ref = orc.masked_attention(q, k, v, mask, scale=scale)
    assert float((out - ref).abs().max()) <= 2e-2 and mean_rel(out, ref) <= 1e-3


@pytest.mark.parametrize("scale", SCALES)
def test_bsa_fwd_rising_and_negative_logits(dev, scale):
    """Logits that grow block after block (the running maximum jumps by far
    more than the lazy-rescale threshold several times) and rows whose
    logits are all strongly negative: the output still equals fp32 masked
    attention."""
    heads, d, length = 2, 128, 1200
    g = torch.Generator().manual_seed(21)
    q = torch.randn((1, heads, length, d), generator=g)
    k = torch.randn((1, heads, length, d), generator=g)
    v = torch.randn((1, heads, length, d), generator=g)
    nb = math.ceil(length / 128)
    ramp = torch.linspace(0.2, 3.0, nb).repeat_interleave(128)[:length]
    k = k * ramp[None, None, :, None]          # later key blocks give much larger |logits|
    q[:, 1] = -q[:, 1].abs()                   # head 1: many large negative logits
    k[:, 1] = k[:, 1].abs()
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    mask = torch.rand((heads, nb, nb), generator=g) < 0.6
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    out = _run_bsa(dev, q, k, v, mask, torch.float16, torch.float32, scale=scale)
    ref = orc.masked_attention(q, k, v, mask, scale=scale)
    assert torch.isfinite(out).all()
    assert float((out - ref).abs().max()) <= 2e-2 and mean_rel(out, ref) <= 1e-3, \
        (float((out - ref).abs().max()), mean_rel(out, ref))


def test_wrappers_reject_bad_index_operands(dev):
    """Index operands must be contiguous int32 on the operands' device, and
    CSR offsets must cover every (head, query block) row: checked on the host
    before any launch."""
    length, heads = 300, 2
    q = torch.randn(1, heads, length, 64).bfloat16().to(dev)
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        ops.prepare_qkv(q, q, q, ident.long(), layout)
    with pytest.raises(ValueError):
        ops.permute_gather(q, ident.long())
    prep = ops.prepare_qkv(q, q, q, ident, layout)
    pol = wan_policy(layout, 0.5)
    row_ptr = torch.from_numpy(pol.row_ptr(heads)).to(dev)
    col_idx, _, _ = ops.block_score_topk(prep, pol, row_ptr)
    with pytest.raises(ValueError):
        ops.bsa_fwd(prep, row_ptr.long(), col_idx)
    with pytest.raises(ValueError):
        ops.bsa_fwd(prep, row_ptr[:-1].contiguous(), col_idx)
    with pytest.raises(ValueError):
        ops.bsa_fwd(prep, row_ptr, col_idx, out_perm=ident.long())
    with pytest.raises(ValueError):
        ops.block_score_topk(prep, pol, row_ptr[1:].contiguous())
    with pytest.raises(ValueError):
        ops.csr_to_mask(row_ptr, col_idx.long(), heads, pol.q_blocks, pol.k_blocks)
    with pytest.raises(RuntimeError):
        ops.bsa_fwd(prep, row_ptr.cpu(), col_idx)
    # the valid call still runs after the rejections
    out = ops.bsa_fwd(prep, row_ptr, col_idx, out_perm=ident)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())


@pytest.mark.parametrize("length,cu_q,cu_k", [
    (1300, [0, 1100, 1300], [0, 1100, 1300]),   # text padding: two sequences, blocks from each start
    (1300, [0, 1152, 1300], [0, 1152, 1300]),   # a split on a block boundary
    (1000, [0, 130, 1000], [0, 130, 1000]),     # a long second sequence
    (1000, [0, 1, 1000], [0, 1, 1000]),         # a one-token first sequence
    (1000, [0, 1000, 1000], [0, 700, 1000]),    # Wan's [0, S, S] / [0, s_k, S]: keys past s_k unused
    (1000, [0, 600, 900], [0, 500, 1000]),      # unequal splits; rows 900.. in no sequence
    (1000, [0, 1000], [0, 1000]),               # one sequence given explicitly
    (900, [0, 0, 900], [0, 0, 900]),            # an empty first sequence
])
def test_bsa_fwd_varlen_matches_oracle(dev, length, cu_q, cu_k):
    """Device cu_seqlens (block_sparse_attn_func's varlen arguments): sequence
    i's queries attend its keys under the mask indexed from each sequence's
    start; rows in no query sequence are zero; the offsets are never read on
    the host. Against the fp32 varlen oracle, which tests pin to dense
    attention under explicit token masks."""
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads, d = 2, 128
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.bfloat16, seed=21)
    q, k, v = synth_qkv(cfg)
    nb = math.ceil(length / 128)
    g = torch.Generator().manual_seed(22)
    mask = torch.rand((heads, nb, nb), generator=g) < 0.4
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ident.to(dev), layout, pool=False)
    row_ptr, col_idx = ops.mask_to_csr(mask.to(dev))
    out = torch.full((1, heads, length, d), 7.0, dtype=torch.float32, device=dev)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    _, lse = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=torch.float32, out=out, cu_seqlens_q=cq,
                         cu_seqlens_k=ck, want_lse=True)
    got = out.cpu()
    ref = orc.varlen_attention(q, k, v, mask, cu_q, cu_k)
    assert float((got - ref).abs().max()) <= 2e-2 and mean_rel(got, ref) <= 1e-3
    covered = torch.zeros(length, dtype=torch.bool)
    for (q0, q1), (k0, k1) in zip(zip(cu_q, cu_q[1:]), zip(cu_k, cu_k[1:])):
        if k1 > k0:
            covered[q0:q1] = True
    assert bool((got[:, :, ~covered] == 0).all())
    assert bool(torch.isneginf(lse.cpu()[:, ~covered]).all())
    assert bool(torch.isfinite(lse.cpu()[:, covered]).all())


@pytest.mark.parametrize("length,cu_q,cu_k,far_rows", [
    (1000, [0, 1000, 1000], [0, 300, 1000], True),   # some rows keep only key blocks past cu_k[1]
    (1000, [0, 600, 1000], [0, 0, 1000], False),     # a first sequence with queries and no keys
    (1000, [0, 600, 901], [0, 600, 901], False),     # the second sequence ends inside a row group
    (1000, [0, 600, 901], [0, 500, 1000], True),     # both at once
])
def test_bsa_fwd_varlen_rows_without_keys(dev, length, cu_q, cu_k, far_rows):
    """Rows of a sequence whose kept blocks all lie past that sequence's keys
    (or whose sequence has no keys) are zero with lse -inf; a four-row group
    of the second-sequence kernel that straddles the sequence's end writes
    its rows past the end as zero. Against the fp32 varlen oracle."""
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads, d = 3, 128
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.bfloat16, seed=23)
    q, k, v = synth_qkv(cfg)
    nb = math.ceil(length / 128)
    g = torch.Generator().manual_seed(24)
    mask = torch.rand((heads, nb, nb), generator=g) < 0.4
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    if far_rows:
        # rows 0..2 of every head keep only blocks 3.. (past 300 keys)
        mask[:, :3, :3] = False
        mask[:, :3, 5] = True
    layout = ScoringLayout(length, length, 16)
    ident = torch.arange(length, dtype=torch.int32)
    prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), ident.to(dev), layout, pool=False)
    row_ptr, col_idx = ops.mask_to_csr(mask.to(dev))
    out = torch.full((1, heads, length, d), 7.0, dtype=torch.float32, device=dev)
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    _, lse = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=torch.float32, out=out, cu_seqlens_q=cq,
                         cu_seqlens_k=ck, want_lse=True)
    got, lse = out.cpu(), lse.cpu()
    ref = orc.varlen_attention(q, k, v, mask, cu_q, cu_k)
    assert float((got - ref).abs().max()) <= 2e-2 and mean_rel(got, ref) <= 1e-3
    live = torch.zeros((heads, length), dtype=torch.bool)
    for (q0, q1), (k0, k1) in zip(zip(cu_q, cu_q[1:]), zip(cu_k, cu_k[1:])):
        nkb = math.ceil((k1 - k0) / 128)
        for r in range(q0, q1):
            live[:, r] = mask[:, (r - q0) // 128, :nkb].any(-1) if nkb > 0 else False
    assert bool((~live).any()), "the case must hold rows without keys"
    assert bool((got[0][~live] == 0).all())
    assert bool(torch.isneginf(lse[~live]).all())
    assert bool(torch.isfinite(lse[live]).all())


@pytest.mark.parametrize("case", ["bf16_d128", "f16_d64", "bf16_operands", "varlen", "q_beyond_f16"])
def test_bsa_fwd_q_source_matches_q_perm(dev, case):
    """dfs_bsa_fwd reading Q from the input through the permutation (q_src,
    q_rows; dfs_prepare_qkv then writes no q_perm) against the same call on
    the prepared q_perm and against fp32 masked attention: the two differ by
    the rounding of Q * scale * log2(e) to f16 only (one rounding from the
    input instead of two), and the second-sequence and scaled instances read
    the same source."""
    import math as _m
    from dfsattn_amd.workloads import DfsConfig, synth_qkv
    heads, d, length, dtype, pv = 3, 128, 1100, torch.bfloat16, torch.float16
    cu = None
    if case == "f16_d64":
        d, dtype = 64, torch.float16
    elif case == "bf16_operands":
        pv = torch.bfloat16
    elif case == "varlen":
        cu = [0, 900, length]
    cfg = DfsConfig("t", (1, 1, length), heads, d, torch.float32, seed=41)
    q, k, v = synth_qkv(cfg)
    if case == "q_beyond_f16":
        q[:, 1] *= 3e5  # head 1's Q exceeds the f16 range: the scaled instance, rows shifted in the kernel
    q, k, v = (x.to(dtype) for x in (q, k, v))
    perm = torch.randperm(length, generator=torch.Generator().manual_seed(42)).to(torch.int32)
    layout = ScoringLayout(length, length, 16)
    nb = _m.ceil(length / 128)
    mask = torch.rand((heads, nb, nb), generator=torch.Generator().manual_seed(43)) < 0.4
    mask[:, torch.arange(nb), torch.arange(nb)] = True
    row_ptr, col_idx = ops.mask_to_csr(mask.to(dev))
    kw = {}
    if cu is not None:
        cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
        kw = dict(cu_seqlens_q=cu_d, cu_seqlens_k=cu_d)
    outs = {}
    for q_operand in (True, False):
        prep = ops.prepare_qkv(q.to(dev), k.to(dev), v.to(dev), perm.to(dev), layout, operand_dtype=pv,
                               pool=False, q_operand=q_operand)
        assert (prep.q_perm is None) == (not q_operand)
        outs[q_operand] = ops.bsa_fwd(prep, row_ptr, col_idx, out_dtype=torch.float32, **kw).cpu()
    qp, kp, vp = (orc.apply_permutation(x.float(), perm.long()) for x in (q, k, v))
    ref = (orc.masked_attention(qp, kp, vp, mask) if cu is None else orc.varlen_attention(qp, kp, vp, mask, cu, cu))
    for q_operand, out in outs.items():
        ma, mr = float((out - ref).abs().max()), mean_rel(out, ref)
        tol = 1e-3 if pv == torch.float16 else 3e-3
        assert ma <= 2e-2 and mr <= tol, (q_operand, ma, mr)
    if pv == torch.bfloat16 or dtype == torch.float16:
        assert torch.equal(outs[True], outs[False])  # the same operand values either way
    elif case != "q_beyond_f16":  # (there one-hot rows may pick another key on a rounding)
        assert mean_rel(outs[False], outs[True]) < 5e-4

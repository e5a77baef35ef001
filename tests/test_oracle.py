"""Pins the CPU oracle against the reference's own known answers, closed forms
and invariants (CPU only)."""
import math

import numpy as np
import pytest
import torch

from oracle import dfs_oracle as orc


# ---- a4: schedule — the reference's known-answer test
# (tests/test_flashinfer64_attention.py:122-144, dynamic ratio == native schedule)
def test_schedule_known_answers_dynamic():
    expected = {11: (False, 0.30), 12: (True, 0.30), 23: (False, 0.30), 24: (True, 0.20),
                35: (False, 0.20), 36: (True, 0.10), 47: (False, 0.10), 48: (False, 0.10),
                49: (False, 0.10)}
    for step, (refresh, ratio) in expected.items():
        got = orc.compute_cache_schedule(step, 12, 12, 0.30, 0.10)
        assert got[0] == refresh
        assert got[1] == pytest.approx(ratio)


def test_schedule_known_answers_fixed_and_errors():
    # dcrt = 0: refresh at every interval (tests/test_flashinfer64_attention.py:146-157)
    for step in (12, 24, 36, 48):
        assert orc.compute_cache_schedule(step, 12, 12, 0.195, 0.0) == (True, 0.195)
    assert orc.compute_cache_schedule(13, 12, 12, 0.195, 0.0)[0] is False
    with pytest.raises(ValueError):
        orc.compute_cache_schedule(0, 12, 0, 0.3, 0.1)
    # 0.3 / 0.1 == 2.9999999999999996 -> ceil 3 -> three refreshes
    assert [s for s in range(50) if orc.compute_cache_schedule(s, 12, 12, 0.3, 0.1)[0]] == [12, 24, 36]


# ---- a1: Hilbert order
def test_hilbert_one_bit_is_inverse_gray_of_interleaved_bits():
    # With one bit per axis the Hilbert index is the Gray-decoded string
    # (x, y, z) with axis 0 most significant: a closed form of Skilling's algorithm.
    pts = np.array([[x, y, z] for x in (0, 1) for y in (0, 1) for z in (0, 1)])
    codes = orc.hilbert_encode(pts, 3, 1)
    for (x, y, z), c in zip(pts, codes):
        b2, b1, b0 = x, x ^ y, x ^ y ^ z
        assert int(c) == (b2 << 2) | (b1 << 1) | b0
    assert [int(c) for c in orc.hilbert_encode(np.array([[0, 0], [0, 1], [1, 1], [1, 0]]), 2, 1)] == [0, 1, 2, 3]


def test_hilbert_matches_the_packages_published_example():
    # numpy-hilbert-curve's own usage example (its README, version 1.0.x):
    # decode([1, 2, 3], 2, 3) gives [[0, 1], [1, 1], [1, 0]], and encode of
    # those points gives [1, 2, 3]. This fixes which axis the finest level
    # steps along first at three levels (the axes swapped give [3, 2, 1]); it
    # does not tell the per-level exchange rule apart from leaving it out,
    # which agree on these first points.
    assert orc.hilbert_encode(np.array([[0, 1], [1, 1], [1, 0]]), 2, 3).tolist() == [1, 2, 3]
    assert int(orc.hilbert_encode(np.array([0, 0]), 2, 3)) == 0


def test_hilbert_decode_matches_the_packages_published_example():
    assert orc.hilbert_decode(np.array([1, 2, 3]), 2, 3).tolist() == [[0, 1], [1, 1], [1, 0]]


@pytest.mark.parametrize("dims,bits", [(2, 3), (3, 2), (3, 4), (3, 7)])
def test_hilbert_decode_inverts_encode(dims, bits):
    # Two separate restatements of the package's published steps must invert
    # each other: the encoder's loop orders, axis order and exchange step are
    # what the decoder undoes (3 x 7 bits: the cfg1/cfg2 grids' bit count).
    side = 1 << bits
    if side ** dims <= 1 << 16:
        grids = np.meshgrid(*[np.arange(side)] * dims, indexing="ij")
        pts = np.stack([g.reshape(-1) for g in grids], axis=1)
    else:
        pts = np.random.default_rng(3).integers(0, side, size=(50000, dims))
    codes = orc.hilbert_encode(pts, dims, bits)
    assert np.array_equal(orc.hilbert_decode(codes, dims, bits), pts)
    assert np.array_equal(orc.hilbert_encode(orc.hilbert_decode(codes, dims, bits), dims, bits), codes)


@pytest.mark.parametrize("dims,bits", [(2, 3), (3, 2), (3, 3)])
def test_hilbert_curve_invariants_on_full_cubes(dims, bits):
    side = 1 << bits
    grids = np.meshgrid(*[np.arange(side)] * dims, indexing="ij")
    pts = np.stack([g.reshape(-1) for g in grids], axis=1)
    codes = orc.hilbert_encode(pts, dims, bits).astype(np.int64)
    assert sorted(codes.tolist()) == list(range(side ** dims))  # bijection onto [0, 2^(n b))
    walk = pts[np.argsort(codes)]
    assert (walk[0] == 0).all()  # starts at the origin
    steps = np.abs(np.diff(walk, axis=0)).sum(axis=1)
    assert (steps == 1).all()  # consecutive indices are unit-adjacent


@pytest.mark.parametrize("grid", [(4, 16, 16), (3, 5, 7), (1, 1, 9), (21, 45, 80)])
def test_hilbert3d_perm_is_a_permutation_with_local_steps(grid):
    f, h, w = grid
    perm = orc.hilbert3d_perm(f, h, w)
    assert sorted(perm.tolist()) == list(range(f * h * w))
    z, rem = np.divmod(perm, h * w)
    y, x = np.divmod(rem, w)
    steps = np.abs(np.diff(z)) + np.abs(np.diff(y)) + np.abs(np.diff(x))
    assert np.median(steps) == 1  # locality of the curve on non-power-of-two grids


# ---- a5/a6: scoring, brute force on a tiny input
def _brute_block_scores(qp, kp, tile, block, video_len, k_tile=None):
    """Loop restatement of attention_wan.py:176-246 / attention_hyvideo.py:331-422
    (query tiles of ``tile`` tokens, key tiles of ``k_tile``)."""
    k_tile = tile if k_tile is None else k_tile
    _, heads, seq_len, dim = qp.shape
    vb, kb = math.ceil(video_len / block), math.ceil(seq_len / block)
    layout = [None] * (kb * block)
    for p in range(video_len):
        layout[p] = p
    for t in range(seq_len - video_len):
        layout[vb * block + t] = video_len + t
    out = torch.zeros(heads, vb, kb, dtype=torch.float64)
    for h in range(heads):
        def tile_mean(x, t, size):
            acc = torch.zeros(dim, dtype=torch.float64)
            for p in range(t * size, (t + 1) * size):
                if layout[p] is not None:
                    acc += x[0, h, layout[p]].double()
            return acc / size
        qt = [tile_mean(qp, t, tile) for t in range(vb * block // tile)]
        kt = [tile_mean(kp, t, k_tile) for t in range(kb * block // k_tile)]
        for i, qi in enumerate(qt):
            s = torch.stack([qi @ kj for kj in kt]) / math.sqrt(dim)
            p = torch.exp(s - s.max())
            p = p / p.sum()
            for j in range(len(kt)):
                out[h, i // (block // tile), j // (block // k_tile)] += p[j]
    return out


@pytest.mark.parametrize("seq,video,tile,k_tile", [
    (300, 300, 16, 16), (256, 256, 32, 32), (290, 250, 16, 16),
    (300, 300, 8, 64), (290, 250, 128, 4), (300, 200, 64, 32)])
def test_block_scores_match_brute_force(seq, video, tile, k_tile):
    torch.manual_seed(0)
    qp, kp = torch.randn(1, 2, seq, 8), torch.randn(1, 2, seq, 8)
    got = orc.block_scores(qp, kp, tile, 128, None if seq == video else video, k_tile=k_tile)
    ref = _brute_block_scores(qp, kp, tile, 128, video, k_tile)
    assert torch.allclose(got.double(), ref, rtol=1e-5, atol=1e-7)
    assert torch.allclose(got.sum(-1).double(), torch.full_like(ref.sum(-1), 128 / tile), rtol=1e-5)


def test_block_scores_reject_tiles_not_dividing_the_block():
    qp = torch.randn(1, 1, 256, 8)
    with pytest.raises(AssertionError, match="k_tile_size"):
        orc.block_scores(qp, qp, 16, 128, k_tile=48)
    with pytest.raises(AssertionError, match="q_tile_size"):
        orc.block_scores(qp, qp, 24, 128)


def test_wan_mask_matches_torch_topk_on_tie_free_scores():
    s = torch.rand(3, 40, 40, generator=torch.Generator().manual_seed(1))
    for ratio in (0.05, 0.3, 0.5, 1.0):
        k = orc.topk_count(ratio, 40)
        assert torch.equal(orc.mask_from_scores_wan(s, ratio), orc.mask_from_scores_torch(s, k))
        assert (orc.mask_from_scores_wan(s, ratio).sum(-1) == k).all()


def test_tie_order_is_lower_column_first():
    s = torch.tensor([[[1.0, 2.0, 2.0, 2.0, 0.5]]])
    assert orc.select_topk(s, 2).tolist() == [[[False, True, True, False, False]]]
    assert bool(orc.boundary_ties(s, 2).item()) and not bool(orc.boundary_ties(s, 3).item())


def test_hunyuan_mask_policy():
    # 931 blocks, dense_start 928 (cfg 2 shape), sparsity 0.3 -> k=279, video budget 276
    s = torch.rand(2, 929, 931, generator=torch.Generator().manual_seed(2))
    m = orc.mask_from_scores_hunyuan(s, 0.3, 118800 + 256, 118800)
    assert m.shape == (2, 931, 931)
    assert m[:, :928, 928:].all() and m[:, 928:].all()
    assert (m[:, :928, :928].sum(-1) == 276).all()
    assert torch.equal(m[:, :928, :928], orc.mask_from_scores_torch(s[:, :928, :928], 276))
    with pytest.raises(AssertionError):
        orc.mask_from_scores_hunyuan(s[:, :, :], 0.002, 118800 + 256, 118800)


# ---- a8: masked attention
def test_masked_attention_matches_dense_closed_form():
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, 2, 300, 16) for _ in range(3))
    mask = torch.rand(2, 3, 3) < 0.5
    mask[:, :, 0] = True
    got = orc.masked_attention(q, k, v, mask)
    ref = orc.dense_attention(q, k, v, orc.expand_block_mask(mask, 300))
    assert torch.allclose(got, ref, atol=1e-5)
    full = torch.ones(2, 3, 3, dtype=torch.bool)
    assert torch.allclose(orc.masked_attention(q, k, v, full), orc.dense_attention(q, k, v), atol=1e-5)


def test_segment_attention_matches_block_diagonal_closed_form():
    """cu_seqlens [0, 300, 430]: the second segment uses mask blocks counted
    from its own first token (token 300 sits in block 0 of that segment)."""
    torch.manual_seed(5)
    q, k, v = (torch.randn(1, 2, 430, 16) for _ in range(3))
    mask = torch.rand(2, 4, 4) < 0.5
    mask[:, :, 0] = True
    got = orc.segment_attention(q, k, v, mask, [0, 300, 430])
    tok = torch.zeros(2, 430, 430, dtype=torch.bool)
    tok[:, :300, :300] = orc.expand_block_mask(mask, 300)
    tok[:, 300:, 300:] = orc.expand_block_mask(mask, 130)
    assert torch.allclose(got, orc.dense_attention(q, k, v, tok), atol=1e-5)
    # a single segment is plain masked attention; an empty trailing one adds nothing
    assert torch.allclose(orc.segment_attention(q, k, v, mask, [0, 430, 430]), orc.masked_attention(q, k, v, mask))


def test_varlen_attention_closed_forms():
    """Separate query and key splits: sequence i's queries attend its own
    keys, blocks counted from each side's start. Checked against dense
    attention under the explicit token mask (a rectangular block-diagonal
    layout), against segment_attention for equal splits, and rows outside
    every query sequence stay zero."""
    torch.manual_seed(6)
    q, k, v = (torch.randn(1, 2, 430, 16) for _ in range(3))
    mask = torch.rand(2, 4, 4) < 0.5
    mask[:, :, 0] = True
    assert torch.allclose(orc.varlen_attention(q, k, v, mask, [0, 300, 430], [0, 300, 430]),
                          orc.segment_attention(q, k, v, mask, [0, 300, 430]))
    # Wan's cross form: every query, keys [0, 250) only (an empty second sequence)
    got = orc.varlen_attention(q, k, v, mask, [0, 430, 430], [0, 250, 430])
    tok = torch.zeros(2, 430, 430, dtype=torch.bool)
    tok[:, :, :250] = orc.expand_block_mask(mask, 430)[:, :, :250]
    assert torch.allclose(got, orc.dense_attention(q, k, v, tok), atol=1e-5)
    # unequal splits: queries [0, 200) / [200, 330) against keys [0, 260) / [260, 430)
    got = orc.varlen_attention(q, k, v, mask, [0, 200, 330], [0, 260, 430])
    tok = torch.zeros(2, 430, 430, dtype=torch.bool)
    tok[:, :200, :260] = orc.expand_block_mask(mask, 260)[:, :200, :260]
    tok[:, 200:330, 260:430] = orc.expand_block_mask(mask, 170)[:, :130, :170]
    ref = orc.dense_attention(q, k, v, tok)
    ref[:, :, 330:] = 0  # rows 330.. belong to no query sequence
    assert torch.allclose(got, ref, atol=1e-5)
    # a sequence without keys gives zero rows
    got = orc.varlen_attention(q, k, v, mask, [0, 300, 430], [0, 430, 430])
    assert torch.equal(got[:, :, 300:], torch.zeros_like(got[:, :, 300:]))


def test_full_reference_call_is_permutation_consistent():
    torch.manual_seed(4)
    q, k, v = (torch.randn(1, 2, 256, 16) for _ in range(3))
    perm = torch.from_numpy(orc.hilbert3d_perm(1, 16, 16))
    out, mask, scores = orc.dfs_attention_reference(q, k, v, perm, 1.0, 16)
    assert mask.all()
    assert torch.allclose(out, orc.dense_attention(q, k, v), atol=1e-5)


# ---- other token orders (order.py:8-436)
@pytest.mark.parametrize("w,h", [(2, 2), (4, 4), (16, 16), (80, 45), (45, 80), (7, 3), (6, 5), (1, 9), (9, 1)])
def test_gilbert_oracle_invariants(w, h):
    """Bijection over the rectangle, starts at the origin, unit steps (the
    generalised curve allows one diagonal step on some even x odd shapes)."""
    cells = orc.gilbert2d(w, h)
    assert sorted(cells) == [(x, y) for x in range(w) for y in range(h)]
    assert cells[0] == (0, 0)
    steps = [(abs(b[0] - a[0]), abs(b[1] - a[1])) for a, b in zip(cells, cells[1:])]
    assert all(s in ((1, 0), (0, 1), (1, 1)) for s in steps)
    assert sum(s == (1, 1) for s in steps) <= 1


@pytest.mark.parametrize("n", [2, 4, 8, 32])
def test_gilbert_oracle_is_the_hilbert_curve_on_power_of_two_squares(n):
    assert orc.gilbert2d(n, n) == [orc.hilbert_d2xy(n, d) for d in range(n * n)]


def test_morton_oracle_against_hand_codes():
    """Order of 2x2x2 and a 4x4 frame written out by hand from the
    interleave x0 y0 z0 x1 y1 z1 ... (x lowest)."""
    cube = orc.morton_perm(2, 2, 2, per_frame=False)
    # (x, y, z) by code 0..7: (0,0,0) (1,0,0) (0,1,0) (1,1,0) (0,0,1) ... -> z*4 + y*2 + x
    assert cube.tolist() == [0, 1, 2, 3, 4, 5, 6, 7]
    frame = orc.morton_perm(1, 4, 4, per_frame=True)
    assert frame.tolist() == [0, 1, 4, 5, 2, 3, 6, 7, 8, 9, 12, 13, 10, 11, 14, 15]
    flat = orc.morton_perm(1, 2, 4, per_frame=False)  # x up to 3, y up to 1, z = 0
    assert flat.tolist() == [0, 1, 4, 5, 2, 3, 6, 7]


def test_axis_and_block_oracles_closed_forms():
    f, h, w = 3, 4, 5
    hwf = orc.axis_order_perm(f, h, w, "hwf")
    assert hwf.tolist() == [z * h * w + y * w + x for y in range(h) for x in range(w) for z in range(f)]
    fwh = orc.axis_order_perm(f, h, w, "fwh")
    assert fwh.tolist() == [z * h * w + y * w + x for z in range(f) for x in range(w) for y in range(h)]
    blk = orc.block3d_perm(2, 2, 4, 1, 2, 2)  # bricks of 1x2x2 over a 2x2x4 grid
    assert blk.tolist() == [0, 1, 4, 5, 2, 3, 6, 7, 8, 9, 12, 13, 10, 11, 14, 15]
    assert sorted(orc.block3d_perm(5, 3, 9, 4, 4, 4).tolist()) == list(range(135))


# ---- DiT attention inputs: RMSNorm and complex RoPE
def _bf16_ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place (same-sign finite values)."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


def test_rmsnorm_oracle_matches_library():
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(11)
    x = torch.randn(37, 640, generator=g) * 3
    w = torch.randn(640, generator=g)
    torch.testing.assert_close(orc.rmsnorm_rows(x, w, 1e-6), F.rms_norm(x, (640,), w, 1e-6), rtol=3e-6, atol=3e-6)
    # eps matters on small rows, as in the library
    tiny = x[:2] * 1e-4
    torch.testing.assert_close(orc.rmsnorm_rows(tiny, w, 1e-6), F.rms_norm(tiny, (640,), w, 1e-6),
                               rtol=3e-6, atol=1e-9)
    xb, wb = x.bfloat16(), w.bfloat16()
    got = orc.rmsnorm_rows(xb, wb, 1e-6)
    ref = F.rms_norm(xb.float(), (640,), wb.float(), 1e-6).bfloat16()
    same_sign = torch.sign(got.float()) == torch.sign(ref.float())
    assert bool(same_sign.all()) and int(_bf16_ulps(got, ref).max()) <= 1
    assert float((got == ref).float().mean()) > 0.99


def test_rope_oracle_matches_complex_product():
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(2, 3, 50, 128, generator=g) * 2).bfloat16()
    ang = torch.rand(50, 64, generator=g, dtype=torch.float64) * 40
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    # the reference's fallback: complex128 product of view_as_complex pairs (replace_wan.py:209-213)
    freqs = torch.complex(cos.double(), sin.double())
    ref = torch.view_as_real(torch.view_as_complex(x.double().unflatten(-1, (-1, 2))) * freqs).flatten(-2)
    assert torch.equal(orc.rope_complex_pairs(x, cos, sin), ref.float().bfloat16())
    assert torch.equal(orc.rope_complex_pairs(x, torch.ones_like(cos), torch.zeros_like(sin)), x)
    # rotation keeps pair norms and -angle undoes +angle
    xf = x.float()
    r = orc.rope_complex_pairs(xf, cos, sin)
    n0 = xf[..., 0::2] ** 2 + xf[..., 1::2] ** 2
    n1 = r[..., 0::2] ** 2 + r[..., 1::2] ** 2
    torch.testing.assert_close(n1, n0, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(orc.rope_complex_pairs(r, cos, -sin), xf, rtol=1e-5, atol=1e-5)
    # a known rotation: angle pi/2 maps (a, b) to (-b, a)
    quarter = orc.rope_complex_pairs(xf[..., :1, :], torch.zeros(1, 64), torch.ones(1, 64))
    assert torch.equal(quarter[..., 0::2], -xf[..., :1, 1::2]) and torch.equal(quarter[..., 1::2], xf[..., :1, 0::2])


def test_norm_rope_heads_oracle_layout():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 9, 3 * 16, generator=g).bfloat16()
    w = torch.rand(48, generator=g) + 0.5
    cos, sin = torch.rand(6, 8, generator=g), torch.rand(6, 8, generator=g)
    out = orc.norm_rope_heads(x, 3, w, 1e-6, cos, sin, rope_skip=3)
    assert out.shape == (2, 3, 9, 16)
    normed = orc.rmsnorm_rows(x, w, 1e-6)
    for b in range(2):
        for h in range(3):
            head = normed[b, :, h * 16:(h + 1) * 16]
            assert torch.equal(out[b, h, :3], head[:3])  # rows before rope_skip are not rotated
            assert torch.equal(out[b, h, 3:], orc.rope_complex_pairs(head[3:], cos, sin))


def test_real_rope_oracle_against_complex_rotation():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(2, 3, 40, 64, generator=g)
    ang = torch.rand(40, 32, generator=g, dtype=torch.float64) * 30
    # real tables repeat each angle over its (even, odd) pair
    cos = torch.cos(ang).float().repeat_interleave(2, dim=-1)
    sin = torch.sin(ang).float().repeat_interleave(2, dim=-1)
    got = orc.rope_real_pairs(x, cos, sin)
    freqs = torch.complex(torch.cos(ang).float().double(), torch.sin(ang).float().double())
    ref = torch.view_as_real(torch.view_as_complex(x.double().unflatten(-1, (-1, 2))) * freqs).flatten(-2)
    torch.testing.assert_close(got.double(), ref, rtol=1e-6, atol=1e-6)
    assert torch.equal(orc.rope_real_pairs(x, torch.ones(40, 64), torch.zeros(40, 64)), x)
    back = orc.rope_real_pairs(got, cos, -sin)
    torch.testing.assert_close(back, x, rtol=1e-5, atol=1e-5)
    quarter = orc.rope_real_pairs(x[..., :1, :], torch.zeros(1, 64), torch.ones(1, 64))
    assert torch.equal(quarter[..., 0::2], -x[..., :1, 1::2]) and torch.equal(quarter[..., 1::2], x[..., :1, 0::2])


def test_head_norm_rope_oracle_layout():
    g = torch.Generator().manual_seed(15)
    x = torch.randn(1, 10, 2 * 16, generator=g).bfloat16()
    w = torch.rand(16, generator=g) + 0.5
    cos, sin = torch.rand(7, 16, generator=g), torch.rand(7, 16, generator=g)
    out = orc.head_norm_rope_heads(x, 2, w, 1e-6, cos, sin, rope_rows=7)
    for h in range(2):
        head = orc.rmsnorm_rows(x[0, :, h * 16:(h + 1) * 16], w, 1e-6)  # each head normalised alone
        assert torch.equal(out[0, h, :7], orc.rope_real_pairs(head[:7], cos, sin))
        assert torch.equal(out[0, h, 7:], head[7:])  # text rows after rope_rows are not rotated

"""Host-side logic and the C-ABI surface (CPU only: no kernel is launched)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from dfsattn_amd import _lib, ops
from dfsattn_amd.layout import (ScoringLayout, TopkPolicy, csr_flops, block_flops, dense_policy,
                                hunyuan_policy, topk_count, wan_policy)
from oracle import dfs_oracle as orc

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dfsattn_amd.h")


def test_library_exports_every_declared_symbol():
    text = open(HEADER).read()
    declared = set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(dfs_\w+)\s*\(", text, flags=re.M))
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.dfs_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("grid", [(4, 16, 16), (3, 5, 7), (1, 1, 1), (2, 3, 1), (21, 45, 80), (33, 45, 80)])
def test_hilbert_c_matches_numpy_oracle(grid):
    got = ops.hilbert3d_perm(*grid).numpy()
    assert np.array_equal(got, orc.hilbert3d_perm(*grid))


def test_abi_rejects_bad_arguments_without_launching():
    fake = ctypes.c_void_p(16)
    with pytest.raises(_lib.DfsKernelError, match="head_dim=96"):
        _lib.call("dfs_prepare_qkv", fake, fake, fake, fake, 2, 1000, 96, 0, 1000, 16, 16, 1,
                  fake, fake, fake, None, None, None, None, None, None)
    with pytest.raises(_lib.DfsKernelError, match="q_tile_size=24"):
        _lib.call("dfs_prepare_qkv", fake, fake, fake, fake, 2, 1000, 128, 0, 1000, 24, 16, 1,
                  fake, fake, fake, None, None, None, None, None, None)
    with pytest.raises(_lib.DfsKernelError, match="k_tile_size=48"):
        _lib.call("dfs_prepare_qkv", fake, fake, fake, fake, 2, 1000, 128, 0, 1000, 16, 48, 1,
                  fake, fake, fake, None, None, None, None, None, None)
    # scoring: tiles below 4 tokens, and the generic scorer without scores_out
    with pytest.raises(_lib.DfsKernelError, match="k_tile_size=2"):
        _lib.call("dfs_block_score_topk", fake, fake, fake, fake, 2, 128, 16, 2, 8, 8, 8, 8, 2, 8, 8,
                  fake, fake, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="pass one"):
        _lib.call("dfs_block_score_topk", fake, fake, fake, fake, 2, 128, 8, 64, 8, 8, 8, 8, 2, 8, 8,
                  fake, fake, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="k_pick"):
        _lib.call("dfs_topk_from_scores", fake, 2, 8, 8, 8, 8, 9, 8, 8, fake, fake, None, None)
    with pytest.raises(_lib.DfsKernelError, match="f16 inputs"):
        _lib.call("dfs_bsa_fwd", fake, fake, fake, fake, fake, 2, 1000, 128, 1, 0, 0.1, fake, 2,
                  None, None, None, None, 1, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="n_seq=3"):
        _lib.call("dfs_bsa_fwd", fake, fake, fake, fake, fake, 2, 1000, 128, 1, 1, 0.1, fake, 2,
                  None, None, fake, fake, 3, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="both cu_seqlens_q and cu_seqlens_k"):
        _lib.call("dfs_bsa_fwd", fake, fake, fake, fake, fake, 2, 1000, 128, 1, 1, 0.1, fake, 2,
                  None, None, fake, None, 2, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="two sequences need cu_seqlens"):
        _lib.call("dfs_bsa_fwd", fake, fake, fake, fake, fake, 2, 1000, 128, 1, 1, 0.1, fake, 2,
                  None, None, None, None, 2, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="q_src needs q_rows"):
        _lib.call("dfs_bsa_fwd", None, fake, fake, fake, fake, 2, 1000, 128, 1, 1, 0.1, fake, 2,
                  None, None, None, None, 1, None, fake, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="bf16 Q/K operands need a bf16 q_src"):
        _lib.call("dfs_bsa_fwd", None, fake, fake, fake, fake, 2, 1000, 128, 0, 0, 0.1, fake, 2,
                  None, None, None, None, 1, None, fake, fake, 1, None)
    with pytest.raises(_lib.DfsKernelError, match="NULL operand"):
        _lib.call("dfs_bsa_fwd", None, fake, fake, fake, fake, 2, 1000, 128, 1, 1, 0.1, fake, 2,
                  None, None, None, None, 1, None, None, None, 0, None)
    with pytest.raises(_lib.DfsKernelError, match="head_dim=96"):
        _lib.call("dfs_prepare_fixup", fake, fake, fake, fake, 2, 1000, 96, fake, fake, fake, fake, fake, None)
    # the allocation-free scorer refuses block sums beyond its 96 MiB scratch
    # before touching a device (64 heads x 1000 x 1000 blocks = 256 MB)
    with pytest.raises(_lib.DfsKernelError, match="scratch holds 100663296"):
        _lib.call("dfs_block_score_topk_noalloc", fake, fake, fake, fake, 64, 128, 16, 16, 1000, 1000, 1000, 1000, 300,
                  1000, 1000, fake, fake, None, None)
    with pytest.raises(_lib.DfsKernelError, match="row_bytes"):
        _lib.call("dfs_permute_gather", fake, fake, fake, 1, 10, 10, 10, 3, None)
    with pytest.raises(_lib.DfsKernelError, match="positive"):
        _lib.call("dfs_hilbert3d_perm", 0, 4, 4, fake)


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.permute_gather(x, torch.arange(128, dtype=torch.int32))


def test_config_shapes_and_policies():
    wan = ScoringLayout(75600, 75600, 16)
    assert (wan.q_blocks, wan.rows, wan.q_tiles, wan.k_tiles) == (591, 75648, 4728, 4728)
    pol = wan_policy(wan, 0.3)
    assert (pol.k_pick, pol.n_cand, pol.dense_row) == (177, 591, 591)
    assert pol.nnz(40) == 4184280
    assert pol.row_ptr(2)[-1] == 2 * 591 * 177
    hy = ScoringLayout(118800 + 256, 118800, 16)
    assert (hy.q_blocks, hy.video_blocks, hy.q_tiles, hy.k_tiles) == (931, 929, 7432, 7448)
    hp = hunyuan_policy(hy, 0.3)
    assert (hp.scored_rows, hp.n_cand, hp.k_pick, hp.dense_col, hp.dense_row) == (929, 928, 276, 928, 928)
    counts = hp.row_counts()
    assert (counts[:928] == 279).all() and (counts[928:] == 931).all()
    assert hp.nnz(24) == 6280920
    # schedule sparsities 0.3 / 0.2 / 0.1 -> Wan top-k 177 / 118 / 59 (0.2 * 591 = 118.2)
    assert [topk_count(s, 591) for s in (0.3, 0.2, 0.1)] == [177, 118, 59]
    d = dense_policy(wan)
    assert (d.row_counts() == 591).all()


def test_policy_errors_follow_the_reference():
    with pytest.raises(AssertionError):
        hunyuan_policy(ScoringLayout(118800 + 256, 118800, 16), 0.002)
    with pytest.raises(RuntimeError, match="tile view"):
        ScoringLayout(129 + 127, 129, 16)  # 2 video blocks + 127 text tokens > 2 blocks
    with pytest.raises(ValueError, match="block_size"):
        ScoringLayout(1000, 1000, 16, block=64)
    with pytest.raises(AssertionError, match="divisible"):
        ScoringLayout(1000, 1000, 48)
    with pytest.raises(RuntimeError, match="out of range"):
        wan_policy(ScoringLayout(1000, 1000, 16), 1.5)


def test_policy_row_counts_match_oracle_masks():
    for seq, video, ratio in ((1000, 1000, 0.3), (1060, 1000, 0.5), (1000, 1000, 0.05), (3256, 3000, 0.2)):
        lay = ScoringLayout(seq, video, 16)
        pol = wan_policy(lay, ratio) if seq == video else hunyuan_policy(lay, ratio)
        s = torch.rand(2, pol.scored_rows, pol.k_blocks)
        m = orc.mask_from_scores_wan(s, ratio) if seq == video else orc.mask_from_scores_hunyuan(s, ratio, seq, video)
        assert np.array_equal(m.sum(-1)[0].numpy(), pol.row_counts())


def test_flop_counts_use_valid_token_blocks():
    mask = np.ones((2, 3, 3), dtype=bool)
    assert block_flops(mask, 300, 64) == 4 * 64 * 300 * 300 * 2
    pol = wan_policy(ScoringLayout(300, 300, 16), 1.0)
    ptr = pol.row_ptr(2)
    cols = np.tile(np.arange(3), 6)
    assert csr_flops(ptr, cols, 2, 300, 64) == block_flops(mask, 300, 64)
    # cfg 1 nominal bound 35.10 TFLOP
    assert abs(4 * 128 * 128 * 128 * 4184280 / 1e12 - 35.10) < 0.01


def test_cu_seqlens_forms():
    """Host cu_seqlens: [0, L] and [0, L, L] are one sequence, [0, a, L] a
    split (including a = 0); other forms are refused. Device tensors are
    never read back (their checks run on the GPU tests)."""
    from dfsattn_amd.core import DfsCore
    check = DfsCore._host_split
    assert DfsCore._sequences(None, 300, torch.device("cpu"), "cu") is None
    assert check([0, 300], 300) is None
    assert check([0, 300, 300], 300) is None
    assert check([0, 250, 300], 300) == [0, 250, 300]
    assert check([0, 0, 300], 300) == [0, 0, 300]
    for bad in ([0, 100, 200, 300], [1, 300], [0, 310, 300], [0, 200], [0, 200, 100, 300]):
        with pytest.raises(NotImplementedError):
            check(bad, 300)


@pytest.mark.parametrize("grid", [(1, 4, 4), (3, 5, 7), (2, 8, 8), (5, 3, 9), (1, 1, 1), (4, 16, 16), (2, 45, 80)])
def test_token_orders_match_oracle(grid):
    from dfsattn_amd.utils import order as od
    f, h, w = grid
    cases = {
        "hilbert2d": (od.hilbert2d_perm(f, h, w), orc.hilbert2d_perm(f, h, w)),
        "morton3d": (od.morton3d_perm(f, h, w), orc.morton_perm(f, h, w, per_frame=False)),
        "morton2d": (od.morton2d_perm(f, h, w), orc.morton_perm(f, h, w, per_frame=True)),
        "hwf": (od.hwf(f, h, w), orc.axis_order_perm(f, h, w, "hwf")),
        "fwh": (od.fwh(f, h, w), orc.axis_order_perm(f, h, w, "fwh")),
        "blk": (od.block3d_perm(f, h, w, 4, 4, 4), orc.block3d_perm(f, h, w, 4, 4, 4)),
        "blk_ragged": (od.block3d_perm(f, h, w, 2, 3, 5), orc.block3d_perm(f, h, w, 2, 3, 5)),
    }
    for name, (got, ref) in cases.items():
        assert got.dtype == torch.long and np.array_equal(got.numpy(), ref), name


def test_morton_bit_spreading_and_dispatch():
    from dfsattn_amd.utils import order as od
    v = torch.tensor([0, 1, 2, 3, 7, (1 << 20), (1 << 21) + 5])
    assert od.part1by2_tensor(v).tolist() == [0, 1, 8, 9, 0b1001001, 1 << 60, 0b1000001]
    assert od.part1by1_tensor(torch.tensor([1, 2, 3, (1 << 31), (1 << 32) + 1])).tolist() == [1, 4, 5, 1 << 62, 1]
    assert od.morton3D_tensor(torch.tensor([1, 0, 0]), torch.tensor([0, 1, 0]), torch.tensor([0, 0, 1])).tolist() == [1, 2, 4]
    assert od.video_perm_for("org", 2, 3, 4) is None
    for name in od.ORDERS[1:]:
        p = od.video_perm_for(name, 3, 8, 8)
        assert sorted(p.tolist()) == list(range(192)), name
    assert torch.equal(od.video_perm_for("blk", 3, 8, 8), od.block3d_perm(3, 8, 8, 4, 4, 4))
    with pytest.raises(ValueError):
        od.video_perm_for("zigzag", 1, 2, 2)


def test_workspace_size_by_tile_pair():
    """The one-pass workspace exists for equal 16- or 32-token tiles only;
    other valid pairs report 0 (two-pass generic scorer), invalid ones -1."""
    ws = _lib.lib().dfs_block_score_topk_workspace_size
    assert ws(40, 16, 16, 591, 591) > 0 and ws(40, 32, 32, 591, 591) > 0
    for qt, kt in ((8, 64), (16, 32), (128, 4), (64, 64), (8, 8)):
        assert ws(40, qt, kt, 591, 591) == 0
    for qt, kt in ((2, 16), (16, 24), (256, 16), (0, 16)):
        assert ws(40, qt, kt, 591, 591) == -1


def test_noalloc_wrapper_runs_under_the_tensors_device(monkeypatch):
    """ops.block_score_topk_noalloc makes the tensors' device current around
    the C call (the library takes its scratch from the stream's device, and
    the launch and the stream then agree whichever device the caller has
    current). Host logic only: the device context and the C call are
    recorded, nothing runs on a GPU."""
    from types import SimpleNamespace
    from dfsattn_amd.layout import ScoringLayout, wan_policy

    events = []

    class FakeDeviceCtx:
        def __init__(self, dev):
            self.dev = dev

        def __enter__(self):
            events.append(("enter", self.dev))

        def __exit__(self, *exc):
            events.append(("exit", self.dev))

    target = torch.device("cuda", 3)
    fake_t = SimpleNamespace(device=target)
    layout = ScoringLayout(1024, 1024, 16)
    pol = wan_policy(layout, 0.3)
    prep = SimpleNamespace(q_hi=fake_t, q_lo=fake_t, k_hi=fake_t, k_lo=fake_t, q_perm=None, k_perm=fake_t,
                           device=target, heads=2, head_dim=64, layout=layout)
    real_empty = torch.empty
    monkeypatch.setattr(ops, "_require_device", lambda *a: None)
    monkeypatch.setattr(ops, "_require_int32", lambda **k: None)
    monkeypatch.setattr(ops, "_ptr", lambda t: None)
    monkeypatch.setattr(ops, "_stream", lambda t: None)
    monkeypatch.setattr(ops.torch, "empty", lambda *a, device=None, **k: real_empty(*a, **k))
    monkeypatch.setattr(ops.torch.cuda, "device", FakeDeviceCtx)
    monkeypatch.setattr(ops._lib, "call", lambda name, *args: events.append(("call", name, args[6], args[7])))
    row_ptr = torch.from_numpy(pol.row_ptr(2))
    ops.block_score_topk_noalloc(prep, pol, row_ptr)
    assert events == [("enter", target), ("call", "dfs_block_score_topk_noalloc", 16, 16), ("exit", target)]

"""The allocation-free scoring entry point (dfs_block_score_topk_noalloc)
against dfs_block_score_topk with caller buffers, through the C-ABI: two
calls in a row, the second smaller (the static scratch keeps the first
call's contents), each bit-exact in columns and mask."""
import pytest
import torch

from dfsattn_amd import ops
from dfsattn_amd.core import row_ptr_for
from dfsattn_amd.layout import ScoringLayout, hunyuan_policy, wan_policy
from dfsattn_amd.workloads import DfsConfig, synth_qkv

pytestmark = pytest.mark.gpu


def _case(dev, grid, heads, d, text_len, sparsity, seed, tiles=(16, 16)):
    cfg = DfsConfig("noalloc", grid, heads, d, torch.bfloat16, text_len=text_len, seed=seed)
    q, k, v = synth_qkv(cfg, device=dev)
    layout = ScoringLayout(cfg.seq_len, cfg.video_len, tiles[0], k_tile=tiles[1])
    policy = hunyuan_policy(layout, sparsity) if text_len else wan_policy(layout, sparsity)
    perm = torch.arange(cfg.seq_len, dtype=torch.int32, device=dev)
    prep = ops.prepare_qkv(q, k, v, perm, layout)
    return prep, policy, row_ptr_for(policy, heads, dev)


def test_noalloc_scoring_matches_buffered_entry(dev):
    cases = [((8, 30, 40), 6, 128, 0, 0.3, 1, (16, 16)),   # 9,600 tokens x 6 heads: 75 x 75 blocks
             ((3, 16, 20), 2, 64, 100, 0.5, 2, (16, 16)),   # smaller, HunyuanVideo policy with text
             ((2, 16, 20), 2, 128, 0, 0.3, 3, (8, 64))]     # smaller still, unequal tiles (generic scorer)
    for grid, heads, d, text_len, sparsity, seed, tiles in cases:
        print(f"noalloc case grid={grid} heads={heads} d={d} text={text_len} tiles={tiles}", flush=True)
        prep, policy, row_ptr = _case(dev, grid, heads, d, text_len, sparsity, seed, tiles)
        col_ref, _, mask_ref = ops.block_score_topk(prep, policy, row_ptr, want_mask=True, one_pass=False)
        col, mask = ops.block_score_topk_noalloc(prep, policy, row_ptr, want_mask=True)
        torch.cuda.synchronize()
        assert torch.equal(col.cpu(), col_ref.cpu())
        assert torch.equal(mask.cpu(), mask_ref.cpu())

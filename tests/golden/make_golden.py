"""Writes the golden fixtures of this directory from the CPU restatement in
``oracle/dfs_oracle.py`` (never from the reference, which is not run).

Each fixture holds the inputs as bf16 bit patterns (uint16: the GPU path takes
bf16, and the oracle runs fp32 on the same values), the Hilbert permutation,
the fp32 block scores, the kept-block mask and the fp32 masked-attention
output in the original token order. They pin the oracle and the synthetic
input generator against silent change; the GPU tests compare the HIP path
with them.

Cases:
  * cfg0    configs[0] shape: 4x16x16 grid (1,024 tokens), 2 heads, d64,
            Wan policy, sparsity 0.3 (k = 2 of 8 blocks).
  * hytext  HunyuanVideo policy with text: 4x8x16 grid (512 video tokens) +
            40 text tokens, 2 heads, d64, sparsity 0.5 (k = 2 of 5 blocks: one
            video block chosen among 4, the text block column and row dense).
  * tail    Wan policy with a ragged last block: 3x7x9 grid (189 tokens,
            last block 61 tokens), 1 head, d64, sparsity 0.5.

Run from the repo root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from dfsattn_amd.workloads import CONFIGS, DfsConfig, synth_qkv  # noqa: E402
from oracle import dfs_oracle as orc  # noqa: E402

CASES = {
    "cfg0": dict(cfg=CONFIGS[0], sparsity=0.3, hunyuan=False),
    "hytext": dict(cfg=DfsConfig("hytext", (4, 8, 16), 2, 64, torch.bfloat16, text_len=40, seed=7),
                   sparsity=0.5, hunyuan=True),
    "tail": dict(cfg=DfsConfig("tail", (3, 7, 9), 1, 64, torch.bfloat16, seed=11), sparsity=0.5, hunyuan=False),
}


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bits_to_f32(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16).float()


def compute_case(name: str) -> dict:
    spec = CASES[name]
    cfg = spec["cfg"]
    q, k, v = synth_qkv(cfg, dtype=torch.float32)
    qb, kb, vb = (bf16_bits(x) for x in (q, k, v))
    qf, kf, vf = (bits_to_f32(x) for x in (qb, kb, vb))
    perm = orc.hilbert3d_perm(*cfg.grid)
    video_len = cfg.video_len if spec["hunyuan"] else None
    out, mask, scores = orc.dfs_attention_reference(qf, kf, vf, torch.from_numpy(perm), spec["sparsity"],
                                                    cfg.tile, video_len=video_len)
    return {"q": qb, "k": kb, "v": vb, "perm": perm.astype(np.int64), "scores": scores.numpy().astype(np.float32),
            "mask": mask.numpy().astype(bool), "out": out.numpy().astype(np.float32),
            "sparsity": np.float64(spec["sparsity"]), "tile": np.int64(cfg.tile),
            "video_len": np.int64(cfg.video_len), "hunyuan": np.bool_(spec["hunyuan"]),
            "grid": np.array(cfg.grid, dtype=np.int64)}


def main() -> None:
    for name in CASES:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **compute_case(name))
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

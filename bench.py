"""Benchmark of the DFS sparse-attention hot path on one MI355X.

Workload: one DFS attention call at the Wan shape,
B=1, 21x45x80 = 75,600 tokens, 40 heads, head_dim 128, bf16, tile 16, block
128, hilbert3d order, sparsity 0.3, mask computed fresh every call. A step is
one full call through the public entry point ``dfs_attention``: Hilbert gather
of Q/K/V (+ tile pooling), block scoring + top-k, block-sparse attention with
the fused inverse permutation.

Prints one JSON line (metric = ms per call, lower is better) with the
roofline of the attention kernel, per-phase kernel times and a CPU baseline
(the fp32 oracle on a bounded sample of the same inputs, scaled up). The
phase times (and so the roofline's achieved rate) come from HIP event pairs
that the call's own phase recorder places around prepare, score + top-k and
attention in every timed step. Two side measurements ride on the same line:
the attention kernel on bf16 operands (the reference kernel's operand
precision) over the same mask, beside the default f16 operands timed in the
same stretch; a less local mask at the same density (K drawn from a field of
its own, so a row's kept blocks spread over the whole row): its whole-call
median and its attention kernel time; and the dense path (``full_attention``
in "flash" mode, every block kept) on the same inputs under ``dense_call``.

The default line also carries the second BASELINE configuration under
``cfg2``: the HunyuanVideo call's time, phases and attention-kernel fraction
of peak over 10 fresh-mask calls; and under ``cfg4`` the 40-block DiT
denoising step with DFS self-attention against the dense step (both skipped
with ``--headline-only``).

``--workload cfg2`` measures the HunyuanVideo call instead (configs[2]:
118,800 video + 256 text tokens, 24 heads), and ``--workload cfg3`` the
mask-cache regime (configs[3]: 50 denoising calls at the cfg1 shape with
Q, K drifting by N(0, 0.02) per step, 12 dense warm-up steps, a mask refresh
every 12 steps, sparsity in {0.1, 0.2, 0.3, 0.5}, sparsity_dcrt 0 and 0.1);
each prints its own JSON line. The default run (cfg1) is the benchmark line.

``--workload cfg4`` times a whole denoising step of a random-init 40-block
Wan-style DiT with DFS self-attention against the same step with
dense self-attention.

The line's ``dtype`` is the MFMA operand type of the DFS kernels (f16: the
bf16 inputs are rounded to f16, a head beyond the f16 range is stored scaled
by a power of two) and ``input_dtype`` the type of the tensors passed in.

``--gemm-calibration`` instead times torch.matmul (hipBLASLt) at 16384^3 in
bf16 and f16: the rate a vendor MFMA-bound kernel sustains on the same box.

``--copy-calibration`` instead runs one plain 1 GiB device copy (torch's copy
kernel), the known-size reference the FETCH_SIZE / WRITE_SIZE counters of the
attention kernel are scaled by. The per-launch HBM traffic those counter runs
give is kept in profiles/bsa_fwd_cfg1_traffic.txt and reported as
``roofline.traffic``.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/f16 MFMA
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "bsa_fwd_cfg1_traffic.txt")


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def run_gpu(args):
    from dfsattn_amd import ops
    from dfsattn_amd.attention_wan import DFS_Attention, dfs_attention, _dfs_attention_instances
    from dfsattn_amd.layout import ScoringLayout, csr_flops, wan_policy
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[1]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("generating cfg1 inputs on the GPU")
    q, k, v = synth_qkv(cfg, device=dev)
    torch.cuda.synchronize()
    log("inputs ready; warmup")
    f, h, w = cfg.grid
    video_perm = hilbert3d_perm(f, h, w)
    L = cfg.seq_len

    # One call per step, mask refreshed every call (step index at a refresh
    # step with cache_flag=True; Wan counts CFG passes, so 2*skip_steps).
    def step():
        return dfs_attention(q, k, v, step_idx=0, skip_steps=0, cache_interval=1, layer_idx=0,
                             sparsity=cfg.sparsity, sparsity_dcrt=0.0, tile_size=cfg.tile,
                             block_size=cfg.block, video_perm=video_perm, cache_flag=True)

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")
    # The timed steps run with the call's own phase recorder on: it records a
    # HIP event pair on the current stream (the stream the kernels run on)
    # around the prepare, score + top-k and attention phases of every call,
    # and never waits for the device, so the phase times come from the timed
    # region itself.
    DFS_Attention.set_record_timing(True)
    t0 = time.perf_counter()
    e0, e1 = _events()
    e0.record()
    for _ in range(args.steps):
        out = step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_per_step = e0.elapsed_time(e1) / args.steps
    spans = DFS_Attention.timing_recorder.rows()
    DFS_Attention.set_record_timing(False)
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/call")
    phase_of = {"qkv_permute": "prepare", "topk_mask": "score_topk", "attention_execution": "attention"}
    ev = {name: [] for name in phase_of.values()}
    for span in spans:
        if span["phase"] in phase_of:
            ev[phase_of[span["phase"]]].append(span["elapsed_ms"])
    assert all(len(v_) == args.steps for v_ in ev.values()), {k_: len(v_) for k_, v_ in ev.items()}
    phase_ms = {k_: float(np.mean(v_)) for k_, v_ in ev.items()}
    log(f"phase times over the timed steps (ms): {phase_ms}")
    entry = next(iter(DFS_Attention._cached_metadata.values()))
    row_ptr, col_idx = entry["row_ptr"], entry["col_idx"]  # the last timed call's mask
    # Median of per-call event pairs over at least 50 further calls.
    per_call = []
    for _ in range(max(50, args.steps)):
        a, b = _events()
        a.record()
        step()
        b.record()
        per_call.append((a, b))
    torch.cuda.synchronize()
    per_call = sorted(a.elapsed_time(b) for a, b in per_call)
    median_ms = per_call[len(per_call) // 2]
    log(f"median of {len(per_call)} calls: {median_ms:.3f} ms")

    layout = ScoringLayout(L, L, cfg.tile)
    pol = wan_policy(layout, cfg.sparsity)
    perm_d = ops.device_perm(video_perm, dev)
    reps = max(3, args.steps)
    flops = csr_flops(row_ptr.cpu().numpy(), col_idx.cpu().numpy(), cfg.heads, L, cfg.head_dim)
    att_tflops = flops / (phase_ms["attention"] * 1e-3) / 1e12
    D = cfg.head_dim
    tensor_bytes = cfg.heads * L * D * 2
    prep_bytes = 3 * 2 * tensor_bytes  # read + write of Q, K, V (pooled outputs are ~1/16 extra)
    score_flop = 2 * layout.q_tiles * layout.k_tiles * D * cfg.heads

    side = {}
    if not args.headline_only:
        side = _side_measurements(args, cfg, dev, q, k, v, video_perm, layout, pol, perm_d, row_ptr, col_idx, flops,
                                  reps)
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()
    return {
        "ms_per_step": ms_per_step,
        "median_ms": median_ms,
        "median_calls": len(per_call),
        "wall_ms_per_step": wall_ms,
        "phase_ms": phase_ms,
        "attention_flop": flops,
        "attention_tflops": att_tflops,
        "prepare_gbs": prep_bytes / (phase_ms["prepare"] * 1e-3) / 1e9,
        "score_pooled_gflop": score_flop / 1e9,
        "density": flops / (4.0 * D * L * L * cfg.heads),
        "side": side,
        "out_shape": list(out.shape),
        "inputs": (q, k, v),
    }


def _side_measurements(args, cfg, dev, q, k, v, video_perm, layout, pol, perm_d, row_ptr, col_idx, flops, reps):
    """The attention kernel on bf16 operands over the headline mask, a less
    local mask at the same density (whole call and attention kernel), and the
    dense path on the same inputs."""
    from dfsattn_amd import ops
    from dfsattn_amd.attention_wan import dfs_attention
    from dfsattn_amd.layout import csr_flops
    from dfsattn_amd.workloads import synth_qkv
    L = cfg.seq_len

    def attention_ms(prep_x, cols):
        """Mean HIP-event time of the attention kernel on the current stream."""
        ops.bsa_fwd(prep_x, row_ptr, cols, out_perm=perm_d)
        times = []
        for _ in range(reps):
            a, b = _events()
            a.record()
            ops.bsa_fwd(prep_x, row_ptr, cols, out_perm=perm_d)
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        return float(np.mean(times))

    # The same mask on bf16 operands (Q, K, V and P in bf16, the reference
    # kernel's operand precision) beside the default f16 operands, timed in
    # the same stretch so that both see the same clock.
    prep_f16 = ops.prepare_qkv(q, k, v, perm_d, layout, pool=False)
    prep16 = ops.prepare_qkv(q, k, v, perm_d, layout, operand_dtype=torch.bfloat16, pool=False)
    f16_ms = attention_ms(prep_f16, col_idx)
    bf16_ms = attention_ms(prep16, col_idx)
    del prep16, prep_f16
    log(f"attention on bf16 operands: {bf16_ms:.3f} ms (f16 operands in the same stretch: {f16_ms:.3f} ms)")

    # A less local mask at the same density: K from a field of its own, so
    # the kept blocks of a row spread over the whole row instead of clustering
    # near the diagonal; the whole call and the attention kernel on it.
    qn, kn, vn = synth_qkv(cfg, device=dev, independent_keys=True)
    call_n = []
    for i in range(max(10, args.warmup + 5)):
        a, b = _events()
        a.record()
        dfs_attention(qn, kn, vn, step_idx=0, skip_steps=0, cache_interval=1, layer_idx=1,
                      sparsity=cfg.sparsity, sparsity_dcrt=0.0, tile_size=cfg.tile, block_size=cfg.block,
                      video_perm=video_perm, cache_flag=True)
        b.record()
        call_n.append((a, b))
    torch.cuda.synchronize()
    call_n = sorted(a.elapsed_time(b) for a, b in call_n[args.warmup:])
    prep_n = ops.prepare_qkv(qn, kn, vn, perm_d, layout)
    col_n, _, _ = ops.block_score_topk(prep_n, pol, row_ptr)
    far_ms = attention_ms(prep_n, col_n)
    flops_n = csr_flops(row_ptr.cpu().numpy(), col_n.cpu().numpy(), cfg.heads, L, cfg.head_dim)
    rows_of = np.repeat(np.arange(cfg.heads * pol.q_blocks) % pol.q_blocks, np.diff(row_ptr.cpu().numpy()))

    def near_diag(cols):
        """Fraction of kept blocks within 8 blocks of their row's diagonal."""
        return float(np.mean(np.abs(cols.cpu().numpy() - rows_of) <= 8))

    less_local = {
        "inputs": "synth_qkv(independent_keys=True): K from its own smoothed field",
        "call_ms_median": round(call_n[len(call_n) // 2], 3),
        "attention_ms": round(far_ms, 3),
        "attention_tflops": round(flops_n / (far_ms * 1e-3) / 1e12, 1),
        "frac": round(flops_n / (far_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "kept_density": round(flops_n / (4.0 * cfg.head_dim * L * L * cfg.heads), 4),
        "kept_within_8_blocks_of_diagonal": round(near_diag(col_n), 4),
        "headline_mask_kept_within_8_blocks_of_diagonal": round(near_diag(col_idx), 4),
    }
    log(f"less local mask: {less_local}")
    del prep_n, qn, kn, vn

    # The dense path (full_attention in "flash" mode: warm-up steps, skip
    # layers and periodic dense steps of the processors) on the same inputs:
    # the same kernel with every block kept.
    from dfsattn_amd.fullattention import full_attention
    full_attention(q, k, v, mode="flash")
    dense = []
    for _ in range(3):
        a, b = _events()
        a.record()
        full_attention(q, k, v, mode="flash")
        b.record()
        dense.append((a, b))
    torch.cuda.synchronize()
    dense_ms = float(np.mean([a.elapsed_time(b) for a, b in dense]))
    dense_flop = 4.0 * L * L * cfg.head_dim * cfg.heads
    dense_call = {"workload": "full_attention(mode='flash') on the cfg1 inputs: every block kept, 3 timed calls "
                              "after 1 untimed",
                  "call_ms": round(dense_ms, 3), "flop": dense_flop,
                  "tflops": round(dense_flop / (dense_ms * 1e-3) / 1e12, 1),
                  "frac": round(dense_flop / (dense_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
    log(f"dense call: {dense_call}")
    return {
        "attention_bf16_operands": {"ms": round(bf16_ms, 3), "tflops": round(flops / (bf16_ms * 1e-3) / 1e12, 1),
                                    "frac": round(flops / (bf16_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                    "f16_operands_ms_same_stretch": round(f16_ms, 3)},
        "less_local_mask": less_local,
        "dense_call": dense_call,
    }


def run_cfg2(args):
    """HunyuanVideo joint attention at configs[2], fresh mask every call."""
    from dfsattn_amd.attention_hyvideo import DFS_Attention, _dfs_attention_instances, dfs_attention
    from dfsattn_amd.layout import csr_flops
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, synth_qkv

    cfg = CONFIGS[2]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("generating cfg2 inputs on the GPU")
    q, k, v = synth_qkv(cfg, device=dev)
    perm = hilbert3d_perm(*cfg.grid)
    seg = {}
    if args.text_valid is not None:
        # text padded to 256 tokens with text_valid of them valid: cu_seqlens [0, valid, L]
        # (replace_hyvideo.py:221-228), the valid and padding tokens as two sequences
        if not 0 <= args.text_valid < cfg.text_len:
            raise SystemExit(f"--text-valid must lie in [0, {cfg.text_len})")
        cu = torch.tensor([0, cfg.video_len + args.text_valid, cfg.seq_len], dtype=torch.int32)
        seg = dict(cu_seqlens_q=cu, cu_seqlens_kv=cu)

    def step():
        return dfs_attention(q, k, v, step_idx=12, skip_steps=12, cache_interval=12, layer_idx=0,
                             sparsity=cfg.sparsity, sparsity_dcrt=0.0, tile_size=cfg.tile, block_size=cfg.block,
                             video_len=cfg.video_len, video_perm=perm, cache_flag=True, **seg)

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")
    DFS_Attention.set_record_timing(True)  # phase event pairs inside the timed calls
    e0, e1 = _events()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    spans = DFS_Attention.timing_recorder.rows()
    DFS_Attention.set_record_timing(False)
    phase_of = {"qkv_permute": "prepare", "topk_mask": "score_topk", "attention_execution": "attention"}
    phase_ms = {name: float(np.mean([r["elapsed_ms"] for r in spans if r["phase"] == ph]))
                for ph, name in phase_of.items()}
    entry = next(iter(DFS_Attention._cached_metadata.values()))
    flops = csr_flops(entry["row_ptr"].cpu().numpy(), entry["col_idx"].cpu().numpy(), cfg.heads, cfg.seq_len,
                      cfg.head_dim)
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()
    log(f"cfg2: {ms:.3f} ms/call, {flops / ms / 1e9:.1f} effective TFLOP/s; phases (ms) {phase_ms}")
    pad = ("" if args.text_valid is None else
           f", text padding: {args.text_valid} valid text tokens, cu_seqlens [0, valid, L] (FLOP counted on the "
           "whole-sequence mask)")
    return {"metric": "DFS attn ms/call @119,056 tok (118,800 video + 256 text),24h,d128 bf16",
            "value": round(ms, 3), "unit": "ms/call", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16", "input_dtype": "bf16", "data": "synthetic (smoothed-field Q/K, iid V, iid text; seeded)",
            "config": {"workload": "cfg2 HunyuanVideo joint attention: 33x45x80 video + 256 text tokens, 24 heads, "
                                   "d128, tile 16, block 128, hilbert3d, sparsity 0.3, fresh mask per call" + pad,
                       "global_batch": 1, "seq_len": cfg.seq_len, "parallelism": "none (1 GPU)"},
            "effective_tflops": round(flops / ms / 1e9, 1), "kept_flop": flops,
            "frac_of_bf16_peak": round(flops / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "phases_ms": {k_: round(v_, 3) for k_, v_ in phase_ms.items()},
            "attention_kernel": {"tflops": round(flops / phase_ms["attention"] / 1e9, 1),
                                 "frac": round(flops / phase_ms["attention"] / 1e9 / PEAK_BF16_TFLOPS, 4)}}


def run_cfg3(args):
    """Mask-cache regime over a sparsity sweep: 50 calls, the
    first 12 dense (full attention on the same kernel), a mask refresh every
    12 steps, Q and K drifting by N(0, 0.02) per step."""
    from dfsattn_amd.attention_wan import DFS_Attention, _compute_cache_schedule, _dfs_attention_instances, dfs_attention
    from dfsattn_amd.fullattention import full_attention
    from dfsattn_amd.utils.order import hilbert3d_perm
    from dfsattn_amd.workloads import CONFIGS, drift, synth_qkv

    cfg = CONFIGS[1]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("generating cfg1 inputs on the GPU")
    q0, k0, v = synth_qkv(cfg, device=dev)
    perm = hilbert3d_perm(*cfg.grid)
    L = cfg.seq_len
    cu = torch.tensor([0, L, L], dtype=torch.int32, device=dev)
    steps, skip, interval = 50, 12, 12
    # One untimed sparse call and one dense call first: a process's first
    # calls allocate the scoring workspace and the dense mask and load the
    # kernels, which would otherwise land in the first sweep point's steps.
    for s in (0.1, 0.5):
        dfs_attention(q0, k0, v, step_idx=2 * skip, skip_steps=skip, cache_interval=interval, layer_idx=0,
                      sparsity=s, sparsity_dcrt=0.0, tile_size=cfg.tile, block_size=cfg.block, video_perm=perm,
                      cache_flag=True)
    full_attention(q0, k0, v, mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu, max_seqlen_q=L, max_seqlen_kv=L)
    torch.cuda.synchronize()
    runs = []
    for dcrt in (0.0, 0.1):
        for s in (0.1, 0.2, 0.3, 0.5):
            DFS_Attention.clear_cache()
            _dfs_attention_instances.clear()
            gen = torch.Generator(device=dev)
            gen.manual_seed(1234)
            q, k = q0.clone(), k0.clone()
            evs = []
            for t in range(steps):
                if t:
                    q, k = drift(q, 0.02, gen), drift(k, 0.02, gen)
                a, b = _events()
                a.record()
                if t < skip:
                    full_attention(q, k, v, mode="flash", cu_seqlens_q=cu, cu_seqlens_kv=cu, max_seqlen_q=L,
                                   max_seqlen_kv=L)
                else:
                    dfs_attention(q, k, v, step_idx=2 * t, skip_steps=skip, cache_interval=interval, layer_idx=0,
                                  sparsity=s, sparsity_dcrt=dcrt, tile_size=cfg.tile, block_size=cfg.block,
                                  video_perm=perm, cache_flag=True)
                b.record()
                evs.append((a, b))
            torch.cuda.synchronize()
            ms = [a.elapsed_time(b) for a, b in evs]
            refresh = [t for t in range(skip, steps)
                       if _compute_cache_schedule(2 * t, 2 * skip, 2 * interval, s, dcrt)[0]]
            cached = [t for t in range(skip, steps) if t not in refresh]
            mean = lambda xs: float(np.mean(xs)) if xs else None  # noqa: E731
            run = {"sparsity": s, "sparsity_dcrt": dcrt, "amortized_ms_per_step": round(mean(ms), 3),
                   "dense_step_ms": round(mean(ms[:skip]), 3),
                   "refresh_steps": refresh, "refresh_step_ms": round(mean([ms[t] for t in refresh]), 3),
                   "cached_step_ms": round(mean([ms[t] for t in cached]), 3),
                   "sparse_amortized_ms": round(mean(ms[skip:]), 3)}
            # a refresh step against the cached step right after it, which
            # runs the mask it selected (the same sparsity, also with dcrt > 0)
            pairs = [ms[t] - ms[t + 1] for t in refresh if t + 1 in cached]
            run["mask_recompute_ms"] = round(mean(pairs), 3) if pairs else None
            log(f"cfg3 s={s} dcrt={dcrt}: {run}")
            runs.append(run)
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()
    base = next(r for r in runs if r["sparsity"] == 0.3 and r["sparsity_dcrt"] == 0.0)
    return {"metric": "DFS mask-cache regime amortized ms/step @75.6k tok,40h,d128 bf16 (50 steps)",
            "value": base["amortized_ms_per_step"], "unit": "ms/step", "n_gpus": 1, "steps": steps, "warmup": 0,
            "ms_per_step": base["amortized_ms_per_step"], "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16", "input_dtype": "bf16",
            "data": "synthetic cfg1 inputs, Q/K drift N(0,0.02) per step (seeded)",
            "config": {"workload": "cfg3 mask-cache regime: 50 calls, skip_steps 12 (dense), cache_interval 12, "
                                   "value = sparsity 0.3, sparsity_dcrt 0", "global_batch": 1, "seq_len": L,
                       "parallelism": "none (1 GPU)"},
            "sweep": runs}


def run_cfg4(args):
    """Full random-init DiT denoising step: 40 Wan-sized blocks
    at 21x45x80 tokens with a 512-token text context, classifier-free
    guidance (conditional + unconditional pass, as the reference's Wan
    pipeline runs a step). The DFS step is a mask-refresh step (real step
    12: the conditional pass selects fresh masks, the unconditional pass
    reuses them); the dense step runs every self-attention with all blocks
    kept (real step 0)."""
    from dfsattn_amd import dit
    from dfsattn_amd.attention_wan import DFS_Attention, _dfs_attention_instances
    from dfsattn_amd.utils.order import hilbert3d_perm

    cfg = dit.DIT_CONFIGS["cfg4"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"building {cfg.name}: {cfg.params() / 1e9:.2f} B parameters, random init on the GPU")
    model = dit.build_model(cfg, dev)
    latent, ctx, neg = dit.synth_inputs(cfg, dev)
    timestep = torch.tensor([500.0], device=dev)
    procs = dit.install_dfs_processors(model, "dfs", 0.3, 16, 128, hilbert3d_perm(*cfg.grid), skip_steps=12,
                                       cache_interval=12, sparsity_dcrt=0.0)
    torch.cuda.synchronize()
    log("model ready")

    def timed(step_idx, label):
        for i in range(args.warmup):
            dit.set_step(procs, step_idx)
            dit.denoise_step(model, latent, timestep, ctx, neg)
            torch.cuda.synchronize()
            log(f"{label} warmup step {i + 1}/{args.warmup} done")
        e0, e1 = _events()
        e0.record()
        for i in range(args.steps):
            dit.set_step(procs, step_idx)
            out = dit.denoise_step(model, latent, timestep, ctx, neg)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        if not bool(torch.isfinite(out).all()):
            raise RuntimeError(f"{label} step produced non-finite values")
        log(f"{label} step: {ms:.1f} ms")
        return ms

    sparse_ms = timed(24, "DFS (s=0.3, refresh)") if args.dit_phase in ("both", "dfs") else None
    dense_ms = timed(0, "dense") if args.dit_phase in ("both", "dense") else None
    DFS_Attention.clear_cache()
    _dfs_attention_instances.clear()
    if sparse_ms is None:
        sparse_ms = float("nan")
    return {"metric": "DiT denoising step ms (40 blocks, 75.6k tok, d5120, CFG) with DFS self-attention s=0.3",
            "value": round(sparse_ms, 1), "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(sparse_ms, 1), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "attention_dtype": "f16",
            "data": "synthetic (random-init N(0, 0.02) bf16 weights, N(0, 1) latent and text context; seeded)",
            "config": {"workload": "cfg4 Wan-style DiT step: 40 blocks, hidden 5120, 40 heads, FFN 13824, "
                                   "QK-RMSNorm + 3D RoPE, 512x4096 text context, latent 21x45x80 tokens, "
                                   "conditional + unconditional pass, DFS refresh step (fresh masks)",
                       "global_batch": 1, "seq_len": cfg.seq_len, "parallelism": "none (1 GPU)"},
            "dense_step_ms": None if dense_ms is None else round(dense_ms, 1),
            "speedup_vs_dense": round(dense_ms / sparse_ms, 3) if sparse_ms and dense_ms else None,
            "params": cfg.params()}


def cpu_baseline(q, k, v):
    """fp32 oracle on the host cores, on the GPU run's own inputs (bf16 values
    in fp32): Hilbert permutation + pooled scoring + top-k of all 40 heads, and
    masked attention of every query block of 6 of the 40 heads (scaled x40/6).
    About 10-12 s of CPU work on a 16-core host."""
    from oracle import dfs_oracle as orc
    from dfsattn_amd.workloads import CONFIGS

    cfg = CONFIGS[1]
    att_heads = [0, 8, 16, 24, 32, 39]
    log("cpu baseline: copying the inputs to the host")
    q, k, v = (x.float().cpu() for x in (q, k, v))
    perm = torch.from_numpy(orc.hilbert3d_perm(*cfg.grid))
    log("cpu baseline: permute + scoring + top-k (40 heads)")
    t0 = time.perf_counter()
    qp, kp, vp = (orc.apply_permutation(x, perm) for x in (q, k, v))
    scores = orc.block_scores(qp, kp, cfg.tile, cfg.block, None, head_chunk=4)
    mask = orc.mask_from_scores_wan(scores, cfg.sparsity)
    t_score = time.perf_counter() - t0
    log(f"cpu baseline: scoring took {t_score:.1f} s; masked attention of {len(att_heads)} heads")
    n_qb = math.ceil(cfg.seq_len / cfg.block)
    t1 = time.perf_counter()
    orc.masked_attention(qp, kp, vp, mask, cfg.block, heads=att_heads)
    t_att = time.perf_counter() - t1
    log(f"cpu baseline: attention sample took {t_att:.1f} s")
    scale = cfg.heads / len(att_heads)
    full_s = t_score + t_att * scale
    return {
        "value": round(full_s * 1e3, 1),
        "unit": "ms/call",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"cfg1 fp32 oracle on the benchmark inputs: permute+scoring+top-k of all 40 heads "
                   f"({t_score:.1f} s) + masked attention of all {n_qb} query blocks of "
                   f"{len(att_heads)}/40 heads ({t_att:.1f} s, x{scale:.2f}); unpermute not timed"),
        "host": {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
                 "torch_threads": torch.get_num_threads(), "cpu_model": _cpu_model()},
    }


def read_traffic():
    """Per-launch HBM bytes of the attention kernel at cfg1 from the committed
    counter summary (``traffic_bytes_per_launch: N``), or None."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def copy_calibration():
    """One 1 GiB device-to-device copy (after an untimed fill), for scaling
    the FETCH_SIZE / WRITE_SIZE counters: the copy kernel's dispatch reads
    and writes exactly 2**30 bytes."""
    n = 1 << 28
    src = torch.empty(n, dtype=torch.float32, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4}), flush=True)


def gemm_calibration():
    """The sustained rate of the vendor's dense GEMM (torch.matmul, which
    runs hipBLASLt) at 16384^3 in bf16 and f16: what an MFMA-bound library
    kernel reaches on this box, next to which the attention kernel's
    fraction of the 2.5 PFLOP/s peak is read."""
    dev = torch.device("cuda:0")
    n = 16384
    res = {}
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        a = torch.randn(n, n, device=dev, dtype=dt)
        b = torch.randn(n, n, device=dev, dtype=dt)
        c = torch.empty(n, n, device=dev, dtype=dt)
        for _ in range(3):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            torch.matmul(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 10
        res[name] = {"ms": round(ms, 3), "tflops": round(2 * n ** 3 / ms / 1e9, 1),
                     "frac_of_peak": round(2 * n ** 3 / ms / 1e9 / PEAK_BF16_TFLOPS, 4)}
        del a, b, c
    print(json.dumps({"gemm_calibration": res, "shape": [n, n, n]}), flush=True)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 20; 2 for cfg4)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 5; 1 for cfg4)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--gemm-calibration", action="store_true")
    ap.add_argument("--workload", choices=("cfg1", "cfg2", "cfg3", "cfg4"), default="cfg1")
    ap.add_argument("--text-valid", type=int, default=None,
                    help="cfg2: valid text tokens of the 256 (the rest padding, cu_seqlens [0, valid, L])")
    ap.add_argument("--dit-phase", choices=("both", "dfs", "dense"), default="both",
                    help="cfg4: time the DFS step, the dense step or both")
    ap.add_argument("--headline-only", action="store_true",
                    help="cfg1: skip the bf16-operand and less-local-mask side measurements (for profiling runs)")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 2 if args.workload == "cfg4" else 20
    if args.warmup is None:
        args.warmup = 1 if args.workload == "cfg4" else 5
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the DFS hot path is benchmarked on a single MI355X "
              "(multi-GPU sharding by head is a design note, not part of this build).", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gemm_calibration:
        gemm_calibration()
        return
    if args.workload != "cfg1":
        line = {"cfg2": run_cfg2, "cfg3": run_cfg3, "cfg4": run_cfg4}[args.workload](args)
        print(json.dumps(line), flush=True)
        return
    res = run_gpu(args)
    inputs = res.pop("inputs")
    cfg2 = None
    if not args.headline_only:
        # The second BASELINE configuration (HunyuanVideo joint attention,
        # configs[2]) as extra keys of the same line: whole call, phases and
        # the attention kernel's fraction of peak over a few fresh-mask calls.
        log("cfg2 (HunyuanVideo shape) for the extra keys")
        c2 = run_cfg2(argparse.Namespace(steps=10, warmup=3, text_valid=None))
        torch.cuda.empty_cache()
        cfg2 = {"workload": "configs[2]: 33x45x80 video + 256 text tokens (119,056), 24 heads, d128, bf16, tile 16, "
                            "sparsity 0.3, fresh mask per call; 10 timed calls after 3 untimed",
                "call_ms": c2["value"], "attention_ms": c2["phases_ms"]["attention"],
                "attention_tflops": c2["attention_kernel"]["tflops"], "attention_frac": c2["attention_kernel"]["frac"],
                "call_frac": c2["frac_of_bf16_peak"], "phases_ms": c2["phases_ms"], "kept_flop": c2["kept_flop"]}
    cfg4 = None
    if not args.headline_only:
        # the whole 40-block DiT denoising step (both CFG passes)
        # with DFS self-attention at a mask-refresh step, beside the dense
        # step, one timed step each after one untimed.
        log("cfg4 (40-block DiT step) for the extra keys")
        c4 = run_cfg4(argparse.Namespace(steps=1, warmup=1, dit_phase="both"))
        torch.cuda.empty_cache()
        cfg4 = {"workload": c4["config"]["workload"] + "; 1 timed step after 1 untimed",
                "dfs_step_ms": c4["value"], "dense_step_ms": c4["dense_step_ms"],
                "speedup_vs_dense": c4["speedup_vs_dense"], "params": c4["params"]}
    cpu = None if args.no_cpu_baseline else cpu_baseline(*inputs)
    del inputs
    att_ms = res["phase_ms"]["attention"]
    line = {
        "metric": "DFS attn ms/call @75.6k tok,40h,d128 bf16; % bf16 MFMA peak on kept blocks",
        "value": round(res["ms_per_step"], 3),
        "unit": "ms/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "input_dtype": "bf16",
        "data": "synthetic (smoothed-field Q/K, iid V; seeded)",
        "config": {"workload": "cfg1 Wan single DFS call: B=1, 21x45x80=75600 tokens, 40 heads, d128, "
                               "tile 16, block 128, hilbert3d, sparsity 0.3, fresh mask per call",
                   "global_batch": 1, "seq_len": 75600, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(res["attention_tflops"], 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(res["attention_tflops"] / PEAK_BF16_TFLOPS, 4), "traffic": read_traffic(),
                     "kernel": "bsa_fwd_split_kernel", "kernel_ms": round(att_ms, 3),
                     "algorithmic_flop": res["attention_flop"]},
        "median_ms_per_call": round(res["median_ms"], 3),
        "median_of_calls": res["median_calls"],
        "phases_ms": {k_: round(v_, 3) for k_, v_ in res["phase_ms"].items()},
        "prepare_gbs": round(res["prepare_gbs"], 1),
        "kept_density": round(res["density"], 4),
        **res["side"],
        "cfg2": cfg2,
        "cfg4": cfg4,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

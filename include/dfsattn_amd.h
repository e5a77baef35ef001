/*
 * dfsattn_amd.h — C-ABI of the MI355X (gfx950) DFS sparse-attention hot path.
 *
 * Every entry point returns 0 on success and a non-zero status on failure;
 * dfs_last_error() then returns a thread-local message. Pointers are raw
 * device pointers unless stated otherwise, sizes are int64, and every GPU
 * entry point enqueues work on the caller's stream and never synchronises.
 * None of them allocates device memory: callers own every buffer.
 *
 * Tensor layouts (B = 1 everywhere, as in the reference, which asserts it at
 * dfsattn/attention_wan.py:222,288):
 *   - q, k, v, out        [H][L][D] row-major (the reference's [1,H,L,D]).
 *   - perm                int32 [L]; execution (Hilbert) row i reads source
 *                         row perm[i]. For HunyuanVideo the tail L_video..L-1
 *                         is the identity (dfsattn/attention_hyvideo.py:161-174).
 *   - q_perm, k_perm      [H][R][D], R = ceil(L/128)*128 (rows >= L are zero).
 *   - v_t                 [H][R/128][D][128] in the PV operand dtype (bf16 or
 *                         f16): each 128-token block transposed, tokens in
 *                         a fixed order inside every 16-token group.
 *   - pooled hi / lo      bf16 [H][tiles][D]: tile mean split as hi + lo.
 *   - row_ptr, col_idx    int32 CSR over the [H][Qb][Kb] block mask;
 *                         row r = h*Qb + qb, columns ascending.
 *
 * dtype codes: 0 = bf16, 1 = f16, 2 = f32.
 */
#ifndef DFSATTN_AMD_H
#define DFSATTN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dfs_stream_t; /* == hipStream_t */

enum { DFS_DTYPE_BF16 = 0, DFS_DTYPE_F16 = 1, DFS_DTYPE_F32 = 2 };

/* Last error message of the calling thread ("" if none). */
const char* dfs_last_error(void);

/* ABI version; bumped whenever a signature below changes (2: scoring workspace; 3: device cu_seqlens
 * and per-head operand exponents in the attention call, per-head overflow flags and dfs_prepare_fixup;
 * 4: separate query and key tile sizes in preparation and scoring; 5: Q read from the input by
 * the attention kernel, q_perm optional). */
int dfs_abi_version(void);

/*
 * Host function. Writes the 3D Hilbert order of an f x h x w latent grid:
 * perm_out[i] = z*h*w + y*w + x of the i-th token along the curve, with the
 * coordinate columns (x, y, z) = (w-index, h-index, f-index) and
 * num_bits = max(1, ceil(log2(max(f, h, w)))).
 * Replaces dfsattn/utils/order.py:206-258 (hilbert3d_perm), including the
 * numpy-hilbert-curve encode() it calls at order.py:250.
 */
int dfs_hilbert3d_perm(int64_t f, int64_t h, int64_t w, int64_t* perm_out);

/*
 * Bit-exact row gather: dst[h][i] = src[h][perm[i]] for i < n_perm and zero
 * rows for n_perm <= i < dst_rows. row_bytes must be a multiple of 2.
 * Out-of-range perm entries produce zero rows.
 * Replaces DFS_Attention._apply_permutation_in_place, tensor[:, :, perm, :]
 * (dfsattn/attention_wan.py:128-135; attention_hyvideo.py:177-184).
 */
int dfs_permute_gather(const void* src, const int32_t* perm, void* dst,
                       int64_t heads, int64_t src_rows, int64_t n_perm,
                       int64_t dst_rows, int64_t row_bytes, dfs_stream_t stream);

/*
 * Bit-exact row scatter (inverse permutation): dst[h][perm[i]] = src[h][i]
 * for i < n_perm. Rows of dst not named by perm are left untouched.
 * Replaces DFS_Attention._apply_inverse_permutation, tensor[:, :, inv, :]
 * with inv[perm] = arange (dfsattn/attention_wan.py:113-125, 138-145).
 */
int dfs_permute_scatter(const void* src, const int32_t* perm, void* dst,
                        int64_t heads, int64_t src_rows, int64_t n_perm,
                        int64_t dst_rows, int64_t row_bytes, dfs_stream_t stream);

/*
 * Fused permute of Q, K, V into the attention operand layouts plus mean
 * pooling of Q over q_tile_size-token tiles and of K over k_tile_size-token
 * tiles in the scoring layout (each a divisor of 128; the reference's
 * q_tile_size / k_tile_size, attention_wan.py:94-95, 192-205).
 *   dtype        0 (bf16) or 1 (f16) for the inputs q, k, v.
 *   video_len    L for Wan; the video token count for HunyuanVideo. The
 *                scoring layout is [video | zero pad to 128 | text | zero
 *                pad to ceil(L/128)*128] (attention_hyvideo.py:331-365;
 *                for Wan, attention_wan.py:176-189).
 *   operand_dtype  dtype of q_perm, k_perm and v_t: 0 keeps the bf16 bits
 *                (bf16 inputs only); 1 holds f16 (bf16 inputs are rounded
 *                to f16, exact for values inside the f16 range).
 *   q_pool_*     [H][ceil(video_len/128)*128/q_tile_size][D] (may all be
 *   k_pool_*     [H][ceil(L/128)*128/k_tile_size][D]  NULL to skip pooling:
 *                cached steps).
 *                Means of the input values, whatever operand_dtype.
 *   q_perm       may be NULL: Q is then only pooled and range-flagged, and
 *                dfs_bsa_fwd reads it from the input (q_src, q_rows).
 *   overflow     optional int32 [3][H] flags (Q, K, V per head), zeroed by
 *                the caller; entry [t][h] is set when bf16 inputs are
 *                rounded to f16 and a finite value of tensor t, head h
 *                exceeds the f16 range. Pass them to dfs_prepare_fixup.
 * Replaces the q/k/v gathers of attention_wan.py:173-174, 338-340 and the
 * padding + tile means of attention_wan.py:176-205.
 */
int dfs_prepare_qkv(const void* q, const void* k, const void* v,
                    const int32_t* perm, int64_t heads, int64_t seq_len,
                    int64_t head_dim, int dtype, int64_t video_len,
                    int64_t q_tile_size, int64_t k_tile_size, int operand_dtype,
                    void* q_perm, void* k_perm, void* v_t,
                    uint16_t* q_pool_hi, uint16_t* q_pool_lo,
                    uint16_t* k_pool_hi, uint16_t* k_pool_lo,
                    int32_t* overflow, dfs_stream_t stream);

/*
 * Completes dfs_prepare_qkv for bf16 inputs with f16 operands so that every
 * finite input is represented: for each flagged (tensor, head) it rewrites
 * that head's q_perm, k_perm or v_t from the inputs as x * 2^-e (e >= 1, the
 * smallest exponent that brings the head's largest finite |x| below 2^15)
 * and sets exps[t][h] = e; every other entry of exps ([3][H] int32) is set
 * to 0, and the flags are cleared (with q_perm NULL a flagged Q head is only
 * recorded in exps, nothing is rewritten). dfs_bsa_fwd takes exps and undoes the
 * factors exactly (powers of two). Heads within the f16 range cost one flag
 * read. No reference counterpart: the reference's kernel computes in bf16
 * (block_sparse_attn_func, attention_wan.py:379-386), whose range this keeps.
 */
int dfs_prepare_fixup(const void* q, const void* k, const void* v,
                      const int32_t* perm, int64_t heads, int64_t seq_len,
                      int64_t head_dim, void* q_perm, void* k_perm, void* v_t,
                      int32_t* overflow, int32_t* exps, dfs_stream_t stream);

/*
 * Hierarchical block scoring and top-k in one kernel: pooled QK^T * D^-1/2
 * (bf16 MFMA on the hi/lo split), softmax over all key tiles, sums of tile
 * probabilities per 128x128 block, then per-row top-k.
 *   q_tile_size, k_tile_size  tokens per pooled query / key tile, each a
 *                divisor of 128 of at least 4, as pooled by dfs_prepare_qkv
 *                (attention_wan.py:94-95, 227-246). Equal tiles of 16 or 32
 *                run the tuned kernels; any other pair runs a generic
 *                two-pass kernel that needs scores_out.
 * Row selection policy (same as dfs_topk_from_scores):
 *   scored_rows  number of query-block rows that carry scores
 *                (ceil(video_len/128)).
 *   n_cand       candidate columns 0..n_cand-1 compete for k_pick slots.
 *   dense_col    columns dense_col..Kb-1 are always kept in scored rows.
 *   dense_row    rows dense_row..Qb-1 keep every column.
 *   row_ptr      CSR row offsets [H*Qb+1] consistent with the policy.
 *   col_idx      CSR columns (ascending per row).
 *   scores_out   optional fp32 [H][scored_rows][Kb] block scores (rows from
 *                dense_row on are then scored too). Without a workspace the
 *                kernel accumulates its block sums there instead of in LDS,
 *                which lets more workgroups share a CU (faster).
 *   mask_out     optional uint8 [H][Qb][Kb] block mask.
 *   workspace    optional device buffer of workspace_bytes >= the size from
 *                dfs_block_score_topk_workspace_size (16-byte aligned). With
 *                it, and Kb <= 16 * head_dim, the kernel scores every tile
 *                pair once, keeping unnormalised per-tile block sums there,
 *                instead of twice (a normaliser pass, then a block-sum
 *                pass); scores_out is then only written, not needed.
 * Ties are broken by (score descending, column ascending).
 * Replaces _compute_tile_score + _compute_block_mask
 * (attention_wan.py:157-261; attention_hyvideo.py:310-501).
 */
int dfs_block_score_topk(const uint16_t* q_pool_hi, const uint16_t* q_pool_lo,
                         const uint16_t* k_pool_hi, const uint16_t* k_pool_lo,
                         int64_t heads, int64_t head_dim,
                         int64_t q_tile_size, int64_t k_tile_size,
                         int64_t q_blocks, int64_t k_blocks,
                         int64_t scored_rows, int64_t n_cand, int64_t k_pick,
                         int64_t dense_col, int64_t dense_row,
                         const int32_t* row_ptr, int32_t* col_idx,
                         float* scores_out, uint8_t* mask_out,
                         void* workspace, int64_t workspace_bytes,
                         dfs_stream_t stream);

/*
 * Bytes of the optional dfs_block_score_topk workspace for these sizes
 * (-1 for invalid sizes, 0 for tile sizes without a one-pass form). Host
 * function; no reference counterpart (the reference materialises the whole
 * [H, Qt, Kt] tile-score tensor instead, attention_wan.py:207-209).
 */
int64_t dfs_block_score_topk_workspace_size(int64_t heads, int64_t q_tile_size,
                                            int64_t k_tile_size, int64_t q_blocks,
                                            int64_t k_blocks);

/*
 * dfs_block_score_topk that allocates nothing and takes no caller scratch:
 * the block-sum matrix (heads * scored_rows * k_blocks fp32 values, at most
 * 96 MiB: 55.9 MB at 75.6k tokens x 40 heads, 83.0 MB at 119k tokens x 24
 * heads) lives in a static device array of the library, one per GPU, held
 * until the process ends; larger problems are rejected with an error. The
 * copy used is that of the device `stream` belongs to (the current device
 * for the null stream), whichever device is current. Runs the two-pass form
 * (no workspace); same selection as dfs_block_score_topk with scores_out and
 * no workspace. Calls that overlap on one GPU (several streams or threads)
 * share that array and race; serialise them. No
 * counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
int dfs_block_score_topk_noalloc(const uint16_t* q_pool_hi, const uint16_t* q_pool_lo,
                                 const uint16_t* k_pool_hi, const uint16_t* k_pool_lo,
                                 int64_t heads, int64_t head_dim,
                                 int64_t q_tile_size, int64_t k_tile_size,
                                 int64_t q_blocks, int64_t k_blocks,
                                 int64_t scored_rows, int64_t n_cand, int64_t k_pick,
                                 int64_t dense_col, int64_t dense_row,
                                 const int32_t* row_ptr, int32_t* col_idx,
                                 uint8_t* mask_out, dfs_stream_t stream);

/*
 * Top-k from given fp32 block scores [H][scored_rows][Kb] with the policy
 * above; emits CSR columns and an optional uint8 mask. Given the same fp32
 * scores it selects exactly the set torch.topk + scatter_ selects when no tie
 * straddles the k-th place (attention_wan.py:248-253;
 * attention_hyvideo.py:431-443, 491-501).
 */
int dfs_topk_from_scores(const float* scores, int64_t heads,
                         int64_t q_blocks, int64_t k_blocks,
                         int64_t scored_rows, int64_t n_cand, int64_t k_pick,
                         int64_t dense_col, int64_t dense_row,
                         const int32_t* row_ptr, int32_t* col_idx,
                         uint8_t* mask_out, dfs_stream_t stream);

/*
 * Block-sparse flash-attention forward over the kept 128x128 blocks.
 *   q_perm, k_perm, v_t  as produced by dfs_prepare_qkv (q_perm may be NULL
 *                        with q_src below); dtype is the dtype
 *                        of q_perm and k_perm, pv_dtype that of v_t (f16/f16
 *                        and bf16/bf16 as prepared; bf16/f16 also accepted).
 *                        With f16 q_perm the kernel folds scale * log2(e)
 *                        into Q, rounding Q * scale * log2(e) to f16 (a row
 *                        beyond the f16 range is carried with an exact
 *                        power-of-two factor).
 *   scale                softmax scale (the reference passes None -> D^-1/2).
 *   out                  out_dtype 0/1/2; when out_perm is NULL, out is
 *                        [H][L][D] in execution order; otherwise row i is
 *                        written to out[h][out_perm[i]] (fused unpermute).
 *   lse                  optional fp32 [H][L] natural-log sum-exp (execution
 *                        order).
 *   cu_seqlens_q/_k      optional device int32 [n_seq + 1] offsets of the
 *                        query and key sequences in execution order (both
 *                        or neither; n_seq 1 or 2). Sequence i: queries
 *                        [cq[i], cq[i+1]) attend keys [ck[i], ck[i+1])
 *                        under the block mask indexed from each sequence's
 *                        own start (the mask repeated per sequence); rows in
 *                        no query sequence are zero. Offsets are read on the
 *                        device (no host synchronisation) and trusted, as by
 *                        the reference's varlen kernel, clamped to [0, L].
 *                        Sequence 0 runs on the MFMA kernel, sequence 1 on
 *                        an fp32 kernel sized for short padding segments.
 *                        Without them: one sequence of L tokens.
 *   exps                 optional int32 [3][H] per-head exponents written by
 *                        dfs_prepare_fixup (q_perm, k_perm, v_t hold
 *                        x * 2^-e); NULL means all zero.
 *   q_src, q_rows        optional: Q read from the input instead of q_perm
 *                        (which may then be NULL): execution row r < L is
 *                        row q_rows[r] of q_src [H][L][D] (the permutation
 *                        dfs_prepare_qkv took), in q_src_dtype (bf16 or f16;
 *                        bf16 Q/K operands need bf16). Each workgroup reads
 *                        its 128 rows once, so the gather costs nothing
 *                        measurable and the preparation skips the q_perm
 *                        write. exps[0][h] then only marks a head whose Q
 *                        exceeds the f16 range (its rows are scaled by the
 *                        kernel, row by row).
 * Keys past a sequence's end in its last block are masked out; rows with no
 * kept block give 0. CSR columns must ascend.
 * Replaces block_sparse_attn_func (attention_wan.py:379-386;
 * attention_hyvideo.py:1075-1082), including its cu_seqlens_q /
 * cu_seqlens_k arguments, and, with out_perm, the final inverse gather
 * (attention_wan.py:390).
 */
int dfs_bsa_fwd(const void* q_perm, const void* k_perm, const void* v_t,
                const int32_t* row_ptr, const int32_t* col_idx,
                int64_t heads, int64_t seq_len, int64_t head_dim, int dtype,
                int pv_dtype, float scale, void* out, int out_dtype,
                const int32_t* out_perm, float* lse,
                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                int64_t n_seq, const int32_t* exps, const void* q_src,
                const int32_t* q_rows, int q_src_dtype, dfs_stream_t stream);

/* uint8/bool block mask [H][Qb][Kb] -> per-row counts int32 [H*Qb].
 * Part of the bool-mask interface of block_sparse_attn_func
 * (base_blockmask, attention_wan.py:359). */
int dfs_mask_row_counts(const uint8_t* mask, int64_t rows, int64_t k_blocks,
                        int32_t* counts, dfs_stream_t stream);

/* uint8/bool block mask -> CSR columns given row_ptr (exclusive scan of the
 * counts above). */
int dfs_mask_to_csr(const uint8_t* mask, int64_t rows, int64_t k_blocks,
                    const int32_t* row_ptr, int32_t* col_idx,
                    dfs_stream_t stream);

/* CSR -> uint8 block mask [rows][Kb] (the reference's cached bool
 * block_mask, attention_wan.py:252-253, 465-470). */
int dfs_csr_to_mask(const int32_t* row_ptr, const int32_t* col_idx,
                    int64_t rows, int64_t k_blocks, uint8_t* mask,
                    dfs_stream_t stream);

/*
 * Fused QK RMSNorm + complex RoPE + head split of the DiT attention inputs.
 * Element (b, l, h, d) of x is x[b*x_sb + l*x_sl + h*x_sh + d] and of out
 * out[b*o_sb + l*o_sl + h*o_sh + d] (element strides, multiples of 8; the
 * channel stride is 1), so x may be the projection output [B][L][H*D]
 * (x_sh = D) and out the attention layout [B][H][L][D] (o_sh = L*D), or both
 * the same tensor (in place). dtype (x and out): bf16 or f16.
 *   - weight != NULL: RMSNorm over the H*D channels of each token in fp32,
 *     y = (x * rstd) * w, rstd = 1/sqrt(sum(x^2)/(H*D) + eps), rounded to
 *     dtype (weight_dtype bf16, f16 or f32). Replaces triton_rmsnorm_forward
 *     (dfsattn/kernels/triton/rmsnorm.py:51) as called at
 *     replace_wan.py:163-166.
 *   - cos/sin != NULL: fp32 tables [L - rope_skip][D/2]; token l >= rope_skip
 *     has each (even, odd) channel pair of every head rotated by
 *     (cos, sin)[l - rope_skip] in float64, rounded through fp32 to dtype.
 *     Replaces apply_qk_rope_inplace_cossin_complex
 *     (dfsattn/kernels/csrc/ops.h:207-261, called at replace_wan.py:31-42
 *     with len_text_prompt = rope_skip).
 * With neither, the call is the head-split copy of replace_wan.py:181-183.
 * heads*head_dim <= 8192, head_dim a multiple of 8.
 */
int dfs_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int64_t x_sh,
                  void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
                  int64_t batch, int64_t seq_len, int64_t heads,
                  int64_t head_dim, int dtype, const void* weight,
                  int weight_dtype, float eps, const float* cos_table,
                  const float* sin_table, int64_t rope_skip,
                  dfs_stream_t stream);

/*
 * The HunyuanVideo form of the above (same layouts and strides):
 *   - weight != NULL: RMSNorm of each head's D channels (weight [D]),
 *     replacing the reference's rms_norm_forward (kernels/csrc/ops.h:52-75)
 *     as applied per head by apply_qk_norm (kernels/__init__.py), called at
 *     replace_hyvideo.py:252-253. D a power of two <= 512.
 *   - cos/sin != NULL: fp32 tables [rope_rows][D]; token l < rope_rows has
 *     each (even, odd) channel pair rotated, out[2i] = x[2i]*cos[2i] -
 *     x[2i+1]*sin[2i], out[2i+1] = x[2i+1]*cos[2i+1] + x[2i]*sin[2i+1], every
 *     product and sum rounded in fp32; the text rows after rope_rows are not
 *     rotated. Replaces apply_qk_rope_inplace_cossin_txtlast
 *     (kernels/csrc/ops.h:146-205) as called by apply_qk_rope_single/double
 *     (replace_hyvideo.py:262-268).
 */
int dfs_head_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int64_t x_sh,
                       void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
                       int64_t batch, int64_t seq_len, int64_t heads,
                       int64_t head_dim, int dtype, const void* weight,
                       int weight_dtype, float eps, const float* cos_table,
                       const float* sin_table, int64_t rope_rows,
                       dfs_stream_t stream);

/*
 * DiT block elementwise steps around the attention (the Wan transformer
 * block of diffusers that the reference's Wan driver loads,
 * wan21_t2v_inference.py:102-103; not part of the reference's own code).
 * x, out: [rows][channels] contiguous, bf16 or f16; fp32 vectors of
 * `channels` entries, each optional (NULL skips its step):
 *   out = (LayerNorm(x, eps) * weight + bias) * (1 + scale) + shift,
 * the LayerNorm over the channels in fp32 (biased variance), every product
 * and sum rounded in fp32 in that order, the result rounded to dtype.
 * channels: a multiple of 8, at most 8192.
 */
int dfs_adaln_modulate(const void* x, int64_t rows, int64_t channels,
                       int dtype, const float* weight, const float* bias,
                       const float* scale, const float* shift, float eps,
                       void* out, dfs_stream_t stream);

/* out = x + y * gate (gate fp32 [channels], broadcast over rows), computed
 * in fp32 (product rounded, then the sum) and rounded to dtype; x, y, out
 * [rows][channels] contiguous bf16 or f16 (out may alias x). */
int dfs_gated_residual(const void* x, const void* y, const float* gate,
                       int64_t rows, int64_t channels, int dtype, void* out,
                       dfs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DFSATTN_AMD_H */

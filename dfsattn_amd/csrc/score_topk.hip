// Hierarchical block scoring and per-row top-k block selection.
//
// Scoring (reference: dfsattn/attention_wan.py:157-253 and
// dfsattn/attention_hyvideo.py:310-501): with pooled tile means q_i, k_j,
//   P[i, j]      = softmax_j( q_i . k_j * D^-1/2 )   over ALL key tiles j
//   score[a, b]  = sum_{i in query block a} sum_{j in key block b} P[i, j]
// followed by a top-k over each row a. In the default (wide) kernel each of a
// workgroup's four waves owns 32 query tiles of one head; the workgroup streams
// the head's pooled key tiles in 32-tile chunks through LDS into bf16 MFMAs on
// a hi/lo split (q.k ~= qh.kh + qh.kl + ql.kh, relative error ~2^-16), so the
// scores track the fp32 computation closely. With a caller workspace the
// scores are made in one pass (per-tile block sums kept in the workspace while
// the softmax normaliser accumulates, scaled at the end); without one, pass 1
// builds the normaliser and pass 2 recomputes the scores into block sums. The
// same workgroup then selects the top-k of every row it owns, one wave per
// row, emitting CSR column indices for the attention kernel.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"
#include "lds_copy.h"

namespace dfs {
namespace {

__device__ __forceinline__ void lds_sync_wave() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

// Order-preserving map of an fp32 score to uint32 (NaN sorts above +inf, as in
// torch.topk).
__device__ __forceinline__ uint32_t order_key(float s) {
  const uint32_t u = __float_as_uint(s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive prefix sum over the 64 lanes: shifts within rows of 16, then the
// row totals carried by DPP row broadcasts.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return x;
}

__device__ __forceinline__ uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Selection of one mask row by one wave.
//  * columns [0, n_cand): the k_pick largest scores, ties broken by lower
//    column first (radix select on the order keys, up to 4 x 8-bit digits);
//  * columns [n_cand, dense_col): never kept;
//  * columns [dense_col, kb): always kept.
// cols receives the kept columns in ascending order; mask_row (optional) the
// uint8 mask. hist is 256 * NSUB words of wave-private LDS: NSUB copies of the
// digit histogram, interleaved per digit, with lane l counting into copy
// l % NSUB, so lanes whose keys share a digit split over NSUB addresses (the
// leading digits of block scores take few values, and the LDS serialises
// atomics on one address). The digits stop early once every key sharing the
// k-th key's leading digits is kept: the set is then fixed without resolving
// the remaining bits.
template <int NSUB = 1>
__device__ __forceinline__ void select_row(const float* scores, int n_cand, int k_pick, int dense_col, int kb,
                                           int32_t* cols, uint8_t* mask_row, uint32_t* hist, int lane) {
  static_assert(NSUB == 1 || NSUB == 2 || NSUB == 4, "sub-histograms per digit");
  uint32_t prefix = 0, pmask = 0;
  int remaining = k_pick;
  const uint32_t copy = static_cast<uint32_t>(lane) & (NSUB - 1);
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = lane; b < 256 * NSUB; b += kWave) hist[b] = 0;
    lds_sync_wave();
    for (int j = lane; j < n_cand; j += kWave) {
      const uint32_t key = order_key(scores[j]);
      if ((key & pmask) == prefix) atomicAdd(&hist[((key >> shift) & 255u) * NSUB + copy], 1u);
    }
    lds_sync_wave();
    // Lane i owns digits 255-4i .. 252-4i, highest first.
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = 0;
#pragma unroll
      for (int k = 0; k < NSUB; ++k) c[i] += hist[(255 - 4 * lane - i) * NSUB + k];
    }
    const uint32_t own = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_incl_scan(own);
    const uint32_t excl = incl - own;
    const bool mine = excl < static_cast<uint32_t>(remaining) &&
                      static_cast<uint32_t>(remaining) <= incl;
    int pick = 0;
    uint32_t above = excl;
    if (mine) {
      while (above + c[pick] < static_cast<uint32_t>(remaining)) above += c[pick++];
    }
    const uint64_t who = __ballot(mine);
    const int src = __ffsll(static_cast<unsigned long long>(who)) - 1;
    const uint32_t in_bin = mine ? c[pick] : 0u;
    const int digit = __builtin_amdgcn_readlane(255 - 4 * lane - pick, src);
    const uint32_t above_d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(above), src));
    const uint32_t bin = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(in_bin), src));
    prefix |= static_cast<uint32_t>(digit) << shift;
    pmask |= 255u << shift;
    remaining -= static_cast<int>(above_d);
    if (bin == static_cast<uint32_t>(remaining)) break;  // the whole bin is kept
  }
  // The k-th largest key agrees with prefix on the bits of pmask; every key
  // above that is kept, and `remaining` of the keys equal to it there, lowest
  // column first.
  const uint64_t below = lanes_below(lane);
  int out = 0, ties = 0;
  for (int base = 0; base < n_cand; base += kWave) {
    const int j = base + lane;
    const bool valid = j < n_cand;
    const uint32_t key = valid ? order_key(scores[j]) & pmask : 0u;
    const bool eq = valid && key == prefix;
    const uint64_t eqb = __ballot(eq);
    const bool take = (valid && key > prefix) ||
                      (eq && ties + __popcll(eqb & below) < remaining);
    const uint64_t tb = __ballot(take);
    if (take) cols[out + __popcll(tb & below)] = j;
    if (mask_row && valid) mask_row[j] = take ? 1 : 0;
    out += __popcll(tb);
    ties += __popcll(eqb);
  }
  if (mask_row)
    for (int j = n_cand + lane; j < dense_col; j += kWave) mask_row[j] = 0;
  for (int j = dense_col + lane; j < kb; j += kWave) {
    cols[out + (j - dense_col)] = j;
    if (mask_row) mask_row[j] = 1;
  }
}

__device__ void dense_row(int kb, int32_t* cols, uint8_t* mask_row, int lane) {
  for (int j = lane; j < kb; j += kWave) {
    cols[j] = j;
    if (mask_row) mask_row[j] = 1;
  }
}

struct Policy {
  int Qb, Kb, scored_rows, n_cand, k_pick, dense_col, dense_row;
};

struct ScoreParams {
  const uint4* q_hi;  // [H][q_tiles][D] bf16
  const uint4* q_lo;
  const uint4* k_hi;  // [H][k_tiles][D] bf16
  const uint4* k_lo;
  const int32_t* row_ptr;
  int32_t* col_idx;
  float* scores_out;
  uint8_t* mask_out;
  float* tile_sums;  // one pass: [H][workgroup][tile_cols][tiles of the workgroup] unnormalised block sums
  int tile_cols;     // key blocks of all 32-tile chunks (Kb rounded up to a chunk)
  Policy pol;
  int q_tiles, k_tiles;
  float scale_log2;
};

// S^T chunk (32 key tiles x 32 query tiles) on the hi/lo split.
template <int D>
__device__ __forceinline__ f32x16 score_chunk(const ScoreParams& p, int h, int chunk, int l32,
                                              int hl, const bf16x8* qh, const bf16x8* ql) {
  constexpr int CPR = D / 8;
  f32x16 acc = {};
  const int kt = chunk * 32 + l32;
  const bool valid = kt < p.k_tiles;
  const int64_t base = (static_cast<int64_t>(h) * p.k_tiles + (valid ? kt : 0)) * CPR + hl;
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    uint4 a_hi = valid ? p.k_hi[base + 2 * ds] : make_uint4(0, 0, 0, 0);
    uint4 a_lo = valid ? p.k_lo[base + 2 * ds] : make_uint4(0, 0, 0, 0);
    const bf16x8 kh = __builtin_bit_cast(bf16x8, a_hi);
    const bf16x8 kl = __builtin_bit_cast(bf16x8, a_lo);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[ds], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[ds], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[ds], acc, 0, 0, 0);
  }
  return acc;
}

// Query fragments of one lane (tile l32, dims hl*8.. of every 16) as
// q' = (q_hi + q_lo) * scale * log2(e) in fp32, split again into bf16 hi/lo:
// the products then arrive in log2 units with no per-score multiply, and the
// split keeps them fp32-accurate.
template <int D>
__device__ __forceinline__ void load_q_prescaled(const ScoreParams& p, bool valid, int64_t base, bf16x8* qh,
                                                 bf16x8* ql) {
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) {
    const uint4 h4 = valid ? p.q_hi[base + 2 * ds] : make_uint4(0, 0, 0, 0);
    const uint4 l4 = valid ? p.q_lo[base + 2 * ds] : make_uint4(0, 0, 0, 0);
    uint32_t hb[8], lb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = (bf16_bits_to_f32(u16_at(h4, i)) + bf16_bits_to_f32(u16_at(l4, i))) * p.scale_log2;
      hb[i] = f32_to_bf16_bits(x);
      lb[i] = f32_to_bf16_bits(x - bf16_bits_to_f32(hb[i]));
    }
    qh[ds] = __builtin_bit_cast(bf16x8, make_uint4(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16),
                                                   hb[4] | (hb[5] << 16), hb[6] | (hb[7] << 16)));
    ql[ds] = __builtin_bit_cast(bf16x8, make_uint4(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16),
                                                   lb[4] | (lb[5] << 16), lb[6] | (lb[7] << 16)));
  }
}

// Exchanges between the two lane halves (lane ^ 32) by v_permlane32_swap.
__device__ __forceinline__ float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Value of lane l ^ 1 (DPP quad permutation [1, 0, 3, 2]).
__device__ __forceinline__ float quad_swap_pairs(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int xhalf_or(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
  return static_cast<int>(r[0] | r[1]);
}
// Lanes of half 0 get a + a', lanes of half 1 get b + b' (primes: the value
// of the same lane in the other half).
__device__ __forceinline__ float xhalf_pair_sum(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Key-tile row held in accumulator register r by lane half hl (32x32 MFMA
// output layout).
__device__ __forceinline__ int acc_row(int r, int hl) { return (r >> 2) * 8 + hl * 4 + (r & 3); }

template <int D, int TPB>
__global__ void __launch_bounds__(256) score_topk_kernel(ScoreParams p) {
  constexpr int CPR = D / 8;
  constexpr int G = 32 / TPB;  // query blocks per workgroup
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const Policy& pol = p.pol;
  float* bsum = smem;                           // [G][Kb]
  float* st_m = bsum + G * pol.Kb;              // [4][2][32]
  float* st_z = st_m + 256;                     // [4][2][32]
  uint32_t* hist = reinterpret_cast<uint32_t*>(st_z + 256);  // [4][256]

  const int h = blockIdx.y;
  const int qb0 = blockIdx.x * G;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  // Rows from dense_row on keep every column; their scores are only needed
  // when the caller asks for the score matrix.
  const int score_rows = p.scores_out ? pol.scored_rows : min(pol.scored_rows, pol.dense_row);
  const bool do_score = qb0 < score_rows;

  if (do_score) {
    // Query fragments: lane column = query tile, 8 dims per lane half.
    bf16x8 qh[D / 16], ql[D / 16];
    const int qt = qb0 * TPB + l32;
    const bool qv = qt < p.q_tiles;
    const int64_t qbase = (static_cast<int64_t>(h) * p.q_tiles + (qv ? qt : 0)) * CPR + hl;
    load_q_prescaled<D>(p, qv, qbase, qh, ql);
    const int nchunks = (p.k_tiles + 31) / 32;

    // Pass 1: running max and normaliser (log2 domain) of every query tile.
    float m = -INFINITY, z = 0.f;
    for (int c = w; c < nchunks; c += 4) {
      const f32x16 acc = score_chunk<D>(p, h, c, l32, hl, qh, ql);
      float t[16];
      float cm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool kv = c * 32 + acc_row(r, hl) < p.k_tiles;
        t[r] = kv ? acc[r] : -INFINITY;
        cm = fmaxf(cm, t[r]);
      }
      const float mn = fmaxf(m, cm);
      if (mn > -INFINITY) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) s += exp2_fast(t[r] - mn);
        z = (m > -INFINITY ? z * exp2_fast(m - mn) : 0.f) + s;
        m = mn;
      }
    }
    st_m[(w * 2 + hl) * 32 + l32] = m;
    st_z[(w * 2 + hl) * 32 + l32] = z;
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) M = fmaxf(M, st_m[e * 32 + l32]);
    float Z = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float me = st_m[e * 32 + l32];
      if (me > -INFINITY) Z += st_z[e * 32 + l32] * exp2_fast(me - M);
    }
    const float invZ = Z > 0.f ? 1.0f / Z : 0.f;

    // Pass 2: tile probabilities summed into 128x128 blocks.
    for (int c = w; c < nchunks; c += 4) {
      const f32x16 acc = score_chunk<D>(p, h, c, l32, hl, qh, ql);
      float pr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool kv = c * 32 + acc_row(r, hl) < p.k_tiles;
        pr[r] = kv ? exp2_fast(acc[r] - M) * invZ : 0.f;
      }
      if constexpr (TPB == 8) {
        // Register group r/4 = key block b of the chunk; halves hold the
        // other four tiles; 8 lanes = the 8 query tiles of a block.
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float s = (pr[4 * b] + pr[4 * b + 1]) + (pr[4 * b + 2] + pr[4 * b + 3]);
          s += __shfl_xor(s, 32);
          s += __shfl_xor(s, 1);
          s += __shfl_xor(s, 2);
          s += __shfl_xor(s, 4);
          const int kbk = c * 4 + b;
          if (hl == 0 && (l32 & 7) == 0 && kbk < pol.Kb) bsum[(l32 >> 3) * pol.Kb + kbk] = s;
        }
      } else {
        // TPB == 4: register group gg and half hl form key block 2*gg + hl.
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          float s = (pr[4 * gg] + pr[4 * gg + 1]) + (pr[4 * gg + 2] + pr[4 * gg + 3]);
          s += __shfl_xor(s, 1);
          s += __shfl_xor(s, 2);
          const int kbk = c * 8 + 2 * gg + hl;
          if ((l32 & 3) == 0 && kbk < pol.Kb) bsum[(l32 >> 2) * pol.Kb + kbk] = s;
        }
      }
    }
    __syncthreads();
    if (p.scores_out) {
      for (int i = tid; i < G * pol.Kb; i += 256) {
        const int g = i / pol.Kb, col = i - g * pol.Kb;
        const int qb = qb0 + g;
        if (qb < pol.scored_rows)
          p.scores_out[(static_cast<int64_t>(h) * pol.scored_rows + qb) * pol.Kb + col] = bsum[i];
      }
    }
  }

  for (int g = w; g < G; g += 4) {
    const int qb = qb0 + g;
    if (qb >= pol.Qb) break;
    const int64_t row = static_cast<int64_t>(h) * pol.Qb + qb;
    int32_t* cols = p.col_idx + p.row_ptr[row];
    uint8_t* mrow = p.mask_out ? p.mask_out + row * pol.Kb : nullptr;
    if (qb >= pol.dense_row || qb >= pol.scored_rows)
      dense_row(pol.Kb, cols, mrow, lane);
    else
      select_row(bsum + g * pol.Kb, pol.n_cand, pol.k_pick, pol.dense_col, pol.Kb, cols, mrow,
                 hist + w * 256, lane);
  }
}

// (head, workgroup within the head) of this workgroup in a grid of
// (workgroups per head) x (heads). Workgroups are dispatched round-robin over
// the 8 XCDs in linear order; when the heads divide evenly, XCD x takes heads
// x, x + 8, ... whole, so the workgroups that stream one head's pooled keys
// share one L2 instead of fetching the same chunks into eight (cfg1: 1/8 of
// them on each XCD, 2.08 GB leaving L2 per launch for 0.64 GB of inputs and
// workspace).
__device__ __forceinline__ void head_major_xcd(int& h, int& wgx) {
  const int nx = gridDim.x, heads = gridDim.y;
  if ((heads & 7) != 0) {
    h = blockIdx.y;
    wgx = blockIdx.x;
    return;
  }
  const int lin = blockIdx.y * nx + blockIdx.x, i = lin >> 3;
  h = (lin & 7) + 8 * (i / nx);
  wgx = i - (i / nx) * nx;
}

// Wide variant: each of the four waves owns its own 32 query tiles (G = 4 *
// 32 / TPB query blocks per workgroup) and every 32-tile chunk of pooled keys
// (hi and lo) is copied once into LDS, double-buffered, for all four waves:
// a quarter of the key traffic of one workgroup per 32 query tiles. The two
// passes run as one stream of 2 * nchunks chunk steps with one barrier each.
// GB (global block sums): the block sums go straight to scores_out (which
// the caller provides) instead of LDS, so a workgroup needs only its key
// chunks and the top-k histograms in LDS and four workgroups fit on a CU.
template <int D, int TPB, bool GB, bool ONE_PASS = false>
__global__ void __launch_bounds__(256, 2) score_topk_wide_kernel(ScoreParams p) {
  constexpr int CPR = D / 8;             // 16-byte chunks per pooled row
  constexpr int QBW = 32 / TPB;          // query blocks per wave
  constexpr int G = 4 * QBW;             // query blocks per workgroup
  constexpr int ROWS = 32;               // key tiles per chunk
  constexpr int TILE = ROWS * D;         // uint16 elements of one hi (or lo) chunk
  constexpr int LOADS = ROWS * D * 2 / 4096;  // 16-byte loads per thread per hi (or lo) chunk
  // The two key-chunk buffers are separate LDS objects ([hi, lo] each), and
  // every chunk step knows its buffer at compile time: the compiler then sees
  // that the copy into one buffer cannot alias the reads of the other and
  // does not wait for the copy in flight before reading the current chunk.
  __shared__ __attribute__((aligned(16))) uint16_t kbuf0[2][TILE];
  __shared__ __attribute__((aligned(16))) uint16_t kbuf1[2][TILE];
  __shared__ float inv_z[ONE_PASS ? 128 : 1];  // one pass: 1/Z of the workgroup's query tiles
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const Policy& pol = p.pol;
  int h, wgx;
  head_major_xcd(h, wgx);
  const int qb0 = wgx * G;
  // [G][Kb] block sums of this workgroup's query blocks
  float* bsum = GB ? (p.scores_out ? p.scores_out + (static_cast<int64_t>(h) * pol.scored_rows + qb0) * pol.Kb
                                   : nullptr)
                   : smem;
  // [4 waves][256 digits][SEL_SUB copies] of the top-k histograms
  constexpr int SEL_SUB = GB ? 4 : 1;
  uint32_t* hist = reinterpret_cast<uint32_t*>(GB ? smem : smem + G * pol.Kb);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int score_rows = p.scores_out ? pol.scored_rows : min(pol.scored_rows, pol.dense_row);
  const int qbw = qb0 + w * QBW;  // first query block of this wave

  if (qb0 < score_rows) {
    bf16x8 qh[D / 16], ql[D / 16];
    const int qt = qbw * TPB + l32;
    const bool qv = qt < p.q_tiles;
    const int64_t qbase = (static_cast<int64_t>(h) * p.q_tiles + (qv ? qt : 0)) * CPR + hl;
    load_q_prescaled<D>(p, qv, qbase, qh, ql);
#pragma unroll
    for (int ds = 0; ds < D / 16; ++ds) asm volatile("" ::"v"(qh[ds]), "v"(ql[ds]));
    const bool wave_scores = qbw < score_rows;
    const int nchunks = (p.k_tiles + ROWS - 1) / ROWS;
    const uint32_t head_bytes = static_cast<uint32_t>(p.k_tiles) * D * 2;
    const auto hrs = make_rsrc(p.k_hi + static_cast<int64_t>(h) * p.k_tiles * CPR, head_bytes);
    const auto lrs = make_rsrc(p.k_lo + static_cast<int64_t>(h) * p.k_tiles * CPR, head_bytes);
    const int ws = __builtin_amdgcn_readfirstlane(w);
    const TileCopy<D * 2> copy(ws, lane);
    constexpr uint32_t CHUNK_BYTES = ROWS * D * 2;
    // Step s (s < nchunks: chunk s; in pass 2 of the two-pass form, chunk
    // s - nchunks) reads buffer s & 1; the buffer is a template argument.
    constexpr std::integral_constant<int, 0> B0{};
    constexpr std::integral_constant<int, 1> B1{};
    auto issue = [&](int step, auto buf) {
      // Past the last step the copy reloads chunk 0 into the buffer nobody
      // reads any more, so the wait count stays fixed and every load stays in
      // range.
      uint16_t(&kb)[2][TILE] = decltype(buf)::value ? kbuf1 : kbuf0;
      const int c = step < 2 * nchunks ? (step < nchunks ? step : step - nchunks) : 0;
      copy.template issue<LOADS>(hrs, c * CHUNK_BYTES, &kb[0][0], ws);
      copy.template issue<LOADS>(lrs, c * CHUNK_BYTES, &kb[1][0], ws);
    };
    // fn(s, buffer of s) for s in [s0, s1), buffers as compile-time constants.
    auto for_steps = [&](int s0, int s1, auto fn) {
      int st = s0;
      if ((st & 1) && st < s1) fn(st++, B1);
      for (; st + 1 < s1; st += 2) {
        fn(st, B0);
        fn(st + 1, B1);
      }
      if (st < s1) fn(st, B0);
    };
    // S'^T chunk (32 key tiles x 32 query tiles) on the hi/lo split, Q
    // prescaled so S' is in log2 units. The two K operand reads of step ds + 1
    // are issued before the three MFMAs of step ds (pinned by scheduling-group
    // barriers), so their LDS latency runs under those MFMAs.
    auto chunk_scores = [&](auto buf) {
      uint16_t(&kb)[2][TILE] = decltype(buf)::value ? kbuf1 : kbuf0;
      const uint16_t* kh = &kb[0][0];
      const uint16_t* kl = &kb[1][0];
      constexpr int DS = D / 16;
      uint4 ah[2], al[2];
      ah[0] = lds_chunk<CPR>(kh, l32, hl);
      al[0] = lds_chunk<CPR>(kl, l32, hl);
      f32x16 acc = {};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        if (ds + 1 < DS) {
          ah[(ds + 1) & 1] = lds_chunk<CPR>(kh, l32, (ds + 1) * 2 + hl);
          al[(ds + 1) & 1] = lds_chunk<CPR>(kl, l32, (ds + 1) * 2 + hl);
        }
        const bf16x8 a = __builtin_bit_cast(bf16x8, ah[ds & 1]);
        const bf16x8 b = __builtin_bit_cast(bf16x8, al[ds & 1]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qh[ds], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, ql[ds], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, qh[ds], acc, 0, 0, 0);
      }
      constexpr int kMfma = 0x008, kDsRead = 0x100;
      __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 0);
#pragma unroll
      for (int ds = 0; ds + 1 < DS; ++ds) {
        __builtin_amdgcn_sched_group_barrier(kDsRead, 2, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, 3, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kMfma, 3, 0);
      return acc;
    };

    issue(0, B0);
    if constexpr (ONE_PASS) {
      // One pass: exp2(s - m) against a reference m shared by the two lane
      // halves of a query tile (the first chunk's maximum; moved only when a
      // chunk's sum exceeds 2^64, as below), summed per (query tile, key
      // block) into the workspace row of the tile while the normaliser z
      // accumulates; the rows are scaled by 1/Z and summed into blocks at the
      // end. Half the MFMA work of the two-pass form.
      // Workspace of this workgroup: [tile_cols][G * TPB] (key block major), so
      // the 32 tiles of a wave write and read each key block's sums as one
      // contiguous 128-byte line. U(kb) is this lane's tile's sum for key block kb.
      constexpr int WG_TILES = G * TPB;
      float* const ubase = p.tile_sums +
                           (static_cast<int64_t>(h) * gridDim.x + wgx) * p.tile_cols * WG_TILES + w * 32 + l32;
      auto U = [&](int kb) -> float& { return ubase[static_cast<int64_t>(kb) * WG_TILES]; };
      constexpr int BPC = ROWS / TPB;  // key blocks per chunk
      constexpr int NST = BPC / 2;     // key-block sums one lane stores per chunk
      // Workspace column of pending sum j of chunk c for this lane.
      auto st_col = [&](int c, int j) { return TPB == 8 ? c * 4 + 2 * hl + j : c * 8 + 2 * j + hl; };
      float m = -INFINITY, z = 0.f;
      float pend[NST];  // this lane's sums of the previous chunk, stored one step late
      // A chunk's sums are stored one step late, after the next chunk's
      // barrier, copy issue and operand reads, so the wait for that copy at
      // the top of a step does not also wait for stores issued just before it.
      auto flush = [&](int c) {
#pragma unroll
        for (int j = 0; j < NST; ++j) U(st_col(c, j)) = pend[j];
      };
      for_steps(0, nchunks, [&](int c, auto buf) {
        wait_vmcnt_0();
        block_barrier();
        issue(c + 1, std::integral_constant<int, 1 - decltype(buf)::value>{});
        if (!wave_scores) return;
        const f32x16 acc = chunk_scores(buf);  // s' (log2 units)
        // The previous chunk's sums go out after this chunk's operand reads:
        // issued before them, the stores made the compiler wait for part of
        // the next chunk's copy ahead of the reads in every other step.
        if (c > 0) flush(c - 1);
        const int lim = (c + 1) * ROWS <= p.k_tiles ? ROWS : p.k_tiles - c * ROWS;  // valid key tiles
        auto joint_max = [&]() {
          float cm = -INFINITY;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row(r, hl) < lim) cm = fmaxf(cm, acc[r]);
          return xhalf_max(cm);
        };
        // exp2(s' - ref) summed over the four key tiles of register group b
        // (u[b]); returns this lane's sum over all its key tiles. Only the
        // last chunk can hold key tiles past the end.
        float u[4];
        auto sums = [&](float ref) {
          float pr[16];
          if (lim == ROWS) {
#pragma unroll
            for (int r = 0; r < 16; ++r) pr[r] = exp2_fast(acc[r] - ref);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) pr[r] = acc_row(r, hl) < lim ? exp2_fast(acc[r] - ref) : 0.f;
          }
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) u[g4] = (pr[4 * g4] + pr[4 * g4 + 1]) + (pr[4 * g4 + 2] + pr[4 * g4 + 3]);
          return (u[0] + u[1]) + (u[2] + u[3]);
        };
        if (!(m > -INFINITY)) m = joint_max();  // the first chunk with valid keys
        float sum = sums(m);
        const int ovf = xhalf_or(!(sum <= 0x1p64f));
        if (__any(ovf)) {
          if (ovf) {  // a logit far above the reference: move it to this chunk's maximum
            const float mn = fmaxf(m, joint_max());
            const float f = exp2_fast(m - mn);
            z *= f;
            __threadfence_block();  // this lane's earlier row stores are visible to its loads
            for (int j = hl; j < c * BPC; j += 2) U(j) *= f;
            m = mn;
          }
          sum = sums(m);
        }
        z += sum;
        if constexpr (TPB == 8) {
          // Register group b holds key block b of the chunk, its 8 key tiles
          // split over the two lane halves: half 0 keeps blocks 0, 1 and
          // half 1 blocks 2, 3, each summed over both halves.
          pend[0] = xhalf_pair_sum(u[0], u[2]);
          pend[1] = xhalf_pair_sum(u[1], u[3]);
        } else {
#pragma unroll
          for (int j = 0; j < NST; ++j) pend[j] = u[j];  // group j, half hl: key block 2j + hl
        }
      });
      if (wave_scores && nchunks > 0) flush(nchunks - 1);
      wait_vmcnt_0();  // the trailing (empty) copies and the last sums have retired
      if (wave_scores) {
        const float Z = xhalf_sum(z);  // same reference in both halves
        if (hl == 0) inv_z[w * 32 + l32] = Z > 0.f ? 1.0f / Z : 0.f;
      }
      __threadfence_block();  // the workspace rows written above are visible to the workgroup's loads
      __syncthreads();        // inv_z is written and no wave reads the key chunks any more
    } else {
    // Pass 1: normaliser z of every query tile (one per lane half) against a
    // reference m in the log2 domain: m is the maximum of the tile's first
    // chunk; later chunks add exp2(s - m) without a maximum, and only a
    // chunk whose sum exceeds 2^64 (some s - m > 64) moves m. Any reference
    // gives the same softmax; with terms at most 2^64 and fp32's range down
    // to 2^-126 nothing of weight is lost and no block sum can overflow.
    // Only the last chunk can hold key tiles past the end.
    float m = -INFINITY, z = 0.f;
    for_steps(0, nchunks, [&](int c, auto buf) {
      wait_vmcnt_0();
      block_barrier();
      issue(c + 1, std::integral_constant<int, 1 - decltype(buf)::value>{});
      if (wave_scores) {
        const f32x16 acc = chunk_scores(buf);
        const int lim = (c + 1) * ROWS <= p.k_tiles ? ROWS : p.k_tiles - c * ROWS;  // valid key tiles
        auto masked_max = [&]() {
          float cm = -INFINITY;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row(r, hl) < lim) cm = fmaxf(cm, acc[r]);
          return cm;
        };
        auto exp_sum = [&](float ref) {
          float sum = 0.f;
          if (lim == ROWS) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sum += exp2_fast(acc[r] - ref);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (acc_row(r, hl) < lim) sum += exp2_fast(acc[r] - ref);
          }
          return sum;
        };
        if (!(m > -INFINITY)) m = masked_max();  // the tile's first chunk (stays -inf without valid keys)
        if (m > -INFINITY) {
          float sum = exp_sum(m);
          if (!(sum <= 0x1p64f)) {  // a logit far above the reference: move it to this chunk's maximum
            const float mn = fmaxf(m, masked_max());
            z *= exp2_fast(m - mn);
            m = mn;
            sum = exp_sum(m);
          }
          z += sum;
        }
      }
    });
    // Combine the two lane halves (same query tile, different key tiles).
    const float m_o = __shfl_xor(m, 32), z_o = __shfl_xor(z, 32);
    const float M = fmaxf(m, m_o);
    float Z = 0.f;
    if (m > -INFINITY) Z += z * exp2_fast(m - M);
    if (m_o > -INFINITY) Z += z_o * exp2_fast(m_o - M);
    const float invZ = Z > 0.f ? 1.0f / Z : 0.f;

    // Pass 2: tile probabilities summed into 128x128 blocks.
    for_steps(nchunks, 2 * nchunks, [&](int step, auto buf) {
      const int c = step - nchunks;
      wait_vmcnt_0();
      block_barrier();
      issue(step + 1, std::integral_constant<int, 1 - decltype(buf)::value>{});
      if (!wave_scores) return;
      const f32x16 acc = chunk_scores(buf);
      float pr[16];
      if ((c + 1) * ROWS <= p.k_tiles) {
#pragma unroll
        for (int r = 0; r < 16; ++r) pr[r] = exp2_fast(acc[r] - M);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          pr[r] = c * ROWS + acc_row(r, hl) < p.k_tiles ? exp2_fast(acc[r] - M) : 0.f;
      }
      // exp2(s - M) summed over a query tile's key tiles of the block, scaled
      // by that tile's 1/Z, then summed over the block's query tiles
      if constexpr (TPB == 8) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float sum = (pr[4 * b] + pr[4 * b + 1]) + (pr[4 * b + 2] + pr[4 * b + 3]);
          sum += __shfl_xor(sum, 32);
          sum *= invZ;
          sum += __shfl_xor(sum, 1);
          sum += __shfl_xor(sum, 2);
          sum += __shfl_xor(sum, 4);
          const int kbk = c * 4 + b;
          const int g = w * QBW + (l32 >> 3);
          if (hl == 0 && (l32 & 7) == 0 && kbk < pol.Kb && (!GB || qb0 + g < pol.scored_rows))
            bsum[g * pol.Kb + kbk] = sum;
        }
      } else {
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          float sum = ((pr[4 * gg] + pr[4 * gg + 1]) + (pr[4 * gg + 2] + pr[4 * gg + 3])) * invZ;
          sum += __shfl_xor(sum, 1);
          sum += __shfl_xor(sum, 2);
          const int kbk = c * 8 + 2 * gg + hl;
          const int g = w * QBW + (l32 >> 2);
          if ((l32 & 3) == 0 && kbk < pol.Kb && (!GB || qb0 + g < pol.scored_rows)) bsum[g * pol.Kb + kbk] = sum;
        }
      }
    });
    wait_vmcnt_0();  // the trailing (empty) copies have retired
    __syncthreads();  // with GB: the block sums in global memory are visible to the workgroup
    }
    if (!GB && p.scores_out) {
      for (int i = tid; i < G * pol.Kb; i += 256) {
        const int g = i / pol.Kb, col = i - g * pol.Kb;
        const int qb = qb0 + g;
        if (qb < pol.scored_rows)
          p.scores_out[(static_cast<int64_t>(h) * pol.scored_rows + qb) * pol.Kb + col] = bsum[i];
      }
    }
  }

  if constexpr (ONE_PASS) {
    // Block sums of a row: the sum over its TPB query tiles of (workspace
    // sum) / Z. They are formed for a group of the wave's rows at a time in
    // wave-private LDS rows (the freed key-chunk buffers, ROW_CAP floats per
    // wave), written to scores_out when the caller asked for scores, and the
    // selection reads the LDS rows. The workspace is swept in whole 128-byte
    // lines: lane l reads tiles 4 (l % 8) .. +3 of key block kb0 + l / 8, so
    // one load instruction covers 8 key blocks of the wave's 32 tiles.
    constexpr int ROW_CAP = TILE / 2;  // floats: each key-chunk buffer (2 x TILE uint16) holds two waves' rows
    constexpr int WG_TILES = G * TPB;
    float* const rowbuf = reinterpret_cast<float*>(w < 2 ? &kbuf0[0][0] : &kbuf1[0][0]) + (w & 1) * ROW_CAP;
    const int sub = lane & 7, kq = lane >> 3;
    const int gl = TPB == 8 ? sub >> 1 : sub;            // the row (of the wave's QBW) of this lane's tiles
    const bool writer = TPB == 8 ? (sub & 1) == 0 : true;  // holds the row's sum after the pair exchange
    float iz[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) iz[i] = inv_z[w * 32 + 4 * sub + i];
    const float* src = p.tile_sums + (static_cast<int64_t>(h) * gridDim.x + wgx) * p.tile_cols * WG_TILES +
                       w * 32 + 4 * sub;
    const int rs = max(1, min(QBW, ROW_CAP / pol.Kb));  // rows per group
    int row_beg[QBW];  // CSR starts of the wave's rows, loaded ahead of the sweep
#pragma unroll
    for (int g = 0; g < QBW; ++g)
      row_beg[g] = qbw + g < pol.Qb ? p.row_ptr[static_cast<int64_t>(h) * pol.Qb + qbw + g] : 0;
    for (int g0 = 0; g0 < QBW; g0 += rs) {
      const int ng = min(rs, QBW - g0);
      if (qbw + g0 < min(score_rows, pol.Qb)) {
        const int qbl = qbw + gl;
        const bool need = gl >= g0 && gl < g0 + ng;  // this lane's tiles belong to a row of the group
        const bool mine = writer && need && qbl < score_rows;
        float* dst = rowbuf + (gl - g0) * pol.Kb;
        float* out = p.scores_out && mine ? p.scores_out + (static_cast<int64_t>(h) * pol.scored_rows + qbl) * pol.Kb
                                          : nullptr;
        for (int kb0 = 0; kb0 < pol.Kb; kb0 += 64) {
          float4 a[8];  // eight loads in flight
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int kb = kb0 + 8 * j + kq;
            a[j] = need && kb < pol.Kb
                       ? *reinterpret_cast<const float4*>(src + static_cast<int64_t>(kb) * WG_TILES)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int kb = kb0 + 8 * j + kq;
            float v = (a[j].x * iz[0] + a[j].y * iz[1]) + (a[j].z * iz[2] + a[j].w * iz[3]);
            if constexpr (TPB == 8) v += quad_swap_pairs(v);  // the row's other four tiles
            if (mine && kb < pol.Kb) {
              dst[kb] = v;
              if (out) out[kb] = v;
            }
          }
        }
        lds_sync_wave();
      }
      for (int g = g0; g < g0 + ng; ++g) {
        const int qb = qbw + g;
        if (qb >= pol.Qb) break;
        const int64_t row = static_cast<int64_t>(h) * pol.Qb + qb;
        int32_t* cols = p.col_idx + row_beg[g];
        uint8_t* mrow = p.mask_out ? p.mask_out + row * pol.Kb : nullptr;
        if (qb >= pol.dense_row || qb >= pol.scored_rows)
          dense_row(pol.Kb, cols, mrow, lane);
        else
          select_row<SEL_SUB>(rowbuf + (g - g0) * pol.Kb, pol.n_cand, pol.k_pick, pol.dense_col, pol.Kb, cols,
                              mrow, hist + w * 256 * SEL_SUB, lane);
      }
      lds_sync_wave();  // the next group may overwrite rowbuf
    }
  } else {
    for (int g = 0; g < QBW; ++g) {
      const int qb = qbw + g;
      if (qb >= pol.Qb) break;
      const int64_t row = static_cast<int64_t>(h) * pol.Qb + qb;
      int32_t* cols = p.col_idx + p.row_ptr[row];
      uint8_t* mrow = p.mask_out ? p.mask_out + row * pol.Kb : nullptr;
      if (qb >= pol.dense_row || qb >= pol.scored_rows)
        dense_row(pol.Kb, cols, mrow, lane);
      else
        select_row<SEL_SUB>(bsum + (w * QBW + g) * pol.Kb, pol.n_cand, pol.k_pick, pol.dense_col, pol.Kb, cols,
                            mrow, hist + w * 256 * SEL_SUB, lane);
    }
  }
}

// Block sums of one 32 x 32 chunk of tile probabilities for TPBK key tiles
// per block. pr[r] is this lane's exp2(s - M) for key tile acc_row(r, hl) of
// the chunk and query tile l32, inv_z that query tile's 1/Z. The sum runs over
// a block's key tiles inside the lane (across the lane halves too when a
// block spans them), then 1/Z is applied, then the sum runs over the tpbq
// lanes (query tiles) of a query block. store(qbl, kbl, v) is called by one
// lane per (query block l32 / tpbq of the wave, key block kbl of the chunk).
template <int TPBK, typename Store>
__device__ __forceinline__ void chunk_block_sums(const float* pr, float inv_z, int tpbq, int l32, int hl,
                                                 Store store) {
  constexpr int NV = TPBK <= 4 ? 16 / TPBK : 32 / TPBK;  // key blocks this lane holds sums of
  float v[NV];
  if constexpr (TPBK <= 4) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float* x = pr + i * TPBK;
      if constexpr (TPBK == 1) v[i] = x[0];
      else if constexpr (TPBK == 2) v[i] = x[0] + x[1];
      else v[i] = (x[0] + x[1]) + (x[2] + x[3]);
    }
  } else {
    constexpr int GPB = TPBK / 8;  // register groups of four per key block
#pragma unroll
    for (int b = 0; b < NV; ++b) {
      float t = 0.f;
#pragma unroll
      for (int g = b * GPB; g < (b + 1) * GPB; ++g) t += (pr[4 * g] + pr[4 * g + 1]) + (pr[4 * g + 2] + pr[4 * g + 3]);
      v[b] = t + __shfl_xor(t, 32);  // the block's other half of key tiles
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] *= inv_z;
  for (int off = 1; off < tpbq; off <<= 1)
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] += __shfl_xor(v[i], off);
  if ((l32 & (tpbq - 1)) != 0 || (TPBK >= 8 && hl != 0)) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) store(l32 / tpbq, TPBK <= 4 ? acc_row(i * TPBK, hl) / TPBK : i, v[i]);
}

// Scoring and selection for any query and key tile sizes from 4 to 128
// tokens (q_tile_size and k_tile_size independent, each dividing the block),
// as the reference allows (attention_wan.py:227-246; attention_hyvideo.py:
// 406-422). A plainer form of the wide kernel: each wave owns 32 query tiles
// (32 / tpbq query blocks) and reads the pooled key chunks straight from
// global memory; pass 1 builds each query tile's softmax normaliser, pass 2
// recomputes the chunk scores into block sums in scores_out (which the caller
// provides); then the workgroup's rows are selected. Same hi/lo-split
// products as the tuned kernels, so the scores are as accurate.
template <int D>
__global__ void __launch_bounds__(256) score_topk_tiles_kernel(ScoreParams p, int tpbq, int tpbk) {
  constexpr int CPR = D / 8;
  __shared__ uint32_t hist[4][256];
  const Policy& pol = p.pol;
  const int h = blockIdx.y;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int qbw_n = 32 / tpbq;           // query blocks per wave
  const int G = 4 * qbw_n;                // query blocks per workgroup
  const int qb0 = blockIdx.x * G, qbw = qb0 + w * qbw_n;
  const int rows_to_score = pol.scored_rows;  // scores_out holds every scored row
  float* const bsum = p.scores_out + static_cast<int64_t>(h) * pol.scored_rows * pol.Kb;
  if (qbw < rows_to_score) {
    bf16x8 qh[D / 16], ql[D / 16];
    const int qt = qbw * tpbq + l32;
    const bool qv = qt < p.q_tiles;
    load_q_prescaled<D>(p, qv, (static_cast<int64_t>(h) * p.q_tiles + (qv ? qt : 0)) * CPR + hl, qh, ql);
    const int nchunks = (p.k_tiles + 31) / 32;
    // Pass 1: normaliser of each query tile against a running maximum (log2 units).
    float m = -INFINITY, z = 0.f;
    for (int c = 0; c < nchunks; ++c) {
      const f32x16 acc = score_chunk<D>(p, h, c, l32, hl, qh, ql);
      float cm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (c * 32 + acc_row(r, hl) < p.k_tiles) cm = fmaxf(cm, acc[r]);
      const float mn = fmaxf(m, cm);
      if (mn > -INFINITY) {
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (c * 32 + acc_row(r, hl) < p.k_tiles) sum += exp2_fast(acc[r] - mn);
        z = (m > -INFINITY ? z * exp2_fast(m - mn) : 0.f) + sum;
        m = mn;
      }
    }
    const float m_o = __shfl_xor(m, 32), z_o = __shfl_xor(z, 32);
    const float M = fmaxf(m, m_o);
    float Z = 0.f;
    if (m > -INFINITY) Z += z * exp2_fast(m - M);
    if (m_o > -INFINITY) Z += z_o * exp2_fast(m_o - M);
    const float inv_z = Z > 0.f ? 1.0f / Z : 0.f;
    // Pass 2: block sums of the tile probabilities.
    const int bpc = 32 / tpbk;  // key blocks per chunk
    for (int c = 0; c < nchunks; ++c) {
      const f32x16 acc = score_chunk<D>(p, h, c, l32, hl, qh, ql);
      float pr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        pr[r] = c * 32 + acc_row(r, hl) < p.k_tiles ? exp2_fast(acc[r] - M) : 0.f;
      auto store = [&](int qbl, int kbl, float val) {
        const int qb = qbw + qbl, kb = c * bpc + kbl;
        if (qb < rows_to_score && kb < pol.Kb) bsum[static_cast<int64_t>(qb) * pol.Kb + kb] = val;
      };
      switch (tpbk) {
        case 1: chunk_block_sums<1>(pr, inv_z, tpbq, l32, hl, store); break;
        case 2: chunk_block_sums<2>(pr, inv_z, tpbq, l32, hl, store); break;
        case 4: chunk_block_sums<4>(pr, inv_z, tpbq, l32, hl, store); break;
        case 8: chunk_block_sums<8>(pr, inv_z, tpbq, l32, hl, store); break;
        case 16: chunk_block_sums<16>(pr, inv_z, tpbq, l32, hl, store); break;
        default: chunk_block_sums<32>(pr, inv_z, tpbq, l32, hl, store); break;
      }
    }
  }
  __threadfence_block();  // the block sums in global memory are visible to the workgroup's loads
  __syncthreads();
  for (int g = w; g < G; g += 4) {
    const int qb = qb0 + g;
    if (qb >= pol.Qb) break;
    const int64_t row = static_cast<int64_t>(h) * pol.Qb + qb;
    int32_t* cols = p.col_idx + p.row_ptr[row];
    uint8_t* mrow = p.mask_out ? p.mask_out + row * pol.Kb : nullptr;
    if (qb >= pol.dense_row || qb >= pol.scored_rows)
      dense_row(pol.Kb, cols, mrow, lane);
    else
      select_row(bsum + static_cast<int64_t>(qb) * pol.Kb, pol.n_cand, pol.k_pick, pol.dense_col, pol.Kb, cols,
                 mrow, hist[w], lane);
  }
}

struct TopkParams {
  const float* scores;  // [H][scored_rows][Kb]
  const int32_t* row_ptr;
  int32_t* col_idx;
  uint8_t* mask_out;
  Policy pol;
  int heads;
};

__global__ void __launch_bounds__(256) topk_rows_kernel(TopkParams p) {
  __shared__ uint32_t hist[4][256];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + w;
  const Policy& pol = p.pol;
  if (row >= static_cast<int64_t>(p.heads) * pol.Qb) return;
  const int h = static_cast<int>(row / pol.Qb), qb = static_cast<int>(row % pol.Qb);
  int32_t* cols = p.col_idx + p.row_ptr[row];
  uint8_t* mrow = p.mask_out ? p.mask_out + row * pol.Kb : nullptr;
  if (qb >= pol.dense_row || qb >= pol.scored_rows) {
    dense_row(pol.Kb, cols, mrow, lane);
    return;
  }
  const float* srow = p.scores + (static_cast<int64_t>(h) * pol.scored_rows + qb) * pol.Kb;
  select_row(srow, pol.n_cand, pol.k_pick, pol.dense_col, pol.Kb, cols, mrow, hist[w], lane);
}

int check_policy(const char* name, int64_t heads, int64_t q_blocks, int64_t k_blocks,
                 int64_t scored_rows, int64_t n_cand, int64_t k_pick, int64_t dense_col,
                 int64_t dense_row_start) {
  DFS_REQUIRE(heads > 0 && heads < 65536, "%s: heads=%lld out of range", name, (long long)heads);
  DFS_REQUIRE(q_blocks > 0 && k_blocks > 0 && q_blocks < (1 << 20) && k_blocks < (1 << 20),
              "%s: q_blocks=%lld / k_blocks=%lld out of range", name, (long long)q_blocks,
              (long long)k_blocks);
  DFS_REQUIRE(scored_rows >= 0 && scored_rows <= q_blocks, "%s: scored_rows=%lld not in [0, %lld]",
              name, (long long)scored_rows, (long long)q_blocks);
  DFS_REQUIRE(dense_row_start >= 0 && dense_row_start <= scored_rows,
              "%s: dense_row=%lld must not exceed scored_rows=%lld", name,
              (long long)dense_row_start, (long long)scored_rows);
  DFS_REQUIRE(n_cand >= 0 && n_cand <= dense_col && dense_col <= k_blocks,
              "%s: need 0 <= n_cand=%lld <= dense_col=%lld <= k_blocks=%lld", name,
              (long long)n_cand, (long long)dense_col, (long long)k_blocks);
  DFS_REQUIRE(dense_row_start == 0 || (k_pick >= 1 && k_pick <= n_cand),
              "%s: k_pick=%lld must be in [1, n_cand=%lld] (torch.topk: selected index k out of range)",
              name, (long long)k_pick, (long long)n_cand);
  return 0;
}


// Scratch of the allocation-free entry point: the block-sum matrix of one
// call, in a file-scope device array (one copy per GPU, held until the
// process ends). In host code `scratch` names a host-side stand-in, so its
// device address is looked up once per device and only that address is used.
constexpr int64_t kScratchBytes = int64_t(96) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxDevices] = {};

// Scratch address on the device that `stream` belongs to (the current device
// for the null stream): the kernels run on that stream, so the scratch they
// read must be that device's copy, whichever device is current. The address
// is looked up once per device (hipGetSymbolAddress with that device made
// current for the lookup, the caller's current device restored after).
int scratch_for_stream(const char* name, hipStream_t stream, float** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) {
    set_error("%s: no usable current device (%s)", name, hipGetErrorString(e));
    return 2;
  }
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = -1;
    e = hipStreamGetDevice(stream, &sd);
    if (e != hipSuccess) {
      set_error("%s: hipStreamGetDevice failed: %s", name, hipGetErrorString(e));
      return 2;
    }
    dev = static_cast<int>(sd);
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("%s: device %d out of range", name, dev);
    return 2;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
      set_error("%s: hipSetDevice(%d) failed: %s", name, dev, hipGetErrorString(e));
      return 2;
    }
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (rc != hipSuccess || !ptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev, hipGetErrorString(rc));
      return 2;
    }
    g_scratch[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch[dev];
  return 0;
}

// Tile sizes the scorer takes: 4..128 tokens, dividing the 128-token block.
bool valid_tile(int64_t t) { return t >= 4 && t <= kBlock && kBlock % t == 0; }
// Equal query and key tiles of 16 or 32 tokens run the tuned kernels (one
// pass with a workspace); every other pair runs score_topk_tiles_kernel.
bool tuned_tiles(int64_t q_tile, int64_t k_tile) { return q_tile == k_tile && (q_tile == 16 || q_tile == 32); }

int score_topk_impl(const char* name, const uint16_t* q_pool_hi, const uint16_t* q_pool_lo,
                    const uint16_t* k_pool_hi, const uint16_t* k_pool_lo, int64_t heads, int64_t head_dim,
                    int64_t q_tile_size, int64_t k_tile_size, int64_t q_blocks, int64_t k_blocks,
                    int64_t scored_rows, int64_t n_cand, int64_t k_pick, int64_t dense_col, int64_t dense_row,
                    const int32_t* row_ptr, int32_t* col_idx, float* scores_out, uint8_t* mask_out, void* workspace,
                    int64_t workspace_bytes, dfs_stream_t stream) {
  DFS_REQUIRE(q_pool_hi && q_pool_lo && k_pool_hi && k_pool_lo && row_ptr && col_idx,
              "%s: NULL operand", name);
  DFS_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim=%lld (supported: 64, 128)", name,
              (long long)head_dim);
  DFS_REQUIRE(valid_tile(q_tile_size) && valid_tile(k_tile_size),
              "%s: q_tile_size=%lld, k_tile_size=%lld (each must divide 128 and be at least 4)", name,
              (long long)q_tile_size, (long long)k_tile_size);
  if (int rc = check_policy(name, heads, q_blocks, k_blocks, scored_rows, n_cand, k_pick,
                            dense_col, dense_row))
    return rc;
  if (!tuned_tiles(q_tile_size, k_tile_size)) {
    DFS_REQUIRE(scores_out != nullptr,
                "%s: q_tile_size=%lld, k_tile_size=%lld run the generic scorer, which keeps its block sums "
                "in scores_out: pass one", name, (long long)q_tile_size, (long long)k_tile_size);
    ScoreParams p{};
    p.q_hi = reinterpret_cast<const uint4*>(q_pool_hi);
    p.q_lo = reinterpret_cast<const uint4*>(q_pool_lo);
    p.k_hi = reinterpret_cast<const uint4*>(k_pool_hi);
    p.k_lo = reinterpret_cast<const uint4*>(k_pool_lo);
    p.row_ptr = row_ptr;
    p.col_idx = col_idx;
    p.scores_out = scores_out;
    p.mask_out = mask_out;
    p.pol = Policy{static_cast<int>(q_blocks), static_cast<int>(k_blocks), static_cast<int>(scored_rows),
                   static_cast<int>(n_cand), static_cast<int>(k_pick), static_cast<int>(dense_col),
                   static_cast<int>(dense_row)};
    const int tpbq = static_cast<int>(kBlock / q_tile_size), tpbk = static_cast<int>(kBlock / k_tile_size);
    p.q_tiles = static_cast<int>(scored_rows * tpbq);
    p.k_tiles = static_cast<int>(k_blocks * tpbk);
    p.scale_log2 = static_cast<float>(1.4426950408889634 / sqrt(static_cast<double>(head_dim)));
    const int G = 4 * (32 / tpbq);  // query blocks per workgroup
    const dim3 grid(static_cast<unsigned>((q_blocks + G - 1) / G), static_cast<unsigned>(heads));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (head_dim == 128)
      score_topk_tiles_kernel<128><<<grid, 256, 0, s>>>(p, tpbq, tpbk);
    else
      score_topk_tiles_kernel<64><<<grid, 256, 0, s>>>(p, tpbq, tpbk);
    return check_launch(name);
  }
  const int64_t tile_size = q_tile_size;
  const int tpb = static_cast<int>(kBlock / tile_size);
  const int G = 32 / tpb;
  const size_t smem = (static_cast<size_t>(G) * k_blocks + 512) * sizeof(float) + 4 * 256 * 4;
  DFS_REQUIRE(smem <= 160 * 1024, "%s: k_blocks=%lld needs %zu bytes of LDS (max 163840)", name,
              (long long)k_blocks, smem);
  // The wide kernel holds 4x the block-sum rows beside 2 x 2 key chunks.
  const int Gw = 4 * G;
  const size_t smem_wide = static_cast<size_t>(Gw) * k_blocks * sizeof(float) + 4 * 256 * 4;
  const size_t static_wide = 2 * 2 * 32 * static_cast<size_t>(head_dim) * 2;
  const bool wide = smem_wide + static_wide <= 160 * 1024;
  const bool global_sums = scores_out != nullptr;  // block sums kept in scores_out, not LDS
  const size_t smem_gb = 4 * 256 * 4 * 4;  // four waves' histograms, four copies per digit
  ScoreParams p{};
  p.q_hi = reinterpret_cast<const uint4*>(q_pool_hi);
  p.q_lo = reinterpret_cast<const uint4*>(q_pool_lo);
  p.k_hi = reinterpret_cast<const uint4*>(k_pool_hi);
  p.k_lo = reinterpret_cast<const uint4*>(k_pool_lo);
  p.row_ptr = row_ptr;
  p.col_idx = col_idx;
  p.scores_out = scores_out;
  p.mask_out = mask_out;
  p.pol = Policy{static_cast<int>(q_blocks), static_cast<int>(k_blocks), static_cast<int>(scored_rows),
                 static_cast<int>(n_cand), static_cast<int>(k_pick), static_cast<int>(dense_col),
                 static_cast<int>(dense_row)};
  p.q_tiles = static_cast<int>(scored_rows * tpb);
  p.k_tiles = static_cast<int>(k_blocks * tpb);
  p.scale_log2 = static_cast<float>(1.4426950408889634 / sqrt(static_cast<double>(head_dim)));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // The one-pass form keeps one block-sum row per wave in its key-chunk
  // buffers (2048 columns at head_dim 128, 1024 at 64); wider rows take the
  // two-pass form.
  const int64_t row_cap = 32 * head_dim / 2;
  if (workspace && k_blocks <= row_cap) {
    const int64_t need = dfs_block_score_topk_workspace_size(heads, tile_size, tile_size, q_blocks, k_blocks);
    DFS_REQUIRE(workspace_bytes >= need, "%s: workspace of %lld bytes, %lld needed", name,
                (long long)workspace_bytes, (long long)need);
    DFS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "%s: workspace must be 16-byte aligned",
                name);
    p.tile_sums = static_cast<float*>(workspace);
    p.tile_cols = static_cast<int>((k_blocks * tpb + 31) / 32 * (32 / tpb));
    dim3 grid(static_cast<unsigned>((q_blocks + Gw - 1) / Gw), static_cast<unsigned>(heads));
    if (head_dim == 128 && tpb == 8)
      score_topk_wide_kernel<128, 8, true, true><<<grid, 256, smem_gb, s>>>(p);
    else if (head_dim == 128)
      score_topk_wide_kernel<128, 4, true, true><<<grid, 256, smem_gb, s>>>(p);
    else if (tpb == 8)
      score_topk_wide_kernel<64, 8, true, true><<<grid, 256, smem_gb, s>>>(p);
    else
      score_topk_wide_kernel<64, 4, true, true><<<grid, 256, smem_gb, s>>>(p);
    return check_launch(name);
  }
  if (global_sums) {
    dim3 grid(static_cast<unsigned>((q_blocks + Gw - 1) / Gw), static_cast<unsigned>(heads));
    if (head_dim == 128 && tpb == 8)
      score_topk_wide_kernel<128, 8, true><<<grid, 256, smem_gb, s>>>(p);
    else if (head_dim == 128)
      score_topk_wide_kernel<128, 4, true><<<grid, 256, smem_gb, s>>>(p);
    else if (tpb == 8)
      score_topk_wide_kernel<64, 8, true><<<grid, 256, smem_gb, s>>>(p);
    else
      score_topk_wide_kernel<64, 4, true><<<grid, 256, smem_gb, s>>>(p);
    return check_launch(name);
  }
  if (wide) {
    dim3 grid(static_cast<unsigned>((q_blocks + Gw - 1) / Gw), static_cast<unsigned>(heads));
    if (head_dim == 128 && tpb == 8)
      score_topk_wide_kernel<128, 8, false><<<grid, 256, smem_wide, s>>>(p);
    else if (head_dim == 128)
      score_topk_wide_kernel<128, 4, false><<<grid, 256, smem_wide, s>>>(p);
    else if (tpb == 8)
      score_topk_wide_kernel<64, 8, false><<<grid, 256, smem_wide, s>>>(p);
    else
      score_topk_wide_kernel<64, 4, false><<<grid, 256, smem_wide, s>>>(p);
    return check_launch(name);
  }
  dim3 grid(static_cast<unsigned>((q_blocks + G - 1) / G), static_cast<unsigned>(heads));
  if (head_dim == 128 && tpb == 8)
    score_topk_kernel<128, 8><<<grid, 256, smem, s>>>(p);
  else if (head_dim == 128)
    score_topk_kernel<128, 4><<<grid, 256, smem, s>>>(p);
  else if (tpb == 8)
    score_topk_kernel<64, 8><<<grid, 256, smem, s>>>(p);
  else
    score_topk_kernel<64, 4><<<grid, 256, smem, s>>>(p);
  return check_launch(name);
}

}  // namespace
}  // namespace dfs

extern "C" {

int64_t dfs_block_score_topk_workspace_size(int64_t heads, int64_t q_tile_size, int64_t k_tile_size,
                                            int64_t q_blocks, int64_t k_blocks) {
  if (heads <= 0 || q_blocks <= 0 || k_blocks <= 0 || !dfs::valid_tile(q_tile_size) || !dfs::valid_tile(k_tile_size))
    return -1;
  if (!dfs::tuned_tiles(q_tile_size, k_tile_size)) return 0;  // no one-pass form for these tiles
  const int64_t tile_size = q_tile_size;
  const int64_t tpb = dfs::kBlock / tile_size, Gw = 4 * (32 / tpb);
  const int64_t rows = (q_blocks + Gw - 1) / Gw * Gw * tpb;        // tile rows of every workgroup
  const int64_t cols = (k_blocks * tpb + 31) / 32 * (32 / tpb);  // key blocks of every 32-tile chunk
  return heads * rows * cols * static_cast<int64_t>(sizeof(float));
}

int dfs_block_score_topk(const uint16_t* q_pool_hi, const uint16_t* q_pool_lo,
                         const uint16_t* k_pool_hi, const uint16_t* k_pool_lo, int64_t heads,
                         int64_t head_dim, int64_t q_tile_size, int64_t k_tile_size, int64_t q_blocks,
                         int64_t k_blocks, int64_t scored_rows, int64_t n_cand, int64_t k_pick, int64_t dense_col,
                         int64_t dense_row, const int32_t* row_ptr, int32_t* col_idx,
                         float* scores_out, uint8_t* mask_out, void* workspace, int64_t workspace_bytes,
                         dfs_stream_t stream) {
  return dfs::score_topk_impl("dfs_block_score_topk", q_pool_hi, q_pool_lo, k_pool_hi, k_pool_lo, heads, head_dim,
                              q_tile_size, k_tile_size, q_blocks, k_blocks, scored_rows, n_cand, k_pick, dense_col,
                              dense_row, row_ptr, col_idx, scores_out, mask_out, workspace, workspace_bytes, stream);
}

int dfs_block_score_topk_noalloc(const uint16_t* q_pool_hi, const uint16_t* q_pool_lo,
                                 const uint16_t* k_pool_hi, const uint16_t* k_pool_lo, int64_t heads,
                                 int64_t head_dim, int64_t q_tile_size, int64_t k_tile_size, int64_t q_blocks,
                                 int64_t k_blocks, int64_t scored_rows, int64_t n_cand, int64_t k_pick,
                                 int64_t dense_col, int64_t dense_row, const int32_t* row_ptr, int32_t* col_idx,
                                 uint8_t* mask_out, dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "dfs_block_score_topk_noalloc";
  DFS_REQUIRE(heads > 0 && scored_rows > 0 && k_blocks > 0, "%s: empty problem", name);
  const int64_t need = heads * scored_rows * k_blocks * static_cast<int64_t>(sizeof(float));
  DFS_REQUIRE(need <= kScratchBytes,
              "%s: the block sums of %lld heads x %lld rows x %lld key blocks need %lld bytes; the "
              "library's scratch holds %lld (use dfs_block_score_topk with caller buffers)",
              name, (long long)heads, (long long)scored_rows, (long long)k_blocks, (long long)need,
              (long long)kScratchBytes);
  float* sums = nullptr;
  if (int rc = scratch_for_stream(name, reinterpret_cast<hipStream_t>(stream), &sums)) return rc;
  // Two-pass form: the block sums are the only scratch (every entry is
  // written by the kernel, so nothing needs clearing between calls).
  return score_topk_impl(name, q_pool_hi, q_pool_lo, k_pool_hi, k_pool_lo, heads, head_dim, q_tile_size,
                         k_tile_size, q_blocks, k_blocks, scored_rows, n_cand, k_pick, dense_col, dense_row, row_ptr,
                         col_idx, sums, mask_out, nullptr, 0, stream);
}

int dfs_topk_from_scores(const float* scores, int64_t heads, int64_t q_blocks, int64_t k_blocks,
                         int64_t scored_rows, int64_t n_cand, int64_t k_pick, int64_t dense_col,
                         int64_t dense_row, const int32_t* row_ptr, int32_t* col_idx,
                         uint8_t* mask_out, dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "dfs_topk_from_scores";
  DFS_REQUIRE(scores && row_ptr && col_idx, "%s: NULL operand", name);
  if (int rc = check_policy(name, heads, q_blocks, k_blocks, scored_rows, n_cand, k_pick,
                            dense_col, dense_row))
    return rc;
  TopkParams p{};
  p.scores = scores;
  p.row_ptr = row_ptr;
  p.col_idx = col_idx;
  p.mask_out = mask_out;
  p.pol = Policy{static_cast<int>(q_blocks), static_cast<int>(k_blocks), static_cast<int>(scored_rows),
                 static_cast<int>(n_cand), static_cast<int>(k_pick), static_cast<int>(dense_col),
                 static_cast<int>(dense_row)};
  p.heads = static_cast<int>(heads);
  const int64_t rows = heads * q_blocks;
  topk_rows_kernel<<<static_cast<unsigned>((rows + 3) / 4), 256, 0,
                     reinterpret_cast<hipStream_t>(stream)>>>(p);
  return check_launch(name);
}

}  // extern "C"

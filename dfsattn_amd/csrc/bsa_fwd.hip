// Block-sparse flash-attention forward for gfx950 (replaces the external
// block_sparse_attn_func called at dfsattn/attention_wan.py:379-386 and
// dfsattn/attention_hyvideo.py:1075-1082).
//
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (lane column =
// query, registers = keys), so the online-softmax row statistics need one
// exchange between the two lane halves only. P is rounded to f16 (or bf16)
// and multiplied with V^T as O^T += V^T P^T; the register order of the S^T
// accumulator is reused as the token order of the PV operand, which the V^T
// layout matches. K (row-major) and V^T (transposed by the permute kernel)
// tiles are copied straight from global memory into LDS with 16-byte buffer
// loads.
//
// Two schedules:
//  * split (default): one workgroup = one (head, 128-row query block), four
//    waves of 32 query rows walking the row's kept key blocks; two
//    workgroups per CU, single K and V buffers, the K copy of the next block
//    overlapping softmax and PV, the V copy overlapping the next QK^T; the
//    other workgroup on the CU fills the gaps. With f16 operands the row's
//    reference maximum comes from its first block and later blocks skip the
//    maximum (a block is redone only if its P overflows f16); the LDS operand
//    reads run four MFMAs ahead, and the QK phase runs at raised wave
//    priority. A row visits its key blocks in order of distance from its own
//    block, so neighbouring query blocks fetch shared key blocks together.
//  * ping-pong (DFSATTN_AMD_BSA_KERNEL=pp, f16 operands): one eight-wave
//    workgroup per CU for two adjacent query blocks, the two four-wave groups
//    alternating MFMA and softmax phases half a cycle apart (described at the
//    kernel). It overlaps VALU with MFMA work but concentrates the LDS operand
//    reads of a CU into its MFMA phases; at the 75.6k-token shape it runs
//    10-15% slower than split.
//
// LDS rows are 256 bytes; 16-byte chunk c of row r is stored at chunk
// c ^ (r % 16) so the 32 rows read by one MFMA operand fetch hit distinct
// banks.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "lds_copy.h"


namespace dfs {
namespace {

struct BsaParams {
  // L: valid length (query rows computed, keys attended); R: operand rows per
  // head; Lo: out / lse rows per head; Qb = Kb = ceil(L / 128); csr_qb: CSR
  // rows per head (the mask may have been selected over a longer sequence).
  int H, L, R, Qb, Kb, Lo, csr_qb;
  int sched;   // workgroup order: 0 head-major across XCDs, 1 XCD-contiguous
  int rotate;  // rotated key-block sweep (split schedule)
  int pair_order;  // bitmap-built column order (split schedule, default): by distance from the diagonal
  int partner;     // ... with the columns shared with the partner row (qb ^ 1) first
  float scale_log2;
  int out_kind;  // 0 bf16, 1 f16, 2 f32
};

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <bool F16>
struct MfmaOp;
template <>
struct MfmaOp<false> {
  typedef bf16x8 vec;
  typedef bf16x2 pair;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // One v_cvt_pk (round to nearest even) per pair.
  static __device__ __forceinline__ pair pack(float x, float y) {
    return __builtin_convertvector((f32x2){x, y}, pair);
  }
  // acc + x.lo + x.hi in fp32 (v_dot2 with ones).
  static __device__ __forceinline__ float sum2(pair x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(x, (pair){(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  }
};
template <>
struct MfmaOp<true> {
  typedef f16x8 vec;
  typedef f16x2 pair;
  static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ pair pack(float x, float y) {
    return __builtin_convertvector((f32x2){x, y}, pair);
  }
  static __device__ __forceinline__ float sum2(pair x, float acc) {
    return __builtin_amdgcn_fdot2(x, (pair){(_Float16)1.0f, (_Float16)1.0f}, acc, false);
  }
};

// Value of the other lane half (lane ^ 32) combined with this lane's.
__device__ __forceinline__ float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// (head, query block) of this workgroup; false for a padding slot.
// Hardware deals workgroup b to XCD b % 8 and each XCD runs its workgroups in
// increasing b. Head-major mode (default): the i-th workgroup of XCD x takes
// head h = i / S and query block ((x + h) % 8) * S + i % S (S = ceil(Qb / 8)),
// so all eight XCDs sweep the same head together: one head's K/V (38.7 MB at
// 75.6k tokens) stays resident in the shared last-level cache while each
// XCD's L2 serves neighbouring query blocks. The range an XCD takes rotates
// with the head, so rows of unequal length (HunyuanVideo's dense text rows
// at the end of every head) spread over all XCDs instead of one. Mode 1: each XCD owns a contiguous run of
// (head, query block) pairs instead.
__device__ __forceinline__ bool wg_coords(const BsaParams& p, int& h, int& qb) {
  const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
  if (p.sched == 0) {
    const int S = (p.Qb + 7) >> 3;
    h = i / S;
    qb = ((xcd + h) & 7) * S + (i - h * S);
    return qb < p.Qb;
  }
  const int nwg = gridDim.x, per = nwg >> 3, rem = nwg & 7;
  const int id = xcd * per + min(xcd, rem) + i;
  h = id / p.Qb;
  qb = id - h * p.Qb;
  return true;
}

template <int D, typename QkOp>
__device__ __forceinline__ void load_q(const uint16_t* __restrict__ q, const BsaParams& p, int h, int qrow,
                                       int hl, typename QkOp::vec* qf) {
  const uint4* src = reinterpret_cast<const uint4*>(q + (static_cast<int64_t>(h) * p.R + qrow) * D);
#pragma unroll
  for (int s = 0; s < D / 16; ++s) qf[s] = __builtin_bit_cast(typename QkOp::vec, src[2 * s + hl]);
}

// S^T (128 keys x this wave's 32 queries) = K Q^T from an LDS K tile; the
// operands of the next 32-key chunk are fetched while this chunk's MFMAs run.
template <int D, typename QkOp>
__device__ __forceinline__ void qk_tile(const uint16_t* k_tile, const typename QkOp::vec* qf, int l32, int hl,
                                        f32x16* s, const f32x16& init = f32x16{}) {
  constexpr int CPR = D / 8, DS = D / 16;
  uint4 a[2][DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) a[0][ds] = lds_chunk<CPR>(k_tile, l32, ds * 2 + hl);
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    if (kc + 1 < 4) {
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) a[(kc + 1) & 1][ds] = lds_chunk<CPR>(k_tile, (kc + 1) * 32 + l32, ds * 2 + hl);
    }
    s[kc] = init;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      s[kc] = QkOp::run(__builtin_bit_cast(typename QkOp::vec, a[kc & 1][ds]), qf[ds], s[kc]);
  }
}

// Keys >= valid of the block get -inf (only the last block can be partial).
__device__ __forceinline__ void mask_tail(f32x16* s, int valid, int hl) {
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (kc * 32 + (r >> 2) * 8 + hl * 4 + (r & 3) >= valid) s[kc][r] = -INFINITY;
}

// Online-softmax bookkeeping of one block: returns the new running maximum
// (log2 domain) and rescales O and l by exp2(m_old - m_new). With LAZY the
// rescale is skipped when no row's maximum moved (alpha == 1 exactly).
template <int DCH, bool LAZY>
__device__ __forceinline__ float softmax_max(const f32x16* s, float scale_log2, float& m, float& lsum,
                                             f32x16* o) {
  float mx = -INFINITY;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kc][r]);
  const float mnew = fmaxf(m, xhalf_max(mx) * scale_log2);
  if (!LAZY || __any(mnew > m)) {
    const float alpha = exp2_fast(m - mnew);
    lsum *= alpha;
#pragma unroll
    for (int i = 0; i < DCH; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
  }
  m = mnew;
  return mnew;
}

// O^T += V^T P^T, 16 keys per step. P = exp2(S * scale * log2e - m) is formed
// step by step so its VALU work runs under the previous step's MFMAs; it is
// rounded to the PV operand type and the row sum accumulates the rounded
// values (numerator and denominator of O = P V / sum(P) see the same P).
template <int D, typename PvOp>
__device__ __forceinline__ void pv_tile(const uint16_t* v_tile, const f32x16* s, float scale_log2, float mnew,
                                        float& lsum, f32x16* o, int l32, int hl) {
  constexpr int DCH = D / 32;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const f32x16& src = s[ks >> 1];
    const int r0 = (ks & 1) * 8;
    typename PvOp::pair pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = PvOp::pack(exp2_fast(fmaf(src[r0 + 2 * j], scale_log2, -mnew)),
                         exp2_fast(fmaf(src[r0 + 2 * j + 1], scale_log2, -mnew)));
      lsum = PvOp::sum2(pr[j], lsum);
    }
    const typename PvOp::vec pf = __builtin_bit_cast(typename PvOp::vec, pr);
#pragma unroll
    for (int dc = 0; dc < DCH; ++dc) {
      const uint4 a = lds_chunk<16>(v_tile, dc * 32 + l32, ks * 2 + hl);
      o[dc] = PvOp::run(__builtin_bit_cast(typename PvOp::vec, a), pf, o[dc]);
    }
  }
}

// f16 Q fragments with c = scale * log2(e) folded in (q * c rounded to f16),
// so that S^T = K (Q c)^T arrives in log2 units.
template <int D>
__device__ __forceinline__ void load_q_scaled(const uint16_t* __restrict__ q, const BsaParams& p, int h, int qrow,
                                              int hl, f16x8* qf) {
  load_q<D, MfmaOp<true>>(q, p, h, qrow, hl, qf);
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[s][i] = static_cast<_Float16>(static_cast<float>(qf[s][i]) * p.scale_log2);
}

// Lazy online softmax on S' = S c - m, where the running reference m enters
// through the QK MFMA's C input (negm holds -m in every element). On a row's
// first block m becomes the block maximum; later, m moves only when some row
// of the wave sees a block maximum above m + kLazyTau, and O and l are
// rescaled then. The result is the same softmax: numerator and denominator
// share the reference. (With f16 P the split kernel calls this only for a
// row's first block and for a block whose P overflowed f16.)
constexpr float kLazyTau = 8.0f;
template <int DCH>
__device__ __forceinline__ void softmax_lazy(f32x16* s, bool first, float& m, float& lsum, f32x16* o,
                                             f32x16& negm) {
  float mx = -INFINITY;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kc][r]);
  const float bm = xhalf_max(mx);
  if (first || __any(bm > kLazyTau)) {
    float shift = first ? bm : fmaxf(bm, 0.f);
    if (!(shift > -INFINITY)) shift = 0.f;  // a row with every key masked keeps m
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kc][r] -= shift;
    if (!first) {
      const float alpha = exp2_fast(-shift);
      lsum *= alpha;
#pragma unroll
      for (int i = 0; i < DCH; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    }
    m += shift;
#pragma unroll
    for (int r = 0; r < 16; ++r) negm[r] = -m;
  }
}

// O^T += V^T P^T with P = exp2(S') (S' already in log2 units relative to m).
template <int D, typename PvOp>
__device__ __forceinline__ void pv_tile_log2(const uint16_t* v_tile, const f32x16* s, float& lsum, f32x16* o,
                                             int l32, int hl) {
  constexpr int DCH = D / 32;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const f32x16& src = s[ks >> 1];
    const int r0 = (ks & 1) * 8;
    typename PvOp::pair pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = PvOp::pack(exp2_fast(src[r0 + 2 * j]), exp2_fast(src[r0 + 2 * j + 1]));
      lsum = PvOp::sum2(pr[j], lsum);
    }
    const typename PvOp::vec pf = __builtin_bit_cast(typename PvOp::vec, pr);
#pragma unroll
    for (int dc = 0; dc < DCH; ++dc) {
      const uint4 a = lds_chunk<16>(v_tile, dc * 32 + l32, ks * 2 + hl);
      o[dc] = PvOp::run(__builtin_bit_cast(typename PvOp::vec, a), pf, o[dc]);
    }
  }
}

// Scheduling of an MFMA phase: the LDS operand reads run kAhead MFMAs ahead
// of their MFMAs, so each read's latency is covered by the MFMAs before its
// use (in the ping-pong schedule the other wave on the SIMD is doing VALU
// work and cannot fill MFMA gaps; in the split schedule the two waves of a
// SIMD come from independent workgroups and often read at the same time).
// Pinned with scheduling-group barriers:
// kAhead reads, then alternately one MFMA and one read, then the last MFMAs.
constexpr int kAhead = 4;
template <int N>
__device__ __forceinline__ void pin_read_ahead_schedule() {
  constexpr int kMfma = 0x008, kDsRead = 0x100;
  __builtin_amdgcn_sched_group_barrier(kDsRead, kAhead, 0);
#pragma unroll
  for (int i = 0; i < N - kAhead; ++i) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kMfma, kAhead, 0);
}

// O^T += V^T P^T from an LDS V^T tile and P held in registers.
template <int D>
__device__ __forceinline__ void pv_tile_regs(const uint16_t* v_tile, const f16x8* pf, f32x16* o, int l32, int hl) {
  constexpr int DCH = D / 32, N = 8 * DCH;
  uint4 a[N];
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = lds_chunk<16>(v_tile, (i % DCH) * 32 + l32, (i / DCH) * 2 + hl);
#pragma unroll
  for (int i = 0; i < N; ++i)
    o[i % DCH] = MfmaOp<true>::run(__builtin_bit_cast(f16x8, a[i]), pf[i / DCH], o[i % DCH]);
  pin_read_ahead_schedule<N>();
}

// S^T = init + K Q^T from an LDS K tile, with the read-ahead schedule above.
template <int D>
__device__ __forceinline__ void qk_tile_ahead(const uint16_t* k_tile, const f16x8* qf, int l32, int hl, f32x16* s,
                                              const f32x16& init = f32x16{}) {
  constexpr int CPR = D / 8, DS = D / 16, N = 4 * DS;
  uint4 a[N];
#pragma unroll
  for (int i = 0; i < N; ++i) a[i] = lds_chunk<CPR>(k_tile, (i / DS) * 32 + l32, (i % DS) * 2 + hl);
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) s[kc] = init;
#pragma unroll
  for (int i = 0; i < N; ++i)
    s[i / DS] = MfmaOp<true>::run(__builtin_bit_cast(f16x8, a[i]), qf[i % DS], s[i / DS]);
  pin_read_ahead_schedule<N>();
}

// P = exp2(S') of a whole block as f16 PV operands; lblk receives this lane's
// share of the block's row sum (of the rounded values).
__device__ __forceinline__ void make_p(const f32x16* s, f16x8* pf, float& lblk) {
  lblk = 0.f;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const f32x16& src = s[ks >> 1];
    const int r0 = (ks & 1) * 8;
    f16x2 pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = MfmaOp<true>::pack(exp2_fast(src[r0 + 2 * j]), exp2_fast(src[r0 + 2 * j + 1]));
      lblk = MfmaOp<true>::sum2(pr[j], lblk);
    }
    pf[ks] = __builtin_bit_cast(f16x8, pr);
  }
}

// O = O^T / l for row qrow, columns d = dc*32 + g*8 + hl*4 + (0..3); rows past
// L are dropped, rows with no kept block give 0.
template <int D>
__device__ __forceinline__ void store_out(const BsaParams& p, void* __restrict__ out,
                                          const int32_t* __restrict__ out_perm, float* __restrict__ lse,
                                          const f32x16* o, float m, float lsum, int h, int qrow, int hl) {
  constexpr int DCH = D / 32;
  const float ltot = xhalf_sum(lsum);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
  if (qrow >= p.L) return;
  const int orow = out_perm ? out_perm[qrow] : qrow;
  const int64_t obase = (static_cast<int64_t>(h) * p.Lo + orow) * D;
#pragma unroll
  for (int dc = 0; dc < DCH; ++dc)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = dc * 32 + g * 8 + hl * 4;
      const float v0 = o[dc][g * 4 + 0] * inv, v1 = o[dc][g * 4 + 1] * inv;
      const float v2 = o[dc][g * 4 + 2] * inv, v3 = o[dc][g * 4 + 3] * inv;
      if (p.out_kind == DFS_DTYPE_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + obase + d0) = make_float4(v0, v1, v2, v3);
      } else if (p.out_kind == DFS_DTYPE_BF16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + obase + d0) =
            make_uint2(f32_to_bf16_bits(v0) | (f32_to_bf16_bits(v1) << 16),
                       f32_to_bf16_bits(v2) | (f32_to_bf16_bits(v3) << 16));
      } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + obase + d0) =
            make_uint2(f32_to_f16_bits(v0) | (f32_to_f16_bits(v1) << 16),
                       f32_to_f16_bits(v2) | (f32_to_f16_bits(v3) << 16));
      }
    }
  if (lse && hl == 0)
    lse[static_cast<int64_t>(h) * p.Lo + qrow] = ltot > 0.f ? (m + log2f(ltot)) * 0.69314718055994531f : -INFINITY;
}

#define BSA_KERNEL_ARGS                                                                                \
  const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ vt,    \
      const int32_t *__restrict__ row_ptr, const int32_t *__restrict__ col_idx, void *__restrict__ out, \
      const int32_t *__restrict__ out_perm, float *__restrict__ lse, BsaParams p

// Split schedule: two workgroups per CU, single K and V buffers.
template <int D, bool QK_F16, bool PV_F16>
__global__ void __launch_bounds__(256, 2) bsa_fwd_split_kernel(BSA_KERNEL_ARGS) {
  constexpr int DCH = D / 32;
  constexpr int K_LOADS = D / 16;  // buffer loads per thread for a K tile
  constexpr int V_LOADS = D / 16;  // ... for a V^T tile (D rows x 256 bytes)
  constexpr uint32_t TILE_BYTES = 128 * D * 2;
  typedef MfmaOp<QK_F16> QkOp;
  typedef MfmaOp<PV_F16> PvOp;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[128 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[D * 128];
  extern __shared__ int32_t cols[];  // kept key blocks of this row (dynamic)

  int h, qb;
  if (!wg_coords(p, h, qb)) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int64_t row = static_cast<int64_t>(h) * p.csr_qb + qb;
  const int beg = row_ptr[row];
  const int end = beg + min(max(row_ptr[row + 1] - beg, 0), p.Kb);  // a row holds at most Kb blocks
  const int qrow = qb * 128 + w * 32 + l32;

  f32x16 o[DCH];
#pragma unroll
  for (int i = 0; i < DCH; ++i) o[i] = f32x16{};
  // f16 Q/K: S arrives in log2 units relative to m (lazy softmax); bf16 Q/K:
  // S is scaled in the exponent and m is the exact running maximum.
  float m = QK_F16 ? 0.f : -INFINITY, lsum = 0.f;

  if (beg < end) {
    const uint32_t head_bytes = static_cast<uint32_t>(p.R) * D * 2;
    const auto krs = make_rsrc(k + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const auto vrs = make_rsrc(vt + static_cast<int64_t>(h) * p.R * D, head_bytes);
    void* const k_base = k_lds;
    void* const v_base = v_lds;
    const int ws = __builtin_amdgcn_readfirstlane(w);
    const TileCopy<D * 2> kcopy(ws, lane);
    const TileCopy<256> vcopy(ws, lane);
    typename QkOp::vec qf[D / 16];
    if constexpr (QK_F16)
      load_q_scaled<D>(q, p, h, qrow, hl, qf);
    else
      load_q<D, QkOp>(q, p, h, qrow, hl, qf);
    f32x16 negm = f32x16{};  // -m in every element (f16 Q/K)
    // Column list of this row into LDS (read back with uniform ds_reads), and
    // Q fragments forced complete here so no wait for them lands in the loop.
    int n = end - beg;
    if (p.pair_order) {
      // Diagonal-distance order: the row's columns by distance |c - qb| from
      // its own block (c = qb first, then qb - 1, qb + 1, qb - 2, ...). The
      // workgroups resident on an XCD at one time run neighbouring Hilbert
      // query blocks, whose kept columns cluster around their diagonals, so
      // they fetch the same key blocks at about the same time (2% fewer L2
      // misses than ascending partner-first order, 0.4-1.2% faster). Columns
      // live in a bitmap at bit 2|c - qb| + (c > qb), compacted in bit order.
      // With partner set, the columns shared with the partner row (query
      // block qb ^ 1) come first, each group in distance order.
      const int W = (2 * p.Kb + 31) >> 5;
      auto bpos = [&](int c) { return 2 * (c >= qb ? c - qb : qb - c) + (c > qb ? 1 : 0); };
      uint32_t* bm = reinterpret_cast<uint32_t*>(cols + p.Kb);  // [own W][partner W]
      for (int i = tid; i < 2 * W; i += 256) bm[i] = 0u;
      block_barrier();
      for (int i = tid; i < n; i += 256) {
        const int c = col_idx[beg + i];
        if (static_cast<unsigned>(c) < static_cast<unsigned>(p.Kb)) {
          const int b = bpos(c);
          atomicOr(&bm[b >> 5], 1u << (b & 31));
        }
      }
      const int qp = qb ^ 1;
      if (p.partner && qp < p.Qb) {
        const int64_t prow = static_cast<int64_t>(h) * p.csr_qb + qp;
        const int pbeg = row_ptr[prow];
        const int pn = min(max(row_ptr[prow + 1] - pbeg, 0), p.Kb);
        for (int i = tid; i < pn; i += 256) {
          const int c = col_idx[pbeg + i];
          if (static_cast<unsigned>(c) < static_cast<unsigned>(p.Kb)) {
            const int b = bpos(c);
            atomicOr(&bm[W + (b >> 5)], 1u << (b & 31));
          }
        }
      }
      block_barrier();
      if (w == 0) {
        const int per = (W + 63) >> 6;
        const int w0 = lane * per;
        int cs = 0, co = 0;
        for (int j = 0; j < per && w0 + j < W; ++j) {
          cs += __popc(bm[w0 + j] & bm[W + w0 + j]);
          co += __popc(bm[w0 + j] & ~bm[W + w0 + j]);
        }
        int is = cs, io = co;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int ys = __shfl_up(is, off, 64), yo = __shfl_up(io, off, 64);
          if (lane >= off) {
            is += ys;
            io += yo;
          }
        }
        const int n_shared = __shfl(is, 63, 64);
        int ps = is - cs, po = n_shared + io - co;
        for (int j = 0; j < per && w0 + j < W; ++j) {
          const uint32_t own = bm[w0 + j], par = bm[W + w0 + j];
          uint32_t x = own & par;
          while (x) {
            const int b = (w0 + j) * 32 + __ffs(x) - 1;
            cols[ps++] = (b & 1) ? qb + (b >> 1) : qb - (b >> 1);
            x &= x - 1;
          }
          x = own & ~par;
          while (x) {
            const int b = (w0 + j) * 32 + __ffs(x) - 1;
            cols[po++] = (b & 1) ? qb + (b >> 1) : qb - (b >> 1);
            x &= x - 1;
          }
        }
        if (lane == 63) bm[0] = static_cast<uint32_t>(n_shared + io);  // this row's count
      }
      block_barrier();
      n = static_cast<int>(bm[0]);
      block_barrier();  // bm[0] read by everybody before any later LDS write
    } else {
      for (int i = tid; i < n; i += 256) cols[i] = col_idx[beg + i];
    }
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qf[s]));
    block_barrier();
    // Rotated sweep: the i-th workgroup of an XCD starts at the first kept
    // column >= i * Kb / CONC (CONC = workgroups resident per XCD) and wraps
    // around. Workgroups start 1 / CONC of a sweep apart, so at any moment the
    // resident workgroups of an XCD work on neighbouring key blocks and share
    // them in L2. The order is a fixed function of the workgroup, so results
    // are deterministic.
    int j0 = 0;
    if (p.rotate && !p.pair_order) {
      constexpr int CONC = 64;  // 32 CUs per XCD x 2 workgroups per CU
      const int start = static_cast<int>((static_cast<int64_t>(blockIdx.x >> 3) * p.Kb / CONC) % p.Kb);
      int lo = 0, hi = n;  // lower_bound(cols, start)
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (cols[mid] < start) lo = mid + 1; else hi = mid;
      }
      j0 = lo == n ? 0 : lo;
    }
    auto col_at = [&](int t) -> int {
      int j = j0 + t;
      j = j >= n ? j - n : j;
      return __builtin_amdgcn_readfirstlane(cols[j]);
    };
    int kb = col_at(0);
    kcopy.template issue<K_LOADS>(krs, kb * TILE_BYTES, k_base, ws);
    vcopy.template issue<V_LOADS>(vrs, kb * TILE_BYTES, v_base, ws);
    const bool tail_possible = (p.L & 127) != 0;

    for (int t = 0; t < n; ++t) {
      // After the last block the copies reload the current block into the
      // buffers it has just left (in range; nobody reads them again), so every
      // iteration issues the same loads and the vmcnt waits stay fixed.
      const int kb_next = t + 1 < n ? col_at(t + 1) : kb;
      wait_vmcnt<V_LOADS>();  // this wave's K copies have landed
      block_barrier();        // ... and everybody else's
      f32x16 s[4];
      if constexpr (QK_F16) {
        // Raised wave priority for the QK MFMAs: when both waves of a SIMD
        // reach their MFMA phases together, this one runs ahead and the two
        // drift into alternating MFMA and softmax phases (measured 1.6%).
        __builtin_amdgcn_s_setprio(1);
        qk_tile_ahead<D>(k_lds, qf, l32, hl, s, negm);
        __builtin_amdgcn_s_setprio(0);
      } else
        qk_tile<D, QkOp>(k_lds, qf, l32, hl, s);
      block_barrier();  // K tile fully consumed
      kcopy.template issue<K_LOADS>(krs, kb_next * TILE_BYTES, k_base, ws);
      if (tail_possible && kb == p.Kb - 1) {
        int valid = p.L - kb * 128;
        asm volatile("" : "+s"(valid));  // compares stay in this (rare) branch
        mask_tail(s, valid, hl);
      }
      if constexpr (QK_F16 && PV_F16) {
        // The row reference m is set from the first block's maximum. Later
        // blocks skip the maximum: P = exp2(S - m) is formed directly and
        // accepted unless it overflows f16 (some S - m >= 16, which turns
        // the block's row sum inf); only then is the block redone with a
        // moved reference. P <= 2^16 keeps f16's 11-bit precision.
        if (t == 0) softmax_lazy<DCH>(s, true, m, lsum, o, negm);
        f16x8 pf[8];
        float lblk;
        make_p(s, pf, lblk);
        if (t > 0 && __any(!(lblk < INFINITY))) {
          softmax_lazy<DCH>(s, false, m, lsum, o, negm);
          make_p(s, pf, lblk);
        }
        lsum += lblk;
        wait_vmcnt<K_LOADS>();  // V copies landed (the next K may be in flight)
        block_barrier();
        pv_tile_regs<D>(v_lds, pf, o, l32, hl);
      } else if constexpr (QK_F16) {
        softmax_lazy<DCH>(s, t == 0, m, lsum, o, negm);
        wait_vmcnt<K_LOADS>();
        block_barrier();
        pv_tile_log2<D, PvOp>(v_lds, s, lsum, o, l32, hl);
      } else {
        const float mnew = softmax_max<DCH, true>(s, p.scale_log2, m, lsum, o);
        wait_vmcnt<K_LOADS>();
        block_barrier();
        pv_tile<D, PvOp>(v_lds, s, p.scale_log2, mnew, lsum, o, l32, hl);
      }
      block_barrier();  // V tile fully consumed
      vcopy.template issue<V_LOADS>(vrs, kb_next * TILE_BYTES, v_base, ws);
      kb = kb_next;
    }
    wait_vmcnt_0();  // the trailing copies have landed before the workgroup's LDS is released
  }
  store_out<D>(p, out, out_perm, lse, o, m, lsum, h, qrow, hl);
}

// (head, pair of query blocks) of an eight-wave workgroup; head-major across
// XCDs with the per-head rotation of wg_coords.

template <int G>
__device__ __forceinline__ bool group_coords(const BsaParams& p, int& h, int& grp) {
  const int groups = (p.Qb + G - 1) / G;
  const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
  const int S = (groups + 7) >> 3;
  h = i / S;
  grp = ((xcd + h) & 7) * S + (i - h * S);
  return grp < groups;
}

struct BsaArgs {
  const uint16_t *q, *k, *vt;
  const int32_t *row_ptr, *col_idx;
  void* out;
  const int32_t* out_perm;
  float* lse;
};

// Softmax of one block for the ping-pong schedule, in two halves. S (log2
// units, from the prescaled Q) arrives without the running reference; the
// first half takes the block maximum, moves the reference m lazily (when a
// row's maximum exceeds m + kLazyTau, or on the row's first block) rescaling
// O and l, and forms P = exp2(S - m) for keys 0-63; the second half forms P
// for keys 64-127. P (f16, the PV operand order) stays in registers until the
// next MFMA phase. The VALU work of this phase overlaps the other group's
// MFMAs, so the subtraction costs little and saves the 16 registers a C
// input would hold.
template <int DCH>
__device__ __forceinline__ void pp_softmax_first(const f32x16* s, bool first, float& m, float& lsum, f32x16* o,
                                                 f16x8* pf) {
  typedef MfmaOp<true> Op;
  float mx = -INFINITY;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kc][r]);
  const float bm = xhalf_max(mx);
  if (first || __any(bm > m + kLazyTau)) {
    float mnew = first ? bm : fmaxf(bm, m);
    if (!(mnew > -INFINITY)) mnew = m;  // a row with every key masked keeps m
    if (!first) {
      const float alpha = exp2_fast(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int i = 0; i < DCH; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    }
    m = mnew;
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    Op::pair pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = Op::pack(exp2_fast(s[ks >> 1][(ks & 1) * 8 + 2 * j] - m),
                       exp2_fast(s[ks >> 1][(ks & 1) * 8 + 2 * j + 1] - m));
      lsum = Op::sum2(pr[j], lsum);
    }
    pf[ks] = __builtin_bit_cast(f16x8, pr);
  }
}

__device__ __forceinline__ void pp_softmax_second(const f32x16* s, float m, float& lsum, f16x8* pf) {
  typedef MfmaOp<true> Op;
#pragma unroll
  for (int ks = 4; ks < 8; ++ks) {
    Op::pair pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = Op::pack(exp2_fast(s[ks >> 1][(ks & 1) * 8 + 2 * j] - m),
                       exp2_fast(s[ks >> 1][(ks & 1) * 8 + 2 * j + 1] - m));
      lsum = Op::sum2(pr[j], lsum);
    }
    pf[ks] = __builtin_bit_cast(f16x8, pr);
  }
}


// Ping-pong schedule (f16 operands). One workgroup of eight
// waves per CU serves two adjacent query blocks of a head: waves 0-3 (group
// 0) run block 2i, waves 4-7 (group 1) block 2i+1, each group with its own K
// and V buffers and its own column list (the columns both rows keep first, in
// the same order, so the second fetch of a shared key block hits L2). Each
// group alternates an MFMA phase (PV of block k-1, then QK^T of block k) with
// a VALU phase (softmax of block k), and the groups run half a cycle apart:
// every SIMD holds one wave of each group, so one wave's exponentials issue
// while the other's MFMAs run. Every phase has two workgroup barriers (mid,
// end), the same number for all waves, which keeps the groups in step.
// Copies: V(k) is issued at the mid barrier of MFMA phase k (after PV(k-1)
// left the V buffer) and K(k+1) at the start of VALU phase k (after QK^T(k)
// left the K buffer); each lands at least one and a half phases before use.
// A group past its last block issues no copies and keeps taking part in the
// barriers until the other group is done.
template <int D>
__global__ void __launch_bounds__(512, 1) bsa_fwd_pp_kernel(BSA_KERNEL_ARGS) {
  constexpr int DCH = D / 32;
  constexpr int LOADS = D / 16;  // 16-byte loads per thread for one tile (4 waves)
  constexpr uint32_t TILE_BYTES = 128 * D * 2;
  constexpr uint16_t NONE = 0xFFFFu;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][128 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][D * 128];
  __shared__ int n_rows[2];
  extern __shared__ uint32_t dyn[];  // bitmaps [2][W], then columns [2][Kb] (uint16)

  int h, grp;
  if (!group_coords<2>(p, h, grp)) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int g = __builtin_amdgcn_readfirstlane(w >> 2), rg = __builtin_amdgcn_readfirstlane(w & 3);
  const int W = (p.Kb + 31) >> 5;
  uint32_t* bm = dyn;
  uint16_t* cols = reinterpret_cast<uint16_t*>(dyn + 2 * W);  // [2][Kb]

  for (int i = tid; i < 2 * W; i += 512) bm[i] = 0u;
  block_barrier();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int qr = grp * 2 + r;
    if (qr < p.Qb) {
      const int64_t row = static_cast<int64_t>(h) * p.csr_qb + qr;
      const int beg = row_ptr[row];
      const int cnt = min(max(row_ptr[row + 1] - beg, 0), p.Kb);  // a row holds at most Kb blocks
      for (int i = tid; i < cnt; i += 512) {
        const int c = col_idx[beg + i];
        if (static_cast<unsigned>(c) < static_cast<unsigned>(p.Kb)) atomicOr(&bm[r * W + (c >> 5)], 1u << (c & 31));
      }
    }
  }
  block_barrier();
  if (w == 0) {
    // Row r's list: the shared columns ascending, then its own ascending.
    const int per = (W + 63) >> 6;
    const int w0 = lane * per;
    int cs = 0, ca = 0, cb = 0;
    for (int j = 0; j < per && w0 + j < W; ++j) {
      const uint32_t a = bm[w0 + j], b = bm[W + w0 + j];
      cs += __popc(a & b);
      ca += __popc(a & ~b);
      cb += __popc(b & ~a);
    }
    int is = cs, ia = ca, ib = cb;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int ys = __shfl_up(is, off, 64), ya = __shfl_up(ia, off, 64), yb = __shfl_up(ib, off, 64);
      if (lane >= off) {
        is += ys;
        ia += ya;
        ib += yb;
      }
    }
    const int n_shared = __shfl(is, 63, 64);
    int ps = is - cs, pa = n_shared + ia - ca, pb = n_shared + ib - cb;
    for (int j = 0; j < per && w0 + j < W; ++j) {
      const uint32_t a = bm[w0 + j], b = bm[W + w0 + j];
      uint32_t x = a & b;
      while (x) {
        const uint16_t c = static_cast<uint16_t>((w0 + j) * 32 + __ffs(x) - 1);
        x &= x - 1;
        cols[ps] = c;
        cols[p.Kb + ps] = c;
        ++ps;
      }
      x = a & ~b;
      while (x) {
        cols[pa++] = static_cast<uint16_t>((w0 + j) * 32 + __ffs(x) - 1);
        x &= x - 1;
      }
      x = b & ~a;
      while (x) {
        cols[p.Kb + pb++] = static_cast<uint16_t>((w0 + j) * 32 + __ffs(x) - 1);
        x &= x - 1;
      }
    }
    if (lane == 63) {
      n_rows[0] = n_shared + ia;
      n_rows[1] = n_shared + ib;
    }
  }
  block_barrier();
  const int qb = grp * 2 + g;
  const int n = qb < p.Qb ? n_rows[g] : 0;
  const int n_all = max(grp * 2 < p.Qb ? n_rows[0] : 0, grp * 2 + 1 < p.Qb ? n_rows[1] : 0);
  const uint16_t* my_cols = cols + g * p.Kb;
  (void)NONE;

  f32x16 o[DCH];
#pragma unroll
  for (int i = 0; i < DCH; ++i) o[i] = f32x16{};
  float m = 0.f, lsum = 0.f;
  f16x8 qf[D / 16];
  const int qrow = qb * 128 + rg * 32 + l32;
  if (n > 0) load_q_scaled<D>(q, p, h, qrow, hl, qf);

  const uint32_t head_bytes = static_cast<uint32_t>(p.R) * D * 2;
  const auto krs = make_rsrc(k + static_cast<int64_t>(h) * p.R * D, head_bytes);
  const auto vrs = make_rsrc(vt + static_cast<int64_t>(h) * p.R * D, head_bytes);
  void* const k_base = k_lds[g];
  void* const v_base = v_lds[g];
  const TileCopy<D * 2> kcopy(rg, lane);
  const TileCopy<256> vcopy(rg, lane);
  auto col_at = [&](int t) -> int { return t < n ? __builtin_amdgcn_readfirstlane(my_cols[t]) : p.Kb; };
  const bool tail_possible = (p.L & 127) != 0;
#pragma unroll
  for (int s2 = 0; s2 < D / 16; ++s2) asm volatile("" ::"v"(qf[s2]));

  if (g == 0 && n > 0) kcopy.template issue<LOADS>(krs, col_at(0) * TILE_BYTES, k_base, rg);  // group 1: in V(-1)
  f32x16 s[4];
  f16x8 pf[8];
  // MFMA phase kk: PV(kk-1) from the P registers, then QK^T(kk) into s.
  auto mfma_phase = [&](int kk) {
    if (kk >= 1 && kk - 1 < n) {
      __builtin_amdgcn_s_setprio(1);
      pv_tile_regs<D>(v_lds[g], pf, o, l32, hl);
      __builtin_amdgcn_s_setprio(0);
    }
    wait_vmcnt_0();  // K(kk) landed
    block_barrier();
    const int kb = col_at(kk);
    if (kk < n) vcopy.template issue<LOADS>(vrs, kb * TILE_BYTES, v_base, rg);
    if (kk < n) {
      __builtin_amdgcn_s_setprio(1);
      qk_tile_ahead<D>(k_lds[g], qf, l32, hl, s);
      __builtin_amdgcn_s_setprio(0);
      if (tail_possible && kb == p.Kb - 1) {
        int valid = p.L - kb * 128;
        asm volatile("" : "+s"(valid));  // compares stay in this (rare) branch
        mask_tail(s, valid, hl);
      }
    }
    block_barrier();
  };
  // VALU phase kk: softmax of block kk into the P registers.
  auto valu_phase = [&](int kk) {
    const bool more = kk + 1 < n;
    if (more) kcopy.template issue<LOADS>(krs, col_at(kk + 1) * TILE_BYTES, k_base, rg);
    if (kk >= 0 && kk < n) pp_softmax_first<DCH>(s, kk == 0, m, lsum, o, pf);
    block_barrier();
    if (kk >= 0 && kk < n) pp_softmax_second(s, m, lsum, pf);
    // V(kk) landed; K(kk+1), issued after it, may still be in flight (loads
    // complete in issue order). Without a K copy behind it, wait for all.
    if (more) wait_vmcnt<LOADS>(); else wait_vmcnt_0();
    block_barrier();
  };
  // Group 0 runs M(i) V(i), group 1 V(i-1) M(i): the same four barriers per
  // iteration, half a cycle apart. Group 1's V(-1) only waits.
  if (g == 0) {
    for (int i = 0; i <= n_all; ++i) {
      mfma_phase(i);
      valu_phase(i);
    }
  } else {
    for (int i = 0; i <= n_all; ++i) {
      valu_phase(i - 1);
      mfma_phase(i);
    }
  }
  if (qb < p.Qb) store_out<D>(p, out, out_perm, lse, o, m, lsum, h, qrow, hl);
}

enum BsaSchedule { kSplit = 0, kPingPong = 1 };

template <int D>
void launch_pp(const BsaArgs& a, const BsaParams& p, hipStream_t s) {
  const int groups = (p.Qb + 1) / 2, S = (groups + 7) / 8;
  const int W = (p.Kb + 31) / 32;
  const size_t smem = static_cast<size_t>(2 * W) * sizeof(uint32_t) + static_cast<size_t>(2 * p.Kb) * 2;
  bsa_fwd_pp_kernel<D><<<dim3(static_cast<unsigned>(8 * S * p.H)), 512, smem, s>>>(
      a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out, a.out_perm, a.lse, p);
}

template <int D, bool QK_F16, bool PV_F16>
void launch_typed(const BsaArgs& a, const BsaParams& p, BsaSchedule sched, hipStream_t s) {
  // The ping-pong schedule needs f16 operands and keeps 4 tiles (128 KB at
  // D = 128) plus two uint16 column lists in LDS: it runs up to 4096 key
  // blocks; beyond, and for bf16 operands, the split schedule runs.
  if constexpr (QK_F16 && PV_F16)
    if (sched == kPingPong && p.Kb <= 4096) return launch_pp<D>(a, p, s);
  const int S = (p.Qb + 7) / 8;
  dim3 grid(static_cast<unsigned>(p.sched == 0 ? 8 * S * p.H : p.H * p.Qb));
  const size_t smem = static_cast<size_t>(p.Kb) * sizeof(int32_t) +
                      (p.pair_order ? static_cast<size_t>(2 * ((2 * p.Kb + 31) / 32)) * sizeof(uint32_t) : 0);
  bsa_fwd_split_kernel<D, QK_F16, PV_F16><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                                 a.out_perm, a.lse, p);
}

template <int D>
void launch_bsa(const BsaArgs& a, const BsaParams& p, bool qk_f16, bool pv_f16, BsaSchedule sched, hipStream_t s) {
  if (qk_f16)
    launch_typed<D, true, true>(a, p, sched, s);
  else if (pv_f16)
    launch_typed<D, false, true>(a, p, sched, s);
  else
    launch_typed<D, false, false>(a, p, sched, s);
}

}  // namespace
}  // namespace dfs

extern "C" int dfs_bsa_fwd(const void* q_perm, const void* k_perm, const void* v_t,
                           const int32_t* row_ptr, const int32_t* col_idx, int64_t heads,
                           int64_t seq_len, int64_t head_dim, int dtype, int pv_dtype, float scale,
                           void* out, int out_dtype, const int32_t* out_perm, float* lse,
                           int64_t valid_len, dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "dfs_bsa_fwd";
  DFS_REQUIRE(q_perm && k_perm && v_t && row_ptr && col_idx && out, "%s: NULL operand", name);
  DFS_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim=%lld (supported: 64, 128)", name,
              (long long)head_dim);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16, "%s: dtype=%d (supported: bf16, f16)",
              name, dtype);
  DFS_REQUIRE(pv_dtype == DFS_DTYPE_BF16 || pv_dtype == DFS_DTYPE_F16,
              "%s: pv_dtype=%d (supported: bf16, f16)", name, pv_dtype);
  DFS_REQUIRE(!(dtype == DFS_DTYPE_F16 && pv_dtype == DFS_DTYPE_BF16),
              "%s: f16 inputs need an f16 PV operand", name);
  DFS_REQUIRE(out_dtype >= 0 && out_dtype <= 2, "%s: out_dtype=%d", name, out_dtype);
  DFS_REQUIRE(heads > 0 && seq_len > 0, "%s: empty problem", name);
  const int64_t qb = (seq_len + kBlock - 1) / kBlock;
  DFS_REQUIRE(heads * qb < (int64_t(1) << 31) && qb * kBlock * head_dim < (int64_t(1) << 31),
              "%s: problem too large for 32-bit indexing", name);
  // LDS: 64 KB of tiles (split schedule) plus the row's column list.
  DFS_REQUIRE(qb <= 8192, "%s: %lld key blocks exceed the LDS column list", name, (long long)qb);
  DFS_REQUIRE(scale > 0.f && isfinite(scale), "%s: scale must be positive and finite", name);
  if (valid_len == 0) valid_len = seq_len;
  DFS_REQUIRE(valid_len > 0 && valid_len <= seq_len, "%s: valid_len=%lld outside [1, %lld]", name,
              (long long)valid_len, (long long)seq_len);
  const int64_t vb = (valid_len + kBlock - 1) / kBlock;
  BsaArgs a{static_cast<const uint16_t*>(q_perm), static_cast<const uint16_t*>(k_perm),
            static_cast<const uint16_t*>(v_t), row_ptr, col_idx, out, out_perm, lse};
  BsaParams p{};
  p.H = static_cast<int>(heads);
  p.L = static_cast<int>(valid_len);
  p.R = static_cast<int>(qb * kBlock);
  p.Qb = static_cast<int>(vb);
  p.Kb = static_cast<int>(vb);
  p.Lo = static_cast<int>(seq_len);
  p.csr_qb = static_cast<int>(qb);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.out_kind = out_dtype;
  const char* order = getenv("DFSATTN_AMD_BSA_SCHED");
  p.sched = (order && order[0] == '1') ? 1 : 0;
  const char* po = getenv("DFSATTN_AMD_BSA_ORDER");
  // DFSATTN_AMD_BSA_ORDER: unset (default, diagonal-distance order), "pair"
  // (partner-shared columns first, then the rest, each by distance) or
  // "rotate" (each row's own ascending list from a workgroup-dependent start).
  // A valid length below seq_len needs the bitmap orders, which drop columns >= Kb.
  p.pair_order = (po && strcmp(po, "rotate") == 0 && valid_len == seq_len) ? 0 : 1;
  p.partner = (po && strcmp(po, "pair") == 0) ? 1 : 0;
  const char* rot = getenv("DFSATTN_AMD_BSA_ROTATE");
  p.rotate = (rot && rot[0] == '0') ? 0 : 1;
  const char* kern = getenv("DFSATTN_AMD_BSA_KERNEL");
  // DFSATTN_AMD_BSA_KERNEL: "split" (default) or "pp" (ping-pong, f16
  // operands; split otherwise).
  const BsaSchedule sched = (kern && strcmp(kern, "pp") == 0) ? kPingPong : kSplit;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool qk_f16 = dtype == DFS_DTYPE_F16, pv_f16 = pv_dtype == DFS_DTYPE_F16;
  if (head_dim == 128)
    launch_bsa<128>(a, p, qk_f16, pv_f16, sched, s);
  else
    launch_bsa<64>(a, p, qk_f16, pv_f16, sched, s);
  return check_launch(name);
}

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

#include <type_traits>

#include "common.h"
#include "lds_copy.h"


namespace dfs {
namespace {

struct BsaParams {
  // L: query rows computed, Lk: keys attended (host values; segment 0 of
  // device cu_seqlens replaces them per workgroup); R: operand rows per head;
  // Lo: out / lse rows per head; Qb = ceil(L / 128) sets the grid, Kb =
  // ceil(Lk / 128); csr_qb: CSR rows per head (the mask may have been
  // selected over a longer sequence).
  int H, L, Lk, R, Qb, Kb, Lo, csr_qb;
  float scale_log2;
  int scale_all;  // 1: every head runs in the scaled instance (f16 q * c may reach 2^15)
  int out_kind;  // 0 bf16, 1 f16, 2 f32
  // Optional device arrays: cu_q / cu_k, segment offsets in execution order
  // (segment 0 = [0, cu[1])); exps [3][H], per-head power-of-two exponents
  // of the f16 operands (q_perm, k_perm, v_t hold x * 2^-e).
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* exps;
  // Optional Q source read in place of q_perm: execution row r < L is input
  // row q_rows[r] of q_src ([H][L][D], f16 when q_src_f16, else bf16), rows
  // past L are zero. Its exponent exps[0][h] is then only a range mark: the
  // values are read unscaled.
  const uint16_t* q_src;
  const int32_t* q_rows;
  int q_src_f16;
};

// Start of the D-element Q row of execution row qrow of head h: q_perm's row,
// or the input row it comes from (nullptr for a zero row past L). f16 tells
// whether the row holds f16 (else bf16) values.
template <int D>
__device__ __forceinline__ const uint16_t* q_row_ptr(const uint16_t* __restrict__ q, const BsaParams& p, int h,
                                                     int qrow, bool& f16) {
  if (p.q_src) {
    f16 = p.q_src_f16 != 0;
    if (qrow >= p.L) return nullptr;
    return p.q_src + (static_cast<int64_t>(h) * p.L + p.q_rows[qrow]) * D;
  }
  f16 = true;
  return q + (static_cast<int64_t>(h) * p.R + qrow) * D;
}

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
// increasing b. The i-th workgroup of XCD x takes head h = i / S and query
// block ((x + h) % 8) * S + i % S (S = ceil(Qb / 8)), so all eight XCDs sweep
// the same head together: one head's K/V (38.7 MB at 75.6k tokens) stays
// resident in the shared last-level cache while each XCD's L2 serves
// neighbouring query blocks. The range an XCD takes rotates with the head,
// so rows of unequal length (HunyuanVideo's dense text rows at the end of
// every head) spread over all XCDs instead of one.
__device__ __forceinline__ bool wg_coords(const BsaParams& p, int& h, int& qb) {
  const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
  const int S = (p.Qb + 7) >> 3;
  h = i / S;
  qb = ((xcd + h) & 7) * S + (i - h * S);
  return qb < p.Qb;
}

template <int D, typename QkOp>
__device__ __forceinline__ void load_q(const uint16_t* __restrict__ q, const BsaParams& p, int h, int qrow,
                                       int hl, typename QkOp::vec* qf) {
  bool f16;  // the bf16-operand path takes bf16 rows only (q_perm or a bf16 q_src)
  const uint4* src = reinterpret_cast<const uint4*>(q_row_ptr<D>(q, p, h, qrow, f16));
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
    qf[s] = __builtin_bit_cast(typename QkOp::vec, src ? src[2 * s + hl] : make_uint4(0, 0, 0, 0));
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
// so that S^T = K (Q c)^T arrives in log2 units. In the SCALED instance the
// per-head exponents of the f16 operands enter c exactly (q_perm holds
// q 2^-eq and k_perm k 2^-ek, so c' = c 2^(eq + ek)), and a row whose q * c'
// would leave the f16 range is stored as q c' 2^-r (r > 0, the smallest
// power of two that fits): its S arrives as S 2^-r and the kernel multiplies
// it by row_scale = 2^r. The common instance runs heads without exponents at
// a scale where |q c| < 2^15 always holds (f16 q_perm values, or Q source
// values of a head inside the f16 range, times c < 0.5).
template <int D, bool SCALED>
__device__ __forceinline__ void load_q_scaled(const uint16_t* __restrict__ q, const BsaParams& p, int h, int qrow,
                                              int hl, f16x8* qf, float& row_scale) {
  float c = p.scale_log2;
  // q_perm holds q 2^-eq; a Q source is read unscaled
  if (SCALED && p.exps) c = ldexpf(c, (p.q_src ? 0 : p.exps[h]) + p.exps[p.H + h]);
  bool f16;
  const uint4* src = reinterpret_cast<const uint4*>(q_row_ptr<D>(q, p, h, qrow, f16));
  float x[D / 16][8];
  float mx = 0.f;
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const uint4 raw = src ? src[2 * s + hl] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[s][i] = (f16 ? f16_bits_to_f32(u16_at(raw, i)) : bf16_bits_to_f32(u16_at(raw, i))) * c;
      if (SCALED) mx = fmaxf(mx, fabsf(x[s][i]));
    }
  }
  float inv = 1.f;
  row_scale = 1.f;
  if (SCALED) {
    mx = xhalf_max(mx);
    // 2^15 bounds |q c'| after the shift, with room below the f16 maximum.
    const int r = mx >= 32768.f ? ilogbf(mx) - 14 : 0;
    inv = ldexpf(1.f, -r);
    row_scale = ldexpf(1.f, r);
  }
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[s][i] = static_cast<_Float16>(x[s][i] * inv);
}

// Lazy online softmax on S' = S c - m, where the running reference m enters
// through the QK MFMA's C input (negm holds -m in every element, times qinv
// = 2^-r for a row whose Q fragments carry 2^-r). On a row's
// first block m becomes the block maximum; later, m moves only when some row
// of the wave sees a block maximum above m + kLazyTau, and O and l are
// rescaled then. The result is the same softmax: numerator and denominator
// share the reference. (With f16 P the split kernel calls this only for a
// row's first block and for a block whose P overflowed f16.)
constexpr float kLazyTau = 8.0f;
template <int DCH>
__device__ __forceinline__ void softmax_lazy(f32x16* s, bool first, float& m, float& lsum, f32x16* o,
                                             f32x16& negm, float qinv = 1.f) {
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
    for (int r = 0; r < 16; ++r) negm[r] = -m * qinv;  // rows stored as Q c 2^-r: the C input is -m 2^-r
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

// O = O^T / l for row qrow, columns d = dc*32 + g*8 + hl*4 + (0..3), times
// 2^ev for a V operand stored as v 2^-ev; rows past L are dropped, rows with
// no kept block give 0.
template <int D>
__device__ __forceinline__ void store_out(const BsaParams& p, int Lq, int ev, void* __restrict__ out,
                                          const int32_t* __restrict__ out_perm, float* __restrict__ lse,
                                          const f32x16* o, float m, float lsum, int h, int qrow, int hl) {
  constexpr int DCH = D / 32;
  const float ltot = xhalf_sum(lsum);
  const float inv = ltot > 0.f ? ldexpf(1.0f / ltot, ev) : 0.f;  // v_t holds v 2^-ev
  if (qrow >= Lq) return;
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

// Column list of one CSR row into LDS, ordered by distance |c - qb| from the
// row's own block (c = qb first, then qb - 1, qb + 1, qb - 2, ...). The
// workgroups resident on an XCD at one time run neighbouring Hilbert query
// blocks, whose kept columns cluster around their diagonals, so they fetch
// the same key blocks at about the same time (2% fewer L2 misses than
// ascending order with the partner row's shared columns first, 0.4-1.2%
// faster). Columns live in a bitmap at bit 2|c - qb| + (c > qb), compacted in
// bit order. Columns >= Kb (the keys' blocks) are dropped. bm: W words of
// LDS scratch, W = (2 Kb + 31) / 32. Every thread of the NT-thread workgroup
// calls this; it returns the number of columns written to cols.
template <int NT>
__device__ int distance_order_cols(int Kb, const int32_t* __restrict__ col_idx, int qb, int beg, int n,
                                   int32_t* cols, uint32_t* bm, int tid, int w, int lane) {
  const int W = (2 * Kb + 31) >> 5;
  for (int i = tid; i < W; i += NT) bm[i] = 0u;
  block_barrier();
  for (int i = tid; i < n; i += NT) {
    const int c = col_idx[beg + i];
    if (static_cast<unsigned>(c) < static_cast<unsigned>(Kb)) {
      const int b = 2 * (c >= qb ? c - qb : qb - c) + (c > qb ? 1 : 0);
      atomicOr(&bm[b >> 5], 1u << (b & 31));
    }
  }
  block_barrier();
  if (w == 0) {
    const int per = (W + 63) >> 6;
    const int w0 = lane * per;
    int cnt = 0;
    for (int j = 0; j < per && w0 + j < W; ++j) cnt += __popc(bm[w0 + j]);
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    int pos = incl - cnt;
    const int total = __shfl(incl, 63, 64);
    for (int j = 0; j < per && w0 + j < W; ++j) {
      uint32_t x = bm[w0 + j];
      while (x) {
        const int b = (w0 + j) * 32 + __ffs(x) - 1;
        cols[pos++] = (b & 1) ? qb + (b >> 1) : qb - (b >> 1);
        x &= x - 1;
      }
    }
    if (lane == 63) bm[0] = static_cast<uint32_t>(total);  // this row's count
  }
  block_barrier();
  const int count = static_cast<int>(bm[0]);
  block_barrier();  // bm[0] read by everybody before any later LDS write
  return count;
}

#define BSA_KERNEL_ARGS                                                                                \
  const uint16_t *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ vt,    \
      const int32_t *__restrict__ row_ptr, const int32_t *__restrict__ col_idx, void *__restrict__ out, \
      const int32_t *__restrict__ out_perm, float *__restrict__ lse, BsaParams p_in

// Split schedule: two workgroups per CU, single K and V buffers.
// Whether head h runs in the scaled instance: its operands carry exponents
// (Q or K beyond the f16 range), or the scale lets an f16 q * c reach 2^15.
__device__ __forceinline__ bool head_scaled(const BsaParams& p, int h) {
  return p.scale_all || (p.exps && (p.exps[h] | p.exps[p.H + h]) != 0);
}

// One (head, 128-row query block) of the split schedule.
// VARLEN: segment 0 of device cu_seqlens sets the rows and keys (a separate
// instance, so the common one keeps the host lengths as kernel arguments).
// SCALED: rows whose q * c' would leave the f16 range carry 2^-r and S is
// multiplied back by 2^r (the rare instance, for heads with exponents).
template <int D, bool QK_F16, bool PV_F16, bool VARLEN, bool SCALED>
__device__ __forceinline__ void bsa_split_block(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                const uint16_t* __restrict__ vt,
                                                const int32_t* __restrict__ row_ptr,
                                                const int32_t* __restrict__ col_idx, void* __restrict__ out,
                                                const int32_t* __restrict__ out_perm, float* __restrict__ lse,
                                                const BsaParams& p, int h, int qb, uint16_t* k_lds,
                                                uint16_t* v_lds, int32_t* cols) {
  constexpr int DCH = D / 32;
  constexpr int K_LOADS = D / 16;  // buffer loads per thread for a K tile
  constexpr int V_LOADS = D / 16;  // ... for a V^T tile (D rows x 256 bytes)
  constexpr uint32_t TILE_BYTES = 128 * D * 2;
  typedef MfmaOp<QK_F16> QkOp;
  typedef MfmaOp<PV_F16> PvOp;
  // Segment 0 of device cu_seqlens: its query rows and keys (offsets are
  // trusted, as by the reference's varlen kernel, and clamped to the call).
  const int Lq = VARLEN ? min(max(p.cu_q[1], 0), p.L) : p.L;
  const int Lk = VARLEN ? min(max(p.cu_k[1], 0), p.Lk) : p.Lk;
  const int Kb = (Lk + 127) >> 7;
  if (qb * 128 >= Lq) return;  // no row of this block is in the segment
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int64_t row = static_cast<int64_t>(h) * p.csr_qb + qb;
  const int beg = row_ptr[row];
  // A row holds at most as many blocks as the mask has columns (capped by the
  // call's own key blocks; columns past the segment's keys are dropped below).
  const int end = beg + min(max(row_ptr[row + 1] - beg, 0), p.Kb);
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
    float row_scale = 1.f;  // 2^r of a row whose Q fragments carry 2^-r (SCALED)
    if constexpr (QK_F16)
      load_q_scaled<D, SCALED>(q, p, h, qrow, hl, qf, row_scale);
    else
      load_q<D, QkOp>(q, p, h, qrow, hl, qf);
    const float qinv = 1.f / row_scale;
    f32x16 negm = f32x16{};  // -m (times 2^-r) in every element (f16 Q/K)
    // Column list of this row into LDS (read back with uniform ds_reads), and
    // Q fragments forced complete here so no wait for them lands in the loop.
    const int n = distance_order_cols<256>(Kb, col_idx, qb, beg, end - beg, cols,
                                           reinterpret_cast<uint32_t*>(cols + p.Kb), tid, w, lane);
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qf[s]));
    block_barrier();
    auto col_at = [&](int t) -> int { return __builtin_amdgcn_readfirstlane(cols[t]); };
    // n == 0: every kept column lies past this sequence's keys (a shorter
    // key segment), so cols holds nothing to copy; the row stays empty.
    // n is the same for every wave (read from LDS after a barrier).
    int kb = n > 0 ? col_at(0) : 0;
    if (n > 0) {
      kcopy.template issue<K_LOADS>(krs, kb * TILE_BYTES, k_base, ws);
      vcopy.template issue<V_LOADS>(vrs, kb * TILE_BYTES, v_base, ws);
    }

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
        if constexpr (SCALED) {  // rows whose q c' exceeds the f16 range carry 2^-r
#pragma unroll
          for (int kc = 0; kc < 4; ++kc)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kc][r] *= row_scale;
        }
      } else
        qk_tile<D, QkOp>(k_lds, qf, l32, hl, s);
      block_barrier();  // K tile fully consumed
      kcopy.template issue<K_LOADS>(krs, kb_next * TILE_BYTES, k_base, ws);
      if ((Lk & 127) != 0 && kb == (Lk >> 7)) {  // the keys' last block is partial
        int valid = Lk & 127;
        asm volatile("" : "+s"(valid));  // compares stay in this (rare) branch
        mask_tail(s, valid, hl);
      }
      if constexpr (QK_F16 && PV_F16) {
        // The row reference m is set from the first block's maximum. Later
        // blocks skip the maximum: P = exp2(S - m) is formed directly and
        // accepted unless it overflows f16 (some S - m >= 16, which turns
        // the block's row sum inf); only then is the block redone with a
        // moved reference. P <= 2^16 keeps f16's 11-bit precision.
        if (t == 0) softmax_lazy<DCH>(s, true, m, lsum, o, negm, qinv);
        f16x8 pf[8];
        float lblk;
        make_p(s, pf, lblk);
        if (t > 0 && __any(!(lblk < INFINITY))) {
          softmax_lazy<DCH>(s, false, m, lsum, o, negm, qinv);
          make_p(s, pf, lblk);
        }
        lsum += lblk;
        wait_vmcnt<K_LOADS>();  // V copies landed (the next K may be in flight)
        block_barrier();
        pv_tile_regs<D>(v_lds, pf, o, l32, hl);
      } else if constexpr (QK_F16) {
        softmax_lazy<DCH>(s, t == 0, m, lsum, o, negm, qinv);
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
  store_out<D>(p, VARLEN ? min(max(p.cu_q[1], 0), p.L) : p.L, p.exps ? p.exps[2 * p.H + h] : 0, out, out_perm,
               lse, o, m, lsum, h, qrow, hl);
}

template <int D, bool QK_F16, bool PV_F16, bool VARLEN, bool SCALED>
__global__ void __launch_bounds__(256, 2) bsa_fwd_split_kernel(BSA_KERNEL_ARGS) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[128 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[D * 128];
  extern __shared__ int32_t cols[];  // kept key blocks of this row (dynamic)
  if constexpr (!SCALED) {
    // Common instance: one workgroup per (head, query block), XCD-aware.
    int h, qb;
    if (!wg_coords(p_in, h, qb)) return;
    if (QK_F16 && head_scaled(p_in, h)) return;  // the scaled instance's head
    bsa_split_block<D, QK_F16, PV_F16, VARLEN, false>(q, k, vt, row_ptr, col_idx, out, out_perm, lse, p_in, h, qb,
                                                      k_lds, v_lds, cols);
  } else {
    // Scaled instance: a small grid (x: workgroups per head, y: head) whose
    // workgroups walk the query blocks of the heads that carry exponents and
    // exit at once for every other head.
    const int h = blockIdx.y;
    if (!head_scaled(p_in, h)) return;
    for (int qb = blockIdx.x; qb < p_in.Qb; qb += gridDim.x) {
      block_barrier();  // the previous block's LDS reads are done
      bsa_split_block<D, QK_F16, PV_F16, VARLEN, true>(q, k, vt, row_ptr, col_idx, out, out_perm, lse, p_in, h, qb,
                                                       k_lds, v_lds, cols);
    }
  }
}

struct BsaArgs {
  const uint16_t *q, *k, *vt;
  const int32_t *row_ptr, *col_idx;
  void* out;
  const int32_t* out_perm;
  float* lse;
};

struct SegParams {
  int H, L, R, csr_qb, Lo;
  int qk_f16, pv_f16, out_kind;
  float scale_log2;
  const int32_t* cu_q;  // [n_seq + 1] (device)
  const int32_t* cu_k;
  int n_seq;
  const int32_t* exps;  // optional [3][H]
  const uint16_t* q_src;  // optional Q source (as in BsaParams)
  const int32_t* q_rows;
  int q_src_f16;
};

__device__ __forceinline__ float operand_at(const uint16_t* base, int64_t i, bool f16) {
  return f16 ? f16_bits_to_f32(base[i]) : bf16_bits_to_f32(base[i]);
}

// The rows of a call after segment 0 of cu_seqlens, in fp32. A wave takes
// RG = 4 consecutive rows of one query block (they share the block's mask
// row) and walks their kept key blocks 64 keys at a time: one key per lane
// for the scores of the four rows (each K row read once), an exact running
// maximum per row and window, then P V with each lane owning D / 64 head
// dims of the four rows and reading the window's 64 V^T slots of its dims
// once. For n_seq == 2 the rows [cq1, cq2) attend keys [ck1, ck2) under the
// same block mask indexed from each segment's own start (query block
// (r - cq1) / 128 selects the CSR row, key block j covers keys ck1 + 128 j
// ..), as the reference's varlen kernel treats the second sequence of its
// batch (attention_hyvideo.py:1054-1082, the mask repeated per sequence at
// :359). Rows outside every query segment are zero (lse -inf). Windows are
// aligned to 64 keys so that a window's V^T slots are one contiguous run of
// a physical 128-key block; keys of a window outside the column's range are
// masked. Sized for short padding segments (a few hundred tokens).
template <int D>
__global__ void __launch_bounds__(256) bsa_segment_kernel(const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ k,
                                                          const uint16_t* __restrict__ vt,
                                                          const int32_t* __restrict__ row_ptr,
                                                          const int32_t* __restrict__ col_idx,
                                                          void* __restrict__ out, const int32_t* __restrict__ out_perm,
                                                          float* __restrict__ lse, SegParams p) {
  constexpr int RG = 4;        // rows per wave
  constexpr int DPL = D / 64;  // head dims per lane in P V
  constexpr int CPR = D / 8;   // 16-byte chunks of a K row
  __shared__ float qs[4][RG][D];   // the rows' q (times the scale), per wave
  __shared__ float ps[4][RG][64];  // the window's P in V^T slot order, per wave
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wave = blockIdx.x * 4 + w, n_waves = gridDim.x * 4;
  const int cq1 = min(max(p.cu_q[1], 0), p.L);
  const int cq2 = p.n_seq == 2 ? min(max(p.cu_q[2], cq1), p.L) : cq1;
  const int ck1 = p.n_seq == 2 ? min(max(p.cu_k[1], 0), p.L) : 0;
  const int ck2 = p.n_seq == 2 ? min(max(p.cu_k[2], ck1), p.L) : 0;
  const int seg_kb = (ck2 - ck1 + 127) >> 7;
  const bool qk16 = p.qk_f16 != 0, pv16 = p.pv_f16 != 0;
  float sq = p.scale_log2, sv = 1.f;
  if (p.exps) {
    sq = ldexpf(sq, (p.q_src ? 0 : p.exps[h]) + p.exps[p.H + h]);  // a Q source is read unscaled
    sv = ldexpf(1.f, p.exps[2 * p.H + h]);
  }
  auto wave_sync = [] {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  };
  auto half_to_f32 = [](uint32_t bits, bool f16) { return f16 ? f16_bits_to_f32(bits) : bf16_bits_to_f32(bits); };
  const int64_t hq = static_cast<int64_t>(h) * p.R * D;
  const uint4* krows = reinterpret_cast<const uint4*>(k + hq);
  // Element j of execution row r's query (r < L).
  auto q_at = [&](int r, int j) -> float {
    if (p.q_src)
      return operand_at(p.q_src, (static_cast<int64_t>(h) * p.L + p.q_rows[r]) * D + j, p.q_src_f16 != 0);
    return operand_at(q, hq + static_cast<int64_t>(r) * D + j, qk16);
  };

  for (int r0 = cq1 + RG * wave; r0 < p.L; r0 += RG * n_waves) {
    float o[RG][DPL], m[RG], l[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      m[i] = -INFINITY;
      l[i] = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[i][j] = 0.f;
    }
    if (r0 < cq2 && seg_kb > 0) {  // RG divides 128: the group's rows share query block (r0 - cq1) / 128
#pragma unroll
      for (int i = 0; i < RG; ++i)
        for (int j = lane; j < D; j += 64)
          qs[w][i][j] = r0 + i < cq2 ? q_at(r0 + i, j) * sq : 0.f;
      wave_sync();
      const int64_t crow = static_cast<int64_t>(h) * p.csr_qb + ((r0 - cq1) >> 7);
      const int beg = row_ptr[crow], end = row_ptr[crow + 1];
      for (int idx = beg; idx < end; ++idx) {  // columns ascend: stop at the segment's last block
        const int cb = __builtin_amdgcn_readfirstlane(col_idx[idx]);
        if (cb >= seg_kb) break;
        if (cb < 0) continue;
        const int k0 = ck1 + cb * 128, k1 = min(k0 + 128, ck2);
        for (int w0 = k0 & ~63; w0 < k1; w0 += 64) {
          const int key = w0 + lane;
          const bool valid = key >= k0 && key < k1;
          // the window's V^T slots of this lane's dims, loaded with the K row
          const int64_t vb = (static_cast<int64_t>(h) * (p.R / 128) + (w0 >> 7)) * D * 128 + (w0 & 127);
          uint4 vv[DPL][8];
#pragma unroll
          for (int j = 0; j < DPL; ++j)
#pragma unroll
            for (int c = 0; c < 8; ++c)
              vv[j][c] = reinterpret_cast<const uint4*>(vt + vb + static_cast<int64_t>(lane * DPL + j) * 128)[c];
          float s[RG];
#pragma unroll
          for (int i = 0; i < RG; ++i) s[i] = 0.f;
          if (valid) {
            const uint4* kr = krows + static_cast<int64_t>(key) * CPR;
#pragma unroll 2
            for (int c = 0; c < CPR; ++c) {
              asm volatile("" ::: "memory");  // q stays in LDS (read per chunk), not hoisted into registers
              const uint4 kv = kr[c];
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float kf = half_to_f32(u16_at(kv, e), qk16);
#pragma unroll
                for (int i = 0; i < RG; ++i) s[i] += qs[w][i][c * 8 + e] * kf;
              }
            }
          }
          // slot of window key `lane` in its 16-key group: swap23 (an involution)
          const int slot = (lane & ~15) | (lane & 3) | ((lane & 4) << 1) | ((lane & 8) >> 1);
#pragma unroll
          for (int i = 0; i < RG; ++i) {
            const float si = valid ? s[i] : -INFINITY;
            float mx = si;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            const float mnew = fmaxf(m[i], mx);  // finite: the window holds key max(w0, k0) < k1
            const float alpha = exp2_fast(m[i] - mnew);
            const float pk = valid ? exp2_fast(si - mnew) : 0.f;
            float psum = pk;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) psum += __shfl_xor(psum, off, 64);
            l[i] = l[i] * alpha + psum;
#pragma unroll
            for (int j = 0; j < DPL; ++j) o[i][j] *= alpha;
            m[i] = mnew;
            ps[w][i][slot] = pk;
          }
          wave_sync();
#pragma unroll 1
          for (int c = 0; c < 8; ++c) {
            asm volatile("" ::: "memory");  // P of 8 slots read per step, not all at once
            float pc[RG][8];
#pragma unroll
            for (int i = 0; i < RG; ++i)
#pragma unroll
              for (int e = 0; e < 8; ++e) pc[i][e] = ps[w][i][c * 8 + e];
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
              const uint4 vc = c == 0 ? vv[j][0] : c == 1 ? vv[j][1] : c == 2 ? vv[j][2] : c == 3 ? vv[j][3]
                             : c == 4 ? vv[j][4] : c == 5 ? vv[j][5] : c == 6 ? vv[j][6] : vv[j][7];
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float vf = half_to_f32(u16_at(vc, e), pv16);
#pragma unroll
                for (int i = 0; i < RG; ++i) o[i][j] += pc[i][e] * vf;
              }
            }
          }
          wave_sync();  // ps is read before the next window overwrites it
        }
      }
    }
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      const int r = r0 + i;
      if (r >= p.L) break;
      // A group may straddle the second sequence's end: its rows past cq2
      // were scored with q = 0 and belong to no sequence (zero, lse -inf).
      if (r >= cq2) l[i] = 0.f;
      const float inv = l[i] > 0.f ? sv / l[i] : 0.f;
      const int orow = out_perm ? out_perm[r] : r;
      const int64_t ob = (static_cast<int64_t>(h) * p.Lo + orow) * D + lane * DPL;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const float v = o[i][j] * inv;
        if (p.out_kind == DFS_DTYPE_F32)
          static_cast<float*>(out)[ob + j] = v;
        else if (p.out_kind == DFS_DTYPE_BF16)
          static_cast<uint16_t*>(out)[ob + j] = static_cast<uint16_t>(f32_to_bf16_bits(v));
        else
          static_cast<uint16_t*>(out)[ob + j] = static_cast<uint16_t>(f32_to_f16_bits(v));
      }
      if (lse && lane == 0)
        lse[static_cast<int64_t>(h) * p.Lo + r] = l[i] > 0.f ? (m[i] + log2f(l[i])) * 0.69314718055994531f : -INFINITY;
    }
  }
}

template <int D, bool QK_F16, bool PV_F16, bool VARLEN>
void launch_split_as(const BsaArgs& a, const BsaParams& p, hipStream_t s) {
  const size_t smem = static_cast<size_t>(p.Kb) * sizeof(int32_t) +
                      static_cast<size_t>((2 * p.Kb + 31) / 32) * sizeof(uint32_t);
  if (!p.scale_all) {
    const int S = (p.Qb + 7) / 8;
    bsa_fwd_split_kernel<D, QK_F16, PV_F16, VARLEN, false><<<dim3(static_cast<unsigned>(8 * S * p.H)), 256, smem, s>>>(
        a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out, a.out_perm, a.lse, p);
  }
  if constexpr (QK_F16) {
    // Heads with exponents (only when some bf16 input exceeds the f16 range)
    // or every head (large scales): a few workgroups per head.
    if (p.exps || p.scale_all) {
      const unsigned per_head = p.scale_all ? static_cast<unsigned>(p.Qb) : 8u;
      bsa_fwd_split_kernel<D, QK_F16, PV_F16, VARLEN, true>
          <<<dim3(per_head, static_cast<unsigned>(p.H)), 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                                     a.out_perm, a.lse, p);
    }
  }
}

template <int D, bool QK_F16, bool PV_F16>
void launch_split(const BsaArgs& a, const BsaParams& p, hipStream_t s) {
  if (p.cu_q) return launch_split_as<D, QK_F16, PV_F16, true>(a, p, s);
  launch_split_as<D, QK_F16, PV_F16, false>(a, p, s);
}

template <int D>
void launch_bsa(const BsaArgs& a, const BsaParams& p, bool qk_f16, bool pv_f16, hipStream_t s) {
  if (qk_f16)
    launch_split<D, true, true>(a, p, s);
  else if (pv_f16)
    launch_split<D, false, true>(a, p, s);
  else
    launch_split<D, false, false>(a, p, s);
}

}  // namespace
}  // namespace dfs

extern "C" int dfs_bsa_fwd(const void* q_perm, const void* k_perm, const void* v_t,
                           const int32_t* row_ptr, const int32_t* col_idx, int64_t heads,
                           int64_t seq_len, int64_t head_dim, int dtype, int pv_dtype, float scale,
                           void* out, int out_dtype, const int32_t* out_perm, float* lse,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t n_seq,
                           const int32_t* exps, const void* q_src, const int32_t* q_rows, int q_src_dtype,
                           dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "dfs_bsa_fwd";
  DFS_REQUIRE((q_perm || q_src) && k_perm && v_t && row_ptr && col_idx && out, "%s: NULL operand", name);
  DFS_REQUIRE(!q_src || q_rows, "%s: q_src needs q_rows", name);
  DFS_REQUIRE(!q_src || q_src_dtype == DFS_DTYPE_BF16 || q_src_dtype == DFS_DTYPE_F16,
              "%s: q_src_dtype=%d (supported: bf16, f16)", name, q_src_dtype);
  DFS_REQUIRE(!q_src || dtype == DFS_DTYPE_F16 || q_src_dtype == DFS_DTYPE_BF16,
              "%s: bf16 Q/K operands need a bf16 q_src", name);
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
  DFS_REQUIRE(n_seq == 1 || n_seq == 2, "%s: n_seq=%lld (supported: 1 or 2 sequences)", name, (long long)n_seq);
  DFS_REQUIRE((cu_seqlens_q == nullptr) == (cu_seqlens_k == nullptr),
              "%s: pass both cu_seqlens_q and cu_seqlens_k or neither", name);
  DFS_REQUIRE(n_seq == 1 || cu_seqlens_q, "%s: two sequences need cu_seqlens", name);
  BsaArgs a{static_cast<const uint16_t*>(q_perm), static_cast<const uint16_t*>(k_perm),
            static_cast<const uint16_t*>(v_t), row_ptr, col_idx, out, out_perm, lse};
  BsaParams p{};
  p.H = static_cast<int>(heads);
  p.L = p.Lk = static_cast<int>(seq_len);
  p.R = static_cast<int>(qb * kBlock);
  p.Qb = p.Kb = static_cast<int>(qb);
  p.Lo = static_cast<int>(seq_len);
  p.csr_qb = static_cast<int>(qb);
  p.scale_log2 = scale * 1.4426950408889634f;
  // An f16 operand is below 65504 < 2^16, so q * c stays below 2^15 unless
  // c >= 0.5 (a softmax scale >= 0.35); then every head takes the scaled
  // instance, whose rows carry their own powers of two.
  p.scale_all = (dtype == DFS_DTYPE_F16 && p.scale_log2 >= 0.5f) ? 1 : 0;
  p.out_kind = out_dtype;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.exps = exps;
  p.q_src = static_cast<const uint16_t*>(q_src);
  p.q_rows = q_rows;
  p.q_src_f16 = q_src_dtype == DFS_DTYPE_F16 ? 1 : 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool qk_f16 = dtype == DFS_DTYPE_F16, pv_f16 = pv_dtype == DFS_DTYPE_F16;
  if (head_dim == 128)
    launch_bsa<128>(a, p, qk_f16, pv_f16, s);
  else
    launch_bsa<64>(a, p, qk_f16, pv_f16, s);
  if (cu_seqlens_q) {
    SegParams sp{};
    sp.H = p.H;
    sp.L = p.L;
    sp.R = p.R;
    sp.csr_qb = p.csr_qb;
    sp.Lo = p.Lo;
    sp.qk_f16 = qk_f16;
    sp.pv_f16 = pv_f16;
    sp.out_kind = out_dtype;
    sp.scale_log2 = p.scale_log2;
    sp.cu_q = cu_seqlens_q;
    sp.cu_k = cu_seqlens_k;
    sp.n_seq = static_cast<int>(n_seq);
    sp.exps = exps;
    sp.q_src = p.q_src;
    sp.q_rows = q_rows;
    sp.q_src_f16 = p.q_src_f16;
    // Enough waves for a few hundred rows per head; each wave strides over
    // the rows after segment 0.
    const dim3 grid(16, static_cast<unsigned>(heads));
    if (head_dim == 128)
      bsa_segment_kernel<128><<<grid, 256, 0, s>>>(a.q, a.k, a.vt, row_ptr, col_idx, out, out_perm, lse, sp);
    else
      bsa_segment_kernel<64><<<grid, 256, 0, s>>>(a.q, a.k, a.vt, row_ptr, col_idx, out, out_perm, lse, sp);
  }
  return check_launch(name);
}

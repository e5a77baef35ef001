// Block-sparse flash-attention forward for gfx950 (replaces the external
// block_sparse_attn_func called at dfsattn/attention_wan.py:379-386 and
// dfsattn/attention_hyvideo.py:1075-1082).
//
// One workgroup = one (head, 128-row query block); four waves own 32 query
// rows each and walk the CSR list of kept 128-key blocks. K (row-major) and
// V^T (transposed by the permute kernel) tiles are copied straight from
// global memory into LDS with 16-byte buffer loads.
//
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (lane column =
// query, registers = keys), so the online-softmax row statistics need one
// exchange between the two lane halves only. P is rounded to f16 (or bf16)
// and multiplied with V^T as O^T += V^T P^T; the register order of the S^T
// accumulator is reused as the token order of the PV operand, which the V^T
// layout matches.
//
// Two schedules:
//  * pipelined: one workgroup per CU, 512 registers per wave, K and
//    V double-buffered in LDS (128 KB). Iteration i computes QK^T of block
//    i+1 next to the softmax of block i, then P V of block i; one barrier per
//    block, and the copies of the next blocks overlap a whole iteration.
//  * split (default): two workgroups per CU, single K and V buffers, four
//    barriers per block; the other workgroup on the CU fills the gaps.
//
// LDS rows are 256 bytes; 16-byte chunk c of row r is stored at chunk
// c ^ (r % 16) so the 32 rows read by one MFMA operand fetch hit distinct
// banks.
#include <math.h>
#include <stdlib.h>

#include "common.h"

namespace dfs {
namespace {

struct BsaParams {
  int H, L, R, Qb, Kb;
  int sched;   // workgroup order: 0 head-major across XCDs, 1 XCD-contiguous
  int rotate;  // rotated key-block sweep (split schedule)
  float scale_log2;
  int out_kind;  // 0 bf16, 1 f16, 2 f32
};

__device__ __forceinline__ void wait_vmcnt_0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef int32_t sgpr4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over `bytes` bytes starting at `base` (stride 0);
// loads past the end return zero instead of faulting.
__device__ __forceinline__ sgpr4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  sgpr4 r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(a & 0xffffffffu));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int32_t>((a >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(bytes));
  r.w = 0x00020000;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

// 16 bytes per lane from buffer offset voff + soff into LDS at m0 + 16 * lane.
// Issued as inline assembly so the compiler does not serialise every later LDS
// read behind it; the kernels wait for these loads with explicit vmcnt counts
// (the compiler's own vmcnt waits stay correct, only more conservative). The
// asm is volatile, so it keeps its place relative to the barrier asm (which
// carries the memory clobber that orders the LDS reads).
__device__ __forceinline__ void load_lds16(sgpr4 rs, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rs), "s"(soff), "{m0}"(lds));
}

// Copy of one tile into LDS with the chunk swizzle, all 256 threads taking
// part: load j of wave w fills LDS bytes [(4j + w) * 1024, +1024), i.e. 1024/ROWB
// rows. The swizzle depends on the row modulo the chunks per row, which is the
// same for every j, so one per-thread byte offset serves all loads and the j-th
// load only adds j * 4096 to the scalar offset.
template <int ROWB>
struct TileCopy {
  static constexpr int CPR = ROWB / 16;   // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;    // rows per wave instruction
  uint32_t voff;
  __device__ __forceinline__ TileCopy(int wave, int lane) {
    const int r = wave * RPI + lane / CPR;
    voff = static_cast<uint32_t>(r * ROWB + (((lane % CPR) ^ (r % CPR)) * 16));
  }
  // LOADS 16-byte loads per thread (4 * LOADS KiB in all) from byte tile_off.
  template <int LOADS>
  __device__ __forceinline__ void issue(sgpr4 rs, uint32_t tile_off, uint32_t lds_base,
                                        int wave) const {
    // Opaque per call: keeps the compiler from hoisting all LOADS LDS
    // addresses out of the loop into (spilled) scalar registers.
    asm volatile("" : "+s"(lds_base));
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
      load_lds16(rs, lds_base + (j * 4 + wave) * 1024, voff, tile_off + j * 4096);
  }
};

// LDS reads of this wave are complete and every wave reached this point.
__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int CPR>
__device__ __forceinline__ uint4 lds_chunk(const uint16_t* lds, int r, int c) {
  return *reinterpret_cast<const uint4*>(lds + (r * CPR + (c ^ (r % CPR))) * 8);
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
// increasing b. Head-major mode (default): the i-th workgroup of XCD x takes
// head i / S and query block x * S + i % S (S = ceil(Qb / 8)), so all eight
// XCDs sweep the same head together: one head's K/V (38.7 MB at 75.6k tokens)
// stays resident in the shared last-level cache while each XCD's L2 serves
// neighbouring query blocks. Mode 1: each XCD owns a contiguous run of
// (head, query block) pairs instead.
__device__ __forceinline__ bool wg_coords(const BsaParams& p, int& h, int& qb) {
  const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
  if (p.sched == 0) {
    const int S = (p.Qb + 7) >> 3;
    h = i / S;
    qb = xcd * S + (i - h * S);
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
                                        f32x16* s) {
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
    s[kc] = f32x16{};
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
  const int64_t obase = (static_cast<int64_t>(h) * p.L + orow) * D;
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
    lse[static_cast<int64_t>(h) * p.L + qrow] = ltot > 0.f ? (m + log2f(ltot)) * 0.69314718055994531f : -INFINITY;
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
  const int64_t row = static_cast<int64_t>(h) * p.Qb + qb;
  const int beg = row_ptr[row];
  const int end = beg + min(max(row_ptr[row + 1] - beg, 0), p.Kb);  // a row holds at most Kb blocks
  const int qrow = qb * 128 + w * 32 + l32;

  f32x16 o[DCH];
#pragma unroll
  for (int i = 0; i < DCH; ++i) o[i] = f32x16{};
  float m = -INFINITY, lsum = 0.f;

  if (beg < end) {
    const uint32_t head_bytes = static_cast<uint32_t>(p.R) * D * 2;
    const sgpr4 krs = make_rsrc(k + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const sgpr4 vrs = make_rsrc(vt + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const uint32_t k_base = lds_addr(k_lds), v_base = lds_addr(v_lds);
    const int ws = __builtin_amdgcn_readfirstlane(w);
    const TileCopy<D * 2> kcopy(ws, lane);
    const TileCopy<256> vcopy(ws, lane);
    typename QkOp::vec qf[D / 16];
    load_q<D, QkOp>(q, p, h, qrow, hl, qf);
    // Column list of this row into LDS (read back with uniform ds_reads), and
    // Q fragments forced complete here so no wait for them lands in the loop.
    for (int i = tid; i < end - beg; i += 256) cols[i] = col_idx[beg + i];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qf[s]));
    block_barrier();
    const int n = end - beg;
    // Rotated sweep: the i-th workgroup of an XCD starts at the first kept
    // column >= i * Kb / CONC (CONC = workgroups resident per XCD) and wraps
    // around. Workgroups start 1 / CONC of a sweep apart, so at any moment the
    // resident workgroups of an XCD work on neighbouring key blocks and share
    // them in L2. The order is a fixed function of the workgroup, so results
    // are deterministic.
    int j0 = 0;
    if (p.rotate) {
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
      // Past the last block the copies target a block beyond the buffer:
      // out-of-range buffer loads return zero and fetch nothing, so every
      // iteration issues the same number of loads and the waits stay fixed.
      const int kb_next = t + 1 < n ? col_at(t + 1) : p.Kb;
      wait_vmcnt<V_LOADS>();  // this wave's K copies have landed
      block_barrier();        // ... and everybody else's
      f32x16 s[4];
      qk_tile<D, QkOp>(k_lds, qf, l32, hl, s);
      block_barrier();  // K tile fully consumed
      kcopy.template issue<K_LOADS>(krs, kb_next * TILE_BYTES, k_base, ws);
      if (tail_possible && kb == p.Kb - 1) {
        int valid = p.L - kb * 128;
        asm volatile("" : "+s"(valid));  // compares stay in this (rare) branch
        mask_tail(s, valid, hl);
      }
      const float mnew = softmax_max<DCH, true>(s, p.scale_log2, m, lsum, o);
      wait_vmcnt<K_LOADS>();  // V copies landed (the next K may be in flight)
      block_barrier();
      pv_tile<D, PvOp>(v_lds, s, p.scale_log2, mnew, lsum, o, l32, hl);
      block_barrier();  // V tile fully consumed
      vcopy.template issue<V_LOADS>(vrs, kb_next * TILE_BYTES, v_base, ws);
      kb = kb_next;
    }
    wait_vmcnt_0();  // the trailing (empty) copies have retired
  }
  store_out<D>(p, out, out_perm, lse, o, m, lsum, h, qrow, hl);
}

template <int V>
struct Parity {
  static constexpr int value = V;
};

// Pipelined schedule: one workgroup per CU (512 registers per wave), K and V
// double-buffered. Block j lives in buffer j % 2. Iteration i: wait for the
// copies issued one iteration earlier (K of block i+1, V of block i), barrier
// (everybody finished iteration i-1, so K buffer i%2 and V buffer (i+1)%2 are
// free), issue K of block i+2 and V of block i+1, then QK^T of block i+1
// beside the softmax of block i, then P V of block i. Columns are ascending,
// so only the last block can be the partial tail block; it is handled by the
// peeled final iteration.
template <int D, bool QK_F16, bool PV_F16>
__global__ void __launch_bounds__(256, 1) bsa_fwd_pipe_kernel(BSA_KERNEL_ARGS) {
  constexpr int DCH = D / 32;
  constexpr int K_LOADS = D / 16;
  constexpr int V_LOADS = D / 16;
  constexpr uint32_t TILE_BYTES = 128 * D * 2;
  constexpr int TILE = 128 * D;  // uint16 elements per tile
  typedef MfmaOp<QK_F16> QkOp;
  typedef MfmaOp<PV_F16> PvOp;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2 * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2 * TILE];
  extern __shared__ int32_t cols[];

  int h, qb;
  if (!wg_coords(p, h, qb)) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int64_t row = static_cast<int64_t>(h) * p.Qb + qb;
  const int beg = row_ptr[row];
  const int n = min(max(row_ptr[row + 1] - beg, 0), p.Kb);
  const int qrow = qb * 128 + w * 32 + l32;

  f32x16 o[DCH];
#pragma unroll
  for (int i = 0; i < DCH; ++i) o[i] = f32x16{};
  float m = -INFINITY, lsum = 0.f;

  if (n > 0) {
    const uint32_t head_bytes = static_cast<uint32_t>(p.R) * D * 2;
    const sgpr4 krs = make_rsrc(k + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const sgpr4 vrs = make_rsrc(vt + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const uint32_t k_base = lds_addr(k_lds), v_base = lds_addr(v_lds);
    const int ws = __builtin_amdgcn_readfirstlane(w);
    const TileCopy<D * 2> kcopy(ws, lane);
    const TileCopy<256> vcopy(ws, lane);
    typename QkOp::vec qf[D / 16];
    load_q<D, QkOp>(q, p, h, qrow, hl, qf);
    for (int i = tid; i < n; i += 256) cols[i] = col_idx[beg + i];
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qf[s]));
    block_barrier();
    // Column of block j, or the out-of-range sentinel Kb past the end (its
    // copies fetch nothing), so every iteration issues the same loads.
    auto col = [&](int j) -> int {
      const int c = __builtin_amdgcn_readfirstlane(cols[min(j, n - 1)]);
      return j < n ? c : p.Kb;
    };

    // Prologue: K of blocks 0 and 1, V of block 0; QK^T of block 0.
    kcopy.template issue<K_LOADS>(krs, col(0) * TILE_BYTES, k_base, ws);
    kcopy.template issue<K_LOADS>(krs, col(1) * TILE_BYTES, k_base + TILE_BYTES, ws);
    vcopy.template issue<V_LOADS>(vrs, col(0) * TILE_BYTES, v_base, ws);
    wait_vmcnt_0();
    block_barrier();
    f32x16 sa[4], sb[4];
    qk_tile<D, QkOp>(k_lds, qf, l32, hl, sa);

    // One steady-state iteration with compile-time buffer parity PAR (= i % 2).
    auto step = [&](int i, f32x16* s_cur, f32x16* s_next, auto par_tag) {
      constexpr int PAR = decltype(par_tag)::value;
      wait_vmcnt_0();  // K of block i+1, V of block i
      block_barrier();
      kcopy.template issue<K_LOADS>(krs, col(i + 2) * TILE_BYTES, k_base + PAR * TILE_BYTES, ws);
      vcopy.template issue<V_LOADS>(vrs, col(i + 1) * TILE_BYTES, v_base + (1 - PAR) * TILE_BYTES, ws);
      qk_tile<D, QkOp>(k_lds + (1 - PAR) * TILE, qf, l32, hl, s_next);
      const float mnew = softmax_max<DCH, false>(s_cur, p.scale_log2, m, lsum, o);
      pv_tile<D, PvOp>(v_lds + PAR * TILE, s_cur, p.scale_log2, mnew, lsum, o, l32, hl);
      // Interleave: LDS operand reads run ahead, every MFMA is followed by the
      // next read and a few VALU instructions (softmax of this block).
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int g = 0; g < 64; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      }
    };
    int i = 0;
    for (; i + 2 < n; i += 2) {
      step(i, sa, sb, Parity<0>{});
      step(i + 1, sb, sa, Parity<1>{});
    }
    // One or two blocks remain; the last one may be the partial tail block.
    auto last = [&](int j, f32x16* s_cur, auto par_tag) {
      constexpr int PAR = decltype(par_tag)::value;
      wait_vmcnt_0();  // V of block j
      block_barrier();
      const int kb = col(j);
      if ((p.L & 127) != 0 && kb == p.Kb - 1) mask_tail(s_cur, p.L - kb * 128, hl);
      const float mnew = softmax_max<DCH, false>(s_cur, p.scale_log2, m, lsum, o);
      pv_tile<D, PvOp>(v_lds + PAR * TILE, s_cur, p.scale_log2, mnew, lsum, o, l32, hl);
    };
    if (i + 1 < n) {
      step(i, sa, sb, Parity<0>{});
      last(i + 1, sb, Parity<1>{});
    } else {
      last(i, sa, Parity<0>{});
    }
  }
  store_out<D>(p, out, out_perm, lse, o, m, lsum, h, qrow, hl);
}

struct BsaArgs {
  const uint16_t *q, *k, *vt;
  const int32_t *row_ptr, *col_idx;
  void* out;
  const int32_t* out_perm;
  float* lse;
};

template <int D, bool QK_F16, bool PV_F16>
void launch_typed(const BsaArgs& a, const BsaParams& p, bool pipelined, hipStream_t s) {
  const int S = (p.Qb + 7) / 8;
  dim3 grid(static_cast<unsigned>(p.sched == 0 ? 8 * S * p.H : p.H * p.Qb));
  const size_t smem = static_cast<size_t>(p.Kb) * sizeof(int32_t);
  if (pipelined)
    bsa_fwd_pipe_kernel<D, QK_F16, PV_F16><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                                  a.out_perm, a.lse, p);
  else
    bsa_fwd_split_kernel<D, QK_F16, PV_F16><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                                   a.out_perm, a.lse, p);
}

template <int D>
void launch_bsa(const BsaArgs& a, const BsaParams& p, bool qk_f16, bool pv_f16, bool pipelined, hipStream_t s) {
  if (qk_f16)
    launch_typed<D, true, true>(a, p, pipelined, s);
  else if (pv_f16)
    launch_typed<D, false, true>(a, p, pipelined, s);
  else
    launch_typed<D, false, false>(a, p, pipelined, s);
}

}  // namespace
}  // namespace dfs

extern "C" int dfs_bsa_fwd(const void* q_perm, const void* k_perm, const void* v_t,
                           const int32_t* row_ptr, const int32_t* col_idx, int64_t heads,
                           int64_t seq_len, int64_t head_dim, int dtype, int pv_dtype, float scale,
                           void* out, int out_dtype, const int32_t* out_perm, float* lse,
                           dfs_stream_t stream) {
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
  // LDS: 128 KB of tiles (pipelined schedule) plus the row's column list.
  DFS_REQUIRE(qb <= 8192, "%s: %lld key blocks exceed the LDS column list", name, (long long)qb);
  DFS_REQUIRE(scale > 0.f && isfinite(scale), "%s: scale must be positive and finite", name);
  BsaArgs a{static_cast<const uint16_t*>(q_perm), static_cast<const uint16_t*>(k_perm),
            static_cast<const uint16_t*>(v_t), row_ptr, col_idx, out, out_perm, lse};
  BsaParams p{};
  p.H = static_cast<int>(heads);
  p.L = static_cast<int>(seq_len);
  p.R = static_cast<int>(qb * kBlock);
  p.Qb = static_cast<int>(qb);
  p.Kb = static_cast<int>(qb);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.out_kind = out_dtype;
  const char* sched = getenv("DFSATTN_AMD_BSA_SCHED");
  p.sched = (sched && sched[0] == '1') ? 1 : 0;
  const char* rot = getenv("DFSATTN_AMD_BSA_ROTATE");
  p.rotate = (rot && rot[0] == '0') ? 0 : 1;
  const char* kern = getenv("DFSATTN_AMD_BSA_KERNEL");
  const bool pipelined = kern && kern[0] == 'p';  // "pipe" selects the one-workgroup pipelined schedule
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool qk_f16 = dtype == DFS_DTYPE_F16, pv_f16 = pv_dtype == DFS_DTYPE_F16;
  if (head_dim == 128)
    launch_bsa<128>(a, p, qk_f16, pv_f16, pipelined, s);
  else
    launch_bsa<64>(a, p, qk_f16, pv_f16, pipelined, s);
  return check_launch(name);
}

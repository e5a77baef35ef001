// Block-sparse flash-attention forward for gfx950 (replaces the external
// block_sparse_attn_func called at dfsattn/attention_wan.py:379-386 and
// dfsattn/attention_hyvideo.py:1075-1082).
//
// One workgroup = one (head, 128-row query block); four waves own 32 query
// rows each. The workgroup walks the CSR list of kept 128-key blocks. Per
// block, K (row-major) and V^T (transposed by the permute kernel) are copied
// straight from global memory into LDS with 16-byte buffer loads, each in
// its own buffer so the copy of the next K overlaps this block's softmax and
// PV product, and the copy of the next V overlaps the next QK^T.
//
// Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (lane column =
// query, registers = keys), so row statistics of the online softmax need one
// cross-half exchange only. P is rounded to f16 (or bf16) and multiplied with
// V^T as O^T += V^T P^T; the accumulator register order of S^T is reused as
// the token order of the PV operand, which the V^T layout matches.
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
  int sched;  // workgroup order: 0 head-major across XCDs, 1 XCD-contiguous
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
// read behind it; the kernel waits for these loads with explicit vmcnt counts
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

template <int D, bool QK_F16, bool PV_F16>
__global__ void __launch_bounds__(256, 2)
    bsa_fwd_kernel(const uint16_t* __restrict__ q,        // [H][R][D]
                   const uint16_t* __restrict__ k,        // [H][R][D]
                   const uint16_t* __restrict__ vt,       // [H][R/128][D][128]
                   const int32_t* __restrict__ row_ptr,   // [H*Qb+1]
                   const int32_t* __restrict__ col_idx,   // CSR columns
                   void* __restrict__ out, const int32_t* __restrict__ out_perm,
                   float* __restrict__ lse, BsaParams p) {
  constexpr int CPR = D / 8;       // 16-byte chunks per K row
  constexpr int DS = D / 16;       // QK^T k-steps
  constexpr int DCH = D / 32;      // 32-row chunks of O^T
  constexpr int K_LOADS = CPR / 2; // global_load_lds per thread for a K tile
  constexpr int V_LOADS = D / 16;  // ... for a V^T tile (D rows x 256 bytes)
  typedef MfmaOp<QK_F16> QkOp;
  typedef MfmaOp<PV_F16> PvOp;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[128 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[D * 128];
  extern __shared__ int32_t cols[];  // kept key blocks of this row (dynamic)

  // XCD-aware order. Hardware deals workgroup b to XCD b % 8 and each XCD runs
  // its workgroups in increasing b. Head-major mode (default): the i-th
  // workgroup of XCD x takes head i / S and query block x * S + i % S
  // (S = ceil(Qb / 8)), so all eight XCDs sweep the same head together: one
  // head's K/V (38.7 MB at 75.6k tokens) stays resident in the shared last-
  // level cache while each XCD's L2 serves neighbouring query blocks, which
  // keep mostly the same key blocks. Mode 1: each XCD owns a contiguous run
  // of (head, query block) pairs instead.
  int h, qb;
  const int b = blockIdx.x, xcd = b & 7, i = b >> 3;
  if (p.sched == 0) {
    const int S = (p.Qb + 7) >> 3;
    h = i / S;
    qb = xcd * S + (i - h * S);
    if (qb >= p.Qb) return;  // padding slot of the last XCD
  } else {
    const int nwg = gridDim.x, per = nwg >> 3, rem = nwg & 7;
    const int id = xcd * per + min(xcd, rem) + i;
    h = id / p.Qb;
    qb = id - h * p.Qb;
  }

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
    // Per-head buffer resources: K rows [R][D], V^T blocks [R/128][D][128].
    const uint32_t head_bytes = static_cast<uint32_t>(p.R) * D * 2;
    const sgpr4 krs = make_rsrc(k + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const sgpr4 vrs = make_rsrc(vt + static_cast<int64_t>(h) * p.R * D, head_bytes);
    const uint32_t k_base = lds_addr(k_lds), v_base = lds_addr(v_lds);
    const int ws = __builtin_amdgcn_readfirstlane(w);
    const TileCopy<D * 2> kcopy(ws, lane);
    const TileCopy<256> vcopy(ws, lane);
    constexpr uint32_t TILE_BYTES = 128 * D * 2;
    typename QkOp::vec qf[DS];
    {
      const uint4* qsrc = reinterpret_cast<const uint4*>(q + (static_cast<int64_t>(h) * p.R + qrow) * D);
#pragma unroll
      for (int s = 0; s < DS; ++s) qf[s] = __builtin_bit_cast(typename QkOp::vec, qsrc[2 * s + hl]);
    }
    // Column list of this row into LDS (read back with uniform ds_reads), and
    // Q fragments forced complete here so no wait for them lands in the loop.
    for (int i = tid; i < end - beg; i += 256) cols[i] = col_idx[beg + i];
#pragma unroll
    for (int s = 0; s < DS; ++s) asm volatile("" ::"v"(qf[s]));
    block_barrier();
    int kb = cols[0];
    kcopy.template issue<K_LOADS>(krs, kb * TILE_BYTES, k_base, ws);
    vcopy.template issue<V_LOADS>(vrs, kb * TILE_BYTES, v_base, ws);
    const bool tail_possible = (p.L & 127) != 0;

    for (int it = beg; it < end; ++it) {
      const bool more = it + 1 < end;
      const int kb_next = more ? __builtin_amdgcn_readfirstlane(cols[it + 1 - beg]) : 0;
      wait_vmcnt<V_LOADS>();  // this wave's K copies have landed
      block_barrier();        // ... and everybody else's

      // S^T = K Q^T; the LDS operands of the next 32-key chunk are fetched
      // while the current chunk's MFMAs run.
      f32x16 s[4];
      uint4 a[2][DS];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) a[0][ds] = lds_chunk<CPR>(k_lds, l32, ds * 2 + hl);
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        if (kc + 1 < 4) {
#pragma unroll
          for (int ds = 0; ds < DS; ++ds)
            a[(kc + 1) & 1][ds] = lds_chunk<CPR>(k_lds, (kc + 1) * 32 + l32, ds * 2 + hl);
        }
        s[kc] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
          s[kc] = QkOp::run(__builtin_bit_cast(typename QkOp::vec, a[kc & 1][ds]), qf[ds], s[kc]);
      }
      block_barrier();  // K tile fully consumed
      if (more) kcopy.template issue<K_LOADS>(krs, kb_next * TILE_BYTES, k_base, ws);

      // Online softmax in the log2 domain; lane column = query row.
      if (tail_possible && kb == p.Kb - 1) {
        int valid = p.L - kb * 128;
        asm volatile("" : "+s"(valid));  // compares stay in this (rare) branch
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kc * 32 + (r >> 2) * 8 + hl * 4 + (r & 3) >= valid) s[kc][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kc][r]);
      const float mnew = fmaxf(m, xhalf_max(mx) * p.scale_log2);
      // Rescale only when some row's maximum moved (alpha == 1 otherwise).
      if (__any(mnew > m)) {
        const float alpha = exp2_fast(m - mnew);
        lsum *= alpha;
#pragma unroll
        for (int i = 0; i < DCH; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      }
      m = mnew;
      // P = exp2(S * scale * log2e - m), rounded to the PV operand type; the
      // row sum accumulates the rounded values, so numerator and
      // denominator of O = P V / sum(P) see the same P.
      typename PvOp::vec pf[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const f32x16& src = s[ks >> 1];
        const int r0 = (ks & 1) * 8;
        typename PvOp::pair pr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pr[j] = PvOp::pack(exp2_fast(fmaf(src[r0 + 2 * j], p.scale_log2, -mnew)),
                             exp2_fast(fmaf(src[r0 + 2 * j + 1], p.scale_log2, -mnew)));
          lsum = PvOp::sum2(pr[j], lsum);
        }
        pf[ks] = __builtin_bit_cast(typename PvOp::vec, pr);
      }

      if (more) wait_vmcnt<K_LOADS>(); else wait_vmcnt_0();  // V copies landed
      block_barrier();
#pragma unroll
      for (int dc = 0; dc < DCH; ++dc)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const uint4 a = lds_chunk<16>(v_lds, dc * 32 + l32, ks * 2 + hl);
          o[dc] = PvOp::run(__builtin_bit_cast(typename PvOp::vec, a), pf[ks], o[dc]);
        }
      block_barrier();  // V tile fully consumed
      if (more) vcopy.template issue<V_LOADS>(vrs, kb_next * TILE_BYTES, v_base, ws);
      kb = kb_next;
    }
  }

  // Epilogue: O = O^T / l, row qrow, columns d = dc*32 + g*8 + hl*4 + (0..3).
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
    lse[static_cast<int64_t>(h) * p.L + qrow] =
        ltot > 0.f ? (m + log2f(ltot)) * 0.69314718055994531f : -INFINITY;
}

struct BsaArgs {
  const uint16_t *q, *k, *vt;
  const int32_t *row_ptr, *col_idx;
  void* out;
  const int32_t* out_perm;
  float* lse;
};

template <int D>
void launch_bsa(const BsaArgs& a, const BsaParams& p, bool qk_f16, bool pv_f16, hipStream_t s) {
  const int S = (p.Qb + 7) / 8;
  dim3 grid(static_cast<unsigned>(p.sched == 0 ? 8 * S * p.H : p.H * p.Qb));
  const size_t smem = static_cast<size_t>(p.Kb) * sizeof(int32_t);
  if (qk_f16)
    bsa_fwd_kernel<D, true, true><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                        a.out_perm, a.lse, p);
  else if (pv_f16)
    bsa_fwd_kernel<D, false, true><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                         a.out_perm, a.lse, p);
  else
    bsa_fwd_kernel<D, false, false><<<grid, 256, smem, s>>>(a.q, a.k, a.vt, a.row_ptr, a.col_idx, a.out,
                                                          a.out_perm, a.lse, p);
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
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool qk_f16 = dtype == DFS_DTYPE_F16, pv_f16 = pv_dtype == DFS_DTYPE_F16;
  if (head_dim == 128)
    launch_bsa<128>(a, p, qk_f16, pv_f16, s);
  else
    launch_bsa<64>(a, p, qk_f16, pv_f16, s);
  return check_launch(name);
}

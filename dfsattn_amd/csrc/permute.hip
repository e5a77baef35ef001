// Token permutation kernels: bit-exact Hilbert gather / inverse scatter and
// the fused preparation of the attention and scoring operands.
//
// Every row is a contiguous head_dim-element vector (256 bytes at d128 bf16),
// moved with 16-byte accesses so one row is one fully coalesced segment.
#include "common.h"

namespace dfs {
namespace {

template <typename V>
__global__ void __launch_bounds__(256) gather_rows_kernel(
    const V* __restrict__ src, const int32_t* __restrict__ perm, V* __restrict__ dst,
    int64_t src_rows, int n_perm, int dst_rows, int vpr) {
  const int64_t h = blockIdx.y;
  const V* s = src + h * src_rows * vpr;
  V* d = dst + h * static_cast<int64_t>(dst_rows) * vpr;
  const int total = dst_rows * vpr;
  for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += gridDim.x * blockDim.x) {
    const int r = idx / vpr;
    const int c = idx - r * vpr;
    V val{};
    if (r < n_perm) {
      const int pr = perm[r];
      if (pr >= 0 && pr < src_rows) val = s[static_cast<int64_t>(pr) * vpr + c];
    }
    d[idx] = val;
  }
}

template <typename V>
__global__ void __launch_bounds__(256) scatter_rows_kernel(
    const V* __restrict__ src, const int32_t* __restrict__ perm, V* __restrict__ dst,
    int64_t src_rows, int n_perm, int64_t dst_rows, int vpr) {
  const int64_t h = blockIdx.y;
  const V* s = src + h * src_rows * vpr;
  V* d = dst + h * dst_rows * vpr;
  const int total = n_perm * vpr;
  for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += gridDim.x * blockDim.x) {
    const int r = idx / vpr;
    const int c = idx - r * vpr;
    const int pr = perm[r];
    if (pr >= 0 && pr < dst_rows) d[static_cast<int64_t>(pr) * vpr + c] = s[idx];
  }
}

template <typename V>
int launch_rows(bool scatter, const void* src, const int32_t* perm, void* dst,
                int64_t heads, int64_t src_rows, int64_t n_perm, int64_t dst_rows,
                int vpr, hipStream_t stream) {
  const int64_t work = (scatter ? n_perm : dst_rows) * vpr;
  const int64_t blocks = (work + 255) / 256;
  dim3 grid(static_cast<unsigned>(blocks < 2048 ? (blocks > 0 ? blocks : 1) : 2048),
            static_cast<unsigned>(heads));
  if (scatter)
    scatter_rows_kernel<V><<<grid, 256, 0, stream>>>(
        static_cast<const V*>(src), perm, static_cast<V*>(dst), src_rows,
        static_cast<int>(n_perm), dst_rows, vpr);
  else
    gather_rows_kernel<V><<<grid, 256, 0, stream>>>(
        static_cast<const V*>(src), perm, static_cast<V*>(dst), src_rows,
        static_cast<int>(n_perm), static_cast<int>(dst_rows), vpr);
  return check_launch(scatter ? "dfs_permute_scatter" : "dfs_permute_gather");
}

int permute_rows(bool scatter, const void* src, const int32_t* perm, void* dst,
                 int64_t heads, int64_t src_rows, int64_t n_perm, int64_t dst_rows,
                 int64_t row_bytes, hipStream_t stream) {
  const char* name = scatter ? "dfs_permute_scatter" : "dfs_permute_gather";
  DFS_REQUIRE(src && perm && dst, "%s: NULL pointer", name);
  DFS_REQUIRE(heads > 0 && heads < 65536, "%s: heads=%lld out of range", name, (long long)heads);
  DFS_REQUIRE(row_bytes > 0 && row_bytes % 2 == 0, "%s: row_bytes=%lld must be a positive even number",
              name, (long long)row_bytes);
  DFS_REQUIRE(n_perm >= 0 && src_rows >= 0 && dst_rows >= 0, "%s: negative size", name);
  DFS_REQUIRE(scatter ? n_perm <= src_rows : n_perm <= dst_rows,
              "%s: n_perm=%lld exceeds the permuted tensor's rows", name, (long long)n_perm);
  const int64_t rows = scatter ? n_perm : dst_rows;
  DFS_REQUIRE(rows * row_bytes / 2 < (int64_t(1) << 31),
              "%s: %lld rows x %lld bytes per head exceeds the 32-bit per-head index range",
              name, (long long)rows, (long long)row_bytes);
  if (rows == 0) return 0;
  if (row_bytes % 16 == 0)
    return launch_rows<uint4>(scatter, src, perm, dst, heads, src_rows, n_perm, dst_rows,
                              static_cast<int>(row_bytes / 16), stream);
  if (row_bytes % 4 == 0)
    return launch_rows<uint32_t>(scatter, src, perm, dst, heads, src_rows, n_perm, dst_rows,
                                 static_cast<int>(row_bytes / 4), stream);
  return launch_rows<uint16_t>(scatter, src, perm, dst, heads, src_rows, n_perm, dst_rows,
                               static_cast<int>(row_bytes / 2), stream);
}

struct PrepParams {
  const uint4* q;  // [H][L][D] as 16-byte chunks
  const uint4* k;
  const uint4* v;
  const int32_t* perm;
  uint4* q_perm;  // [H][R][D]
  uint4* k_perm;
  uint4* v_t;  // [H][R/128][D][128]
  uint4* q_hi;  // [H][q_tiles][D] bf16
  uint4* q_lo;
  uint4* k_hi;  // [H][k_tiles][D] bf16
  uint4* k_lo;
  int32_t* flags;  // optional [3][H] overflow flags (Q, K, V)
  int L;         // tokens
  int Lv;        // video tokens (== L for Wan)
  int R;         // execution rows per head, ceil(L/128)*128
  int vpad;      // zero rows inserted after the video in the scoring layout
  int q_tiles;   // pooled query tiles (video part of the scoring layout)
  int k_tiles;   // pooled key tiles (whole scoring layout)
  int tile_q;    // tokens per query tile
  int tile_k;    // tokens per key tile
  int in_f16;    // q/k/v are f16 (else bf16)
  int convert;   // bf16 inputs, f16 operands: q_perm, k_perm and v_t get converted values
  int pool;      // write pooled tiles
};

// bf16 -> f16 of eight packed values; *overflow is set when a finite value
// exceeds the f16 range.
__device__ __forceinline__ uint4 bf16x8_to_f16x8(const uint4& v, bool* overflow) {
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float f = bf16_bits_to_f32(u16_at(v, i));
    e[i] = f32_to_f16_bits(f);
    *overflow |= ((e[i] & 0x7fffu) == 0x7c00u) && !isinf(f);
  }
  return make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
}

// Scoring-layout position -> execution row, or -1 for an inserted zero row.
__device__ __forceinline__ int scoring_to_exec(int pos, const PrepParams& p) {
  if (pos < p.Lv) return pos;
  if (pos < p.Lv + p.vpad) return -1;
  const int x = pos - p.vpad;
  return x < p.L ? x : -1;
}

__device__ __forceinline__ void add_chunk(float acc[8], const uint4& v, bool f16) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    acc[i] += f16 ? f16_bits_to_f32(u16_at(v, i)) : bf16_bits_to_f32(u16_at(v, i));
}

// One wave per (tensor, head, scoring tile): gathers the tile's rows into the
// execution layout and writes the tile mean as a bf16 hi/lo pair. Zero rows of
// the scoring layout count toward the mean, as in the reference's zero-padded
// .view(...).mean(3). Tiles past the query tiles still gather text rows of Q.
// Q and K have their own tile sizes (q_tile_size, k_tile_size); either way
// the tiles of a tensor cover the whole scoring layout, every row gathered
// once. Block bx of nbx for (head h of H, tensor Q or K).
template <int D>
__device__ __forceinline__ void prep_qk_tiles(const PrepParams& p, int bx, int nbx, int h, int H, bool is_k) {
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int RPP = kWave / CPR;  // rows covered per pass
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint4* src = (is_k ? p.k : p.q) + static_cast<int64_t>(h) * p.L * CPR;
  // Without q_perm the attention kernel gathers its Q rows from the input
  // itself: Q is then only pooled and range-flagged here.
  const bool store = is_k || p.q_perm != nullptr;
  uint4* dst = store ? (is_k ? p.k_perm : p.q_perm) + static_cast<int64_t>(h) * p.R * CPR : nullptr;

  // Zero-fill execution rows L..R-1 (done by the last block of each tensor/head).
  if (store && bx == nbx - 1) {
    const int n = (p.R - p.L) * CPR;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
      store_stream(dst + static_cast<int64_t>(p.L) * CPR + i, make_uint4(0, 0, 0, 0));
  }

  const int tile = is_k ? p.tile_k : p.tile_q;
  const int t = bx * 4 + wave;
  if (t * tile >= p.R) return;  // past the scoring layout (R tokens) of this tensor
  const int c = lane % CPR;
  const int g = lane / CPR;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  bool overflow = false;
  // Rows in batches of four passes: the permutation reads of a batch, then
  // its row reads, are all in flight before the first store.
  constexpr int BATCH = 4;
  for (int r0 = g; r0 < tile; r0 += BATCH * RPP) {
    int xs[BATCH], ss[BATCH];
    uint4 val[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int r = r0 + b * RPP;
      xs[b] = r < tile ? scoring_to_exec(t * tile + r, p) : -1;
      ss[b] = xs[b] >= 0 ? p.perm[xs[b]] : -1;
    }
#pragma unroll
    for (int b = 0; b < BATCH; ++b)
      val[b] = ss[b] >= 0 && ss[b] < p.L ? load_stream(src + static_cast<int64_t>(ss[b]) * CPR + c)
                                         : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      if (xs[b] < 0) continue;
      const uint4 op = p.convert ? bf16x8_to_f16x8(val[b], &overflow) : val[b];
      if (store) store_stream(dst + static_cast<int64_t>(xs[b]) * CPR + c, op);
      add_chunk(acc, val[b], p.in_f16 != 0);  // tile means of the input values
    }
  }
  if (p.flags && overflow) atomicOr(&p.flags[(is_k ? 1 : 0) * H + h], 1);
  const int n_tiles = is_k ? p.k_tiles : p.q_tiles;
  if (!p.pool || t >= n_tiles) return;
#pragma unroll
  for (int off = CPR; off < kWave; off <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], off);
  if (g != 0) return;
  const float inv = 1.0f / static_cast<float>(tile);
  uint32_t hi[8], lo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float mean = acc[i] * inv;
    hi[i] = f32_to_bf16_bits(mean);
    lo[i] = f32_to_bf16_bits(mean - bf16_bits_to_f32(hi[i]));
  }
  const int64_t o = (static_cast<int64_t>(h) * n_tiles + t) * CPR + c;
  (is_k ? p.k_hi : p.q_hi)[o] = make_uint4(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                           hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16));
  (is_k ? p.k_lo : p.q_lo)[o] = make_uint4(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                           lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16));
}

// Inside every 16-token group of v_t, physical slot s holds token swap23(s):
// bits 2 and 3 exchanged. Lane half j of the PV MFMA then reads its eight
// tokens {4j..4j+3, 8+4j..8+4j+3} as one contiguous 16-byte vector, matching
// the register order of the S^T accumulator it is multiplied with.
__device__ __forceinline__ int swap23(int s) {
  return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1);
}

// One block per (128-token block, head): gathers 128 V rows (zero past L),
// transposes them to [D][128] in 8x8 register tiles, optionally converting
// bf16 to f16, and stages the block in LDS so that the stores leave as whole
// 256-byte rows. The staging runs in two halves (head dims d with d % 8 < 4,
// then the rest) so a block holds 16 KB of LDS at D = 128 and the CU keeps
// its full wave count. In LDS, 16-byte chunk kg of a staged row sits at
// position kg ^ (dg % 16) of the row (dg = d / 8), which keeps the transposed
// writes (16 lanes, 16 rows, one chunk column) free of bank conflicts.
// Token block kb of head h (of H) by the NT = 16 * D / 8 threads tid of the
// workgroup, staged through `stage` (D / 2 * 16 chunks); every thread
// reaches the two barriers, also where kb is past the end.
template <int D>
__device__ __forceinline__ void prep_v_block(const PrepParams& p, int kb, int h, int H, int tid, uint4* stage) {
  constexpr int CPR = D / 8;
  constexpr int NT = 16 * CPR;            // threads
  constexpr int CHUNKS = kBlock / 8;      // 16-byte chunks per v_t row
  constexpr int HALF = D / 2 * CHUNKS;    // staged chunks per half
  const bool active = kb < p.R / kBlock;
  const int dg = tid % CPR;   // 8 head dims: dg*8 .. dg*8+7
  const int kg = tid / CPR;   // 8 physical token slots: kg*8 .. kg*8+7
  const uint4* src = p.v + static_cast<int64_t>(h) * p.L * CPR;
  uint4 rows[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int phys = kg * 8 + i;
    const int tok = kb * kBlock + (phys & ~15) + swap23(phys & 15);
    rows[i] = make_uint4(0, 0, 0, 0);
    if (active && tok < p.L) {
      const int s = p.perm[tok];
      if (s >= 0 && s < p.L) rows[i] = load_stream(src + static_cast<int64_t>(s) * CPR + dg);
    }
  }
  bool overflow = false;
  uint4* dst = p.v_t + (static_cast<int64_t>(h) * (p.R / kBlock) + kb) * D * CHUNKS;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = half * 4 + jj;
      uint32_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t bits = u16_at(rows[i], j);
        if (p.convert) {
          const float f = bf16_bits_to_f32(bits);
          bits = f32_to_f16_bits(f);
          overflow |= ((bits & 0x7fffu) == 0x7c00u) && !isinf(f);  // finite -> inf
        }
        e[i] = bits;
      }
      stage[(dg * 4 + jj) * CHUNKS + (kg ^ (dg & 15))] =
          make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int c = tid; c < HALF; c += NT) {
        const int r = c / CHUNKS, pos = c % CHUNKS;  // staged row r = dg * 4 + jj
        const int sdg = r >> 2, d = sdg * 8 + half * 4 + (r & 3);
        store_stream(dst + d * CHUNKS + (pos ^ (sdg & 15)), stage[c]);
      }
    }
    if (half == 0) __syncthreads();  // every staged chunk is read before the second half overwrites it
  }
  if (p.flags && overflow) atomicOr(&p.flags[2 * H + h], 1);
}

// Q and K: one wave per (tensor, head, scoring tile), four tiles per
// workgroup (grid: tiles / 4, heads, 2).
template <int D>
__global__ void __launch_bounds__(256) prep_qk_kernel(PrepParams p) {
  prep_qk_tiles<D>(p, blockIdx.x, gridDim.x, blockIdx.y, gridDim.y, blockIdx.z == 1);
}

// V: one workgroup per (128-token block, head).
template <int D>
__global__ void __launch_bounds__(16 * (D / 8)) prep_v_kernel(PrepParams p) {
  __shared__ uint4 stage[D / 2 * (kBlock / 8)];
  prep_v_block<D>(p, blockIdx.x, blockIdx.y, gridDim.y, threadIdx.x, stage);
}

// bf16 -> f16 of eight packed values times sc (a power of two).
__device__ __forceinline__ uint4 bf16x8_to_f16x8_scaled(const uint4& v, float sc) {
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = f32_to_f16_bits(bf16_bits_to_f32(u16_at(v, i)) * sc);
  return make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
}

// One workgroup per (head, tensor) of a call whose bf16 inputs were rounded
// to f16 operands. When the prepare kernel flagged the head (a finite value
// beyond the f16 range), the head's operand is rewritten from the inputs as
// x * 2^-e, with e >= 1 the smallest exponent that brings the head's largest
// finite |x| below 2^15, and exps[tensor][h] = e; otherwise exps[tensor][h] =
// 0. The flag is cleared. Powers of two are exact, so the attention kernel
// folds 2^e back into its Q prescale (Q, K) and its output scale (V).
template <int D>
__global__ void __launch_bounds__(1024) prep_fixup_kernel(PrepParams p, int32_t* flags, int32_t* exps) {
  constexpr int CPR = D / 8;
  const int h = blockIdx.x, t = blockIdx.y, H = gridDim.x;
  const int slot = t * H + h;
  if (flags[slot] == 0) {
    if (threadIdx.x == 0) exps[slot] = 0;
    return;
  }
  const uint4* src = (t == 0 ? p.q : t == 1 ? p.k : p.v) + static_cast<int64_t>(h) * p.L * CPR;
  const int n = p.L * CPR;
  float mx = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const uint4 v = src[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = fabsf(bf16_bits_to_f32(u16_at(v, e)));
      if (f < INFINITY) mx = fmaxf(mx, f);  // infinities and NaN stay as they are
    }
  }
  __shared__ float red[16];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = 0.f;
  for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) mx = fmaxf(mx, red[i]);
  const int e = mx >= 32768.f ? max(1, ilogbf(mx) - 14) : 1;
  const float sc = ldexpf(1.f, -e);
  if (t == 0 && p.q_perm == nullptr) {
    // No Q operand to rewrite (the attention kernel reads Q from the input):
    // e only marks the head as beyond the f16 range.
  } else if (t < 2) {
    uint4* dst = (t == 0 ? p.q_perm : p.k_perm) + static_cast<int64_t>(h) * p.R * CPR;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int x = i / CPR, c = i - x * CPR;
      const int s = p.perm[x];
      const uint4 val = (s >= 0 && s < p.L) ? src[static_cast<int64_t>(s) * CPR + c] : make_uint4(0, 0, 0, 0);
      dst[static_cast<int64_t>(x) * CPR + c] = bf16x8_to_f16x8_scaled(val, sc);
    }
  } else {
    // v_t: per 128-token block [D][128] with swap23 slot order; one 16-byte
    // chunk = 8 slots of one head dim.
    const uint16_t* vs = reinterpret_cast<const uint16_t*>(src);
    uint4* dst = p.v_t + static_cast<int64_t>(h) * (p.R / kBlock) * D * (kBlock / 8);
    const int chunks = (p.R / kBlock) * D * (kBlock / 8);
    for (int i = threadIdx.x; i < chunks; i += blockDim.x) {
      const int blk = i / (D * 16), rem = i - blk * (D * 16), d = rem >> 4, kg = rem & 15;
      uint32_t bits[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int phys = kg * 8 + j;
        const int tok = blk * kBlock + (phys & ~15) + swap23(phys & 15);
        float f = 0.f;
        if (tok < p.L) {
          const int s = p.perm[tok];
          if (s >= 0 && s < p.L) f = bf16_bits_to_f32(vs[static_cast<int64_t>(s) * D + d]);
        }
        bits[j] = f32_to_f16_bits(f * sc);
      }
      dst[i] = make_uint4(bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16), bits[4] | (bits[5] << 16),
                          bits[6] | (bits[7] << 16));
    }
  }
  if (threadIdx.x == 0) {
    exps[slot] = e;
    flags[slot] = 0;
  }
}

}  // namespace
}  // namespace dfs

extern "C" {

int dfs_permute_gather(const void* src, const int32_t* perm, void* dst, int64_t heads,
                       int64_t src_rows, int64_t n_perm, int64_t dst_rows, int64_t row_bytes,
                       dfs_stream_t stream) {
  return dfs::permute_rows(false, src, perm, dst, heads, src_rows, n_perm, dst_rows, row_bytes,
                           reinterpret_cast<hipStream_t>(stream));
}

int dfs_permute_scatter(const void* src, const int32_t* perm, void* dst, int64_t heads,
                        int64_t src_rows, int64_t n_perm, int64_t dst_rows, int64_t row_bytes,
                        dfs_stream_t stream) {
  return dfs::permute_rows(true, src, perm, dst, heads, src_rows, n_perm, dst_rows, row_bytes,
                           reinterpret_cast<hipStream_t>(stream));
}

int dfs_prepare_qkv(const void* q, const void* k, const void* v, const int32_t* perm,
                    int64_t heads, int64_t seq_len, int64_t head_dim, int dtype,
                    int64_t video_len, int64_t q_tile_size, int64_t k_tile_size, int operand_dtype, void* q_perm,
                    void* k_perm, void* v_t, uint16_t* q_pool_hi, uint16_t* q_pool_lo,
                    uint16_t* k_pool_hi, uint16_t* k_pool_lo, int32_t* overflow,
                    dfs_stream_t stream) {
  using namespace dfs;
  DFS_REQUIRE(q && k && v && perm && k_perm && v_t, "dfs_prepare_qkv: NULL operand");
  DFS_REQUIRE(head_dim == 64 || head_dim == 128, "dfs_prepare_qkv: head_dim=%lld (supported: 64, 128)",
              (long long)head_dim);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16,
              "dfs_prepare_qkv: dtype=%d (supported: bf16, f16)", dtype);
  DFS_REQUIRE(operand_dtype == DFS_DTYPE_BF16 || operand_dtype == DFS_DTYPE_F16,
              "dfs_prepare_qkv: operand_dtype=%d (supported: bf16, f16)", operand_dtype);
  DFS_REQUIRE(!(dtype == DFS_DTYPE_F16 && operand_dtype == DFS_DTYPE_BF16),
              "dfs_prepare_qkv: f16 inputs need f16 operands");
  DFS_REQUIRE(heads > 0 && heads < 65536, "dfs_prepare_qkv: heads=%lld out of range", (long long)heads);
  DFS_REQUIRE(seq_len > 0 && video_len > 0 && video_len <= seq_len,
              "dfs_prepare_qkv: need 0 < video_len=%lld <= seq_len=%lld", (long long)video_len,
              (long long)seq_len);
  DFS_REQUIRE(q_tile_size > 0 && kBlock % q_tile_size == 0,
              "dfs_prepare_qkv: q_tile_size=%lld must divide 128", (long long)q_tile_size);
  DFS_REQUIRE(k_tile_size > 0 && kBlock % k_tile_size == 0,
              "dfs_prepare_qkv: k_tile_size=%lld must divide 128", (long long)k_tile_size);
  const int64_t kb = (seq_len + kBlock - 1) / kBlock;
  const int64_t vb = (video_len + kBlock - 1) / kBlock;
  const int64_t vpad = vb * kBlock - video_len;
  DFS_REQUIRE(video_len + vpad + (seq_len - video_len) <= kb * kBlock,
              "dfs_prepare_qkv: padded scoring layout (%lld tokens) exceeds %lld blocks; the "
              "reference's tile view fails for this video/text split",
              (long long)(video_len + vpad + (seq_len - video_len)), (long long)kb);
  DFS_REQUIRE(kb * kBlock * head_dim < (int64_t(1) << 31),
              "dfs_prepare_qkv: seq_len=%lld too long for 32-bit per-head indexing", (long long)seq_len);
  const bool pool = q_pool_hi || q_pool_lo || k_pool_hi || k_pool_lo;
  DFS_REQUIRE(!pool || (q_pool_hi && q_pool_lo && k_pool_hi && k_pool_lo),
              "dfs_prepare_qkv: pooled outputs must be all set or all NULL");

  PrepParams p{};
  p.q = static_cast<const uint4*>(q);
  p.k = static_cast<const uint4*>(k);
  p.v = static_cast<const uint4*>(v);
  p.perm = perm;
  p.q_perm = static_cast<uint4*>(q_perm);
  p.k_perm = static_cast<uint4*>(k_perm);
  p.v_t = static_cast<uint4*>(v_t);
  p.q_hi = reinterpret_cast<uint4*>(q_pool_hi);
  p.q_lo = reinterpret_cast<uint4*>(q_pool_lo);
  p.k_hi = reinterpret_cast<uint4*>(k_pool_hi);
  p.k_lo = reinterpret_cast<uint4*>(k_pool_lo);
  p.flags = overflow;
  p.L = static_cast<int>(seq_len);
  p.Lv = static_cast<int>(video_len);
  p.R = static_cast<int>(kb * kBlock);
  p.vpad = static_cast<int>(vpad);
  p.tile_q = static_cast<int>(q_tile_size);
  p.tile_k = static_cast<int>(k_tile_size);
  p.q_tiles = static_cast<int>(vb * kBlock / q_tile_size);
  p.k_tiles = static_cast<int>(kb * kBlock / k_tile_size);
  p.in_f16 = dtype == DFS_DTYPE_F16;
  p.convert = (dtype == DFS_DTYPE_BF16 && operand_dtype == DFS_DTYPE_F16);
  p.pool = pool ? 1 : 0;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Enough four-wave blocks for the smaller of the two tiles (more tiles).
  const int64_t max_tiles = kb * kBlock / (q_tile_size < k_tile_size ? q_tile_size : k_tile_size);
  dim3 gqk(static_cast<unsigned>((max_tiles + 3) / 4), static_cast<unsigned>(heads), 2);
  dim3 gv(static_cast<unsigned>(kb), static_cast<unsigned>(heads));
  if (head_dim == 128) {
    prep_qk_kernel<128><<<gqk, 256, 0, s>>>(p);
    prep_v_kernel<128><<<gv, 16 * 16, 0, s>>>(p);
  } else {
    prep_qk_kernel<64><<<gqk, 256, 0, s>>>(p);
    prep_v_kernel<64><<<gv, 16 * 8, 0, s>>>(p);
  }
  return check_launch("dfs_prepare_qkv");
}

int dfs_prepare_fixup(const void* q, const void* k, const void* v, const int32_t* perm, int64_t heads,
                      int64_t seq_len, int64_t head_dim, void* q_perm, void* k_perm, void* v_t,
                      int32_t* overflow, int32_t* exps, dfs_stream_t stream) {
  using namespace dfs;
  DFS_REQUIRE(q && k && v && perm && k_perm && v_t && overflow && exps, "dfs_prepare_fixup: NULL operand");
  DFS_REQUIRE(head_dim == 64 || head_dim == 128, "dfs_prepare_fixup: head_dim=%lld (supported: 64, 128)",
              (long long)head_dim);
  DFS_REQUIRE(heads > 0 && heads < 65536, "dfs_prepare_fixup: heads=%lld out of range", (long long)heads);
  DFS_REQUIRE(seq_len > 0, "dfs_prepare_fixup: seq_len=%lld", (long long)seq_len);
  const int64_t kb = (seq_len + kBlock - 1) / kBlock;
  DFS_REQUIRE(kb * kBlock * head_dim < (int64_t(1) << 31),
              "dfs_prepare_fixup: seq_len=%lld too long for 32-bit per-head indexing", (long long)seq_len);
  PrepParams p{};
  p.q = static_cast<const uint4*>(q);
  p.k = static_cast<const uint4*>(k);
  p.v = static_cast<const uint4*>(v);
  p.perm = perm;
  p.q_perm = static_cast<uint4*>(q_perm);
  p.k_perm = static_cast<uint4*>(k_perm);
  p.v_t = static_cast<uint4*>(v_t);
  p.L = static_cast<int>(seq_len);
  p.R = static_cast<int>(kb * kBlock);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(heads), 3);
  if (head_dim == 128)
    prep_fixup_kernel<128><<<grid, 1024, 0, s>>>(p, overflow, exps);
  else
    prep_fixup_kernel<64><<<grid, 1024, 0, s>>>(p, overflow, exps);
  return check_launch("dfs_prepare_fixup");
}

}  // extern "C"

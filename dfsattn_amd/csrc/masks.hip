// Conversions between the bool/uint8 block mask of the reference
// (block_sparse_attn_func's base_blockmask, dfsattn/attention_wan.py:252-253,
// 359) and the CSR block lists the attention kernel consumes. One wave per
// mask row.
#include "common.h"

namespace dfs {
namespace {

__global__ void __launch_bounds__(256) mask_counts_kernel(const uint8_t* __restrict__ mask,
                                                          int64_t rows, int kb,
                                                          int32_t* __restrict__ counts) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint8_t* m = mask + row * kb;
  int n = 0;
  for (int j = lane; j < kb; j += kWave) n += m[j] != 0;
  for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off);
  if (lane == 0) counts[row] = n;
}

__global__ void __launch_bounds__(256) mask_to_csr_kernel(const uint8_t* __restrict__ mask,
                                                          int64_t rows, int kb,
                                                          const int32_t* __restrict__ row_ptr,
                                                          int32_t* __restrict__ col_idx) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint8_t* m = mask + row * kb;
  int32_t* out = col_idx + row_ptr[row];
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int n = 0;
  for (int base = 0; base < kb; base += kWave) {
    const int j = base + lane;
    const bool on = j < kb && m[j] != 0;
    const uint64_t bal = __ballot(on);
    if (on) out[n + __popcll(bal & below)] = j;
    n += __popcll(bal);
  }
}

__global__ void __launch_bounds__(256) csr_to_mask_kernel(const int32_t* __restrict__ row_ptr,
                                                          const int32_t* __restrict__ col_idx,
                                                          int64_t rows, int kb,
                                                          uint8_t* __restrict__ mask) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  uint8_t* m = mask + row * kb;
  const int beg = row_ptr[row], end = row_ptr[row + 1];
  // Membership test per column keeps every byte written exactly once.
  for (int j = lane; j < kb; j += kWave) {
    int lo = beg, hi = end;  // columns are ascending: binary search
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (col_idx[mid] < j) lo = mid + 1; else hi = mid;
    }
    m[j] = (lo < end && col_idx[lo] == j) ? 1 : 0;
  }
}

}  // namespace
}  // namespace dfs

extern "C" {

int dfs_mask_row_counts(const uint8_t* mask, int64_t rows, int64_t k_blocks, int32_t* counts,
                        dfs_stream_t stream) {
  DFS_REQUIRE(mask && counts, "dfs_mask_row_counts: NULL operand");
  DFS_REQUIRE(rows >= 0 && k_blocks > 0 && k_blocks < (1 << 30), "dfs_mask_row_counts: bad shape");
  if (rows == 0) return 0;
  dfs::mask_counts_kernel<<<static_cast<unsigned>((rows + 3) / 4), 256, 0,
                            reinterpret_cast<hipStream_t>(stream)>>>(mask, rows,
                                                                     static_cast<int>(k_blocks), counts);
  return dfs::check_launch("dfs_mask_row_counts");
}

int dfs_mask_to_csr(const uint8_t* mask, int64_t rows, int64_t k_blocks, const int32_t* row_ptr,
                    int32_t* col_idx, dfs_stream_t stream) {
  DFS_REQUIRE(mask && row_ptr && col_idx, "dfs_mask_to_csr: NULL operand");
  DFS_REQUIRE(rows >= 0 && k_blocks > 0 && k_blocks < (1 << 30), "dfs_mask_to_csr: bad shape");
  if (rows == 0) return 0;
  dfs::mask_to_csr_kernel<<<static_cast<unsigned>((rows + 3) / 4), 256, 0,
                            reinterpret_cast<hipStream_t>(stream)>>>(
      mask, rows, static_cast<int>(k_blocks), row_ptr, col_idx);
  return dfs::check_launch("dfs_mask_to_csr");
}

int dfs_csr_to_mask(const int32_t* row_ptr, const int32_t* col_idx, int64_t rows, int64_t k_blocks,
                    uint8_t* mask, dfs_stream_t stream) {
  DFS_REQUIRE(row_ptr && col_idx && mask, "dfs_csr_to_mask: NULL operand");
  DFS_REQUIRE(rows >= 0 && k_blocks > 0 && k_blocks < (1 << 30), "dfs_csr_to_mask: bad shape");
  if (rows == 0) return 0;
  dfs::csr_to_mask_kernel<<<static_cast<unsigned>((rows + 3) / 4), 256, 0,
                            reinterpret_cast<hipStream_t>(stream)>>>(
      row_ptr, col_idx, rows, static_cast<int>(k_blocks), mask);
  return dfs::check_launch("dfs_csr_to_mask");
}

}  // extern "C"

// Host-side parts of the C-ABI: error reporting and the 3D Hilbert order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <utility>
#include <vector>

#include "common.h"

namespace dfs {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return 2;
  }
  return 0;
}

// Hilbert index of one point in the convention of numpy-hilbert-curve's
// encode(locs, num_dims, num_bits) (called at dfsattn/utils/order.py:250).
// That library implements Skilling's "Programming the Hilbert curve" (AIP
// Conf. Proc. 707, 2004): the transpose step ("inverse undo" over bit levels
// from the most significant, dimensions in column order), then the bits are
// interleaved level by level with dimension 0 first, and the interleaved
// string is Gray-decoded (prefix XOR) into the integer.
static uint64_t hilbert_index(uint32_t x[3], int dims, int bits) {
  for (uint32_t q = 1u << (bits - 1); q > 1; q >>= 1) {
    const uint32_t p = q - 1;
    for (int i = 0; i < dims; ++i) {
      if (x[i] & q) {
        x[0] ^= p;
      } else {
        const uint32_t t = (x[0] ^ x[i]) & p;
        x[0] ^= t;
        x[i] ^= t;
      }
    }
  }
  uint64_t gray = 0;
  for (int j = bits - 1; j >= 0; --j)
    for (int i = 0; i < dims; ++i) gray = (gray << 1) | ((x[i] >> j) & 1u);
  uint64_t bin = gray;
  for (int s = 1; s < 64; s <<= 1) bin ^= bin >> s;
  return bin;
}

}  // namespace dfs

extern "C" {

const char* dfs_last_error(void) { return dfs::g_error; }

int dfs_abi_version(void) { return 5; }

int dfs_hilbert3d_perm(int64_t f, int64_t h, int64_t w, int64_t* perm_out) {
  DFS_REQUIRE(f > 0 && h > 0 && w > 0, "hilbert3d_perm: grid %lldx%lldx%lld must be positive",
              (long long)f, (long long)h, (long long)w);
  DFS_REQUIRE(perm_out != nullptr, "hilbert3d_perm: perm_out is NULL");
  const int64_t max_dim = std::max(w, std::max(h, f));
  int bits = 1;
  while ((int64_t(1) << bits) < max_dim) ++bits;  // max(1, ceil(log2(max_dim)))
  DFS_REQUIRE(3 * bits <= 63, "hilbert3d_perm: grid too large for a 63-bit Hilbert index");
  const int64_t n = f * h * w;
  std::vector<std::pair<uint64_t, int64_t>> keyed(static_cast<size_t>(n));
  for (int64_t z = 0; z < f; ++z)
    for (int64_t y = 0; y < h; ++y)
      for (int64_t x = 0; x < w; ++x) {
        uint32_t c[3] = {static_cast<uint32_t>(x), static_cast<uint32_t>(y),
                         static_cast<uint32_t>(z)};
        const int64_t idx = z * h * w + y * w + x;
        keyed[static_cast<size_t>(idx)] = {dfs::hilbert_index(c, 3, bits), idx};
      }
  // Indices are unique, so the order (and argsort's result) is unambiguous.
  std::sort(keyed.begin(), keyed.end());
  for (int64_t i = 0; i < n; ++i) perm_out[i] = keyed[static_cast<size_t>(i)].second;
  return 0;
}

}  // extern "C"

// Shared helpers for the gfx950 DFS sparse-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dfsattn_amd.h"

namespace dfs {

// Records a printf-style message as the calling thread's last error.
void set_error(const char* fmt, ...);
// Turns a pending launch error into a status code (0 = ok).
int check_launch(const char* what);

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr int kBlock = 128;  // mask granularity (tokens per block)
constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16));
  return static_cast<float>(h);
}

// Round-to-nearest-even float -> bf16 bits.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  __bf16 b = static_cast<__bf16>(x);
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  _Float16 h = static_cast<_Float16>(x);
  return __builtin_bit_cast(uint16_t, h);
}

// Element of a packed 8 x 16-bit vector held in a uint4.
__device__ __forceinline__ uint32_t u16_at(const uint4& v, int i) {
  uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
  return (i & 1) ? (w >> 16) : (w & 0xffffu);
}

__device__ __forceinline__ float exp2_fast(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// Streaming 16-byte accesses (nontemporal hint) for data a kernel reads or
// writes exactly once: they keep it from displacing cache lines that others
// reuse.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void store_stream(uint4* p, const uint4& v) {
  const u32x4_t t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t*>(p));
}

}  // namespace dfs

#define DFS_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::dfs::set_error(__VA_ARGS__);  \
      return 1;                       \
    }                                 \
  } while (0)

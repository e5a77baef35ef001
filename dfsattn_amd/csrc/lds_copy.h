// Global -> LDS tile copies for gfx950 kernels: raw buffer descriptors,
// 16-byte buffer loads that write LDS directly (no VGPR round trip), explicit
// vmcnt waits and barriers, and the XOR chunk swizzle of 2^k-byte LDS rows.
#pragma once

#include "common.h"

namespace dfs {
namespace {

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

// Copy of one tile into LDS with the chunk swizzle by NW waves: load j of wave
// w fills LDS bytes [(NW*j + w) * 1024, +1024), i.e. 1024/ROWB rows. The
// swizzle depends on the row modulo the chunks per row, which is the same for
// every j, so one per-thread byte offset serves all loads and the j-th load
// only adds j * NW KiB to the scalar offset.
template <int ROWB, int NW = 4>
struct TileCopy {
  static constexpr int CPR = ROWB / 16;   // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;    // rows per wave instruction
  uint32_t voff;
  __device__ __forceinline__ TileCopy(int wave, int lane) {
    const int r = wave * RPI + lane / CPR;
    voff = static_cast<uint32_t>(r * ROWB + (((lane % CPR) ^ (r % CPR)) * 16));
  }
  // LOADS 16-byte loads per thread (NW * LOADS KiB in all) from byte tile_off.
  template <int LOADS>
  __device__ __forceinline__ void issue(sgpr4 rs, uint32_t tile_off, uint32_t lds_base,
                                        int wave) const {
    // Opaque per call: keeps the compiler from hoisting all LOADS LDS
    // addresses out of the loop into (spilled) scalar registers.
    asm volatile("" : "+s"(lds_base));
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
      load_lds16(rs, lds_base + (j * NW + wave) * 1024, voff, tile_off + j * NW * 1024);
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

}  // namespace
}  // namespace dfs

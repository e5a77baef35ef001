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

// Raw buffer resource over `bytes` bytes starting at `base` (stride 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void;

// Copy of one tile into LDS with the chunk swizzle by NW waves, as 16-byte
// buffer loads that write LDS directly (no VGPR round trip): load j of wave w
// reads buffer bytes tile_off + j * NW KiB + voff and fills LDS bytes
// [(NW*j + w) * 1024, +1024) of the tile, i.e. 1024/ROWB rows. The swizzle
// depends on the row modulo the chunks per row, which is the same for every
// j, so one per-thread byte offset serves all loads. The loads go through the
// compiler's buffer-to-LDS builtin, so M0, the hazards around it and the
// waits before later reads of the same LDS object are the compiler's; the
// kernels add explicit vmcnt waits plus a barrier before other waves read
// the tile.
template <int ROWB, int NW = 4>
struct TileCopy {
  static constexpr int CPR = ROWB / 16;   // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;    // rows per wave instruction
  uint32_t voff;
  __device__ __forceinline__ TileCopy(int wave, int lane) {
    const int r = wave * RPI + lane / CPR;
    voff = static_cast<uint32_t>(r * ROWB + (((lane % CPR) ^ (r % CPR)) * 16));
  }
  // LOADS 16-byte loads per thread (NW * LOADS KiB in all) from byte tile_off
  // into the LDS tile at `tile`.
  template <int LOADS>
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, uint32_t tile_off, void* tile, int wave) const {
#pragma unroll
    for (int j = 0; j < LOADS; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void*)(static_cast<char*>(tile) + (j * NW + wave) * 1024), 16, voff,
          static_cast<int>(tile_off + j * NW * 1024), 0, 0);
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

// Fused elementwise kernels of the DiT block around the attention (the Wan
// transformer block of diffusers that the reference's Wan driver loads,
// wan21_t2v_inference.py:102-103): the fp32 LayerNorm with adaLN modulation,
//   y = bf16((LN(x) [* w + b]) * (1 + scale) + shift),
// and the gated residual,
//   out = bf16(float(x) + float(y) * gate),
// each one pass over the rows instead of torch's chain of dtype copies and
// broadcast ops. Every fp32 product and sum is rounded separately, in the
// order torch evaluates the same expressions; only the LayerNorm's reduction
// order differs.
#include "common.h"

namespace dfs {
namespace {

constexpr int kMaxChunks = 16;  // at most 16 x 512 channels per row

__device__ __forceinline__ float to_f32(uint32_t bits, int dtype) {
  return dtype == DFS_DTYPE_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

__device__ __forceinline__ uint32_t from_f32(float v, int dtype) {
  return dtype == DFS_DTYPE_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// One wave per row of C channels (16-byte chunks, 512 channels per wave
// step, the row held in registers for the two-pass mean and variance).
template <int NCH>
__global__ void __launch_bounds__(256) adaln_kernel(const uint16_t* __restrict__ x, int64_t rows, int C, int dtype,
                                                    const float* __restrict__ weight, const float* __restrict__ bias,
                                                    const float* __restrict__ scale, const float* __restrict__ shift,
                                                    float eps, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* xr = x + row * C;
  uint4 v[NCH];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e = j * 512 + lane * 8;
    if (e < C) {
      v[j] = *reinterpret_cast<const uint4*>(xr + e);
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += to_f32(u16_at(v[j], i), dtype);
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(C);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (j * 512 + lane * 8 < C) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = to_f32(u16_at(v[j], i), dtype) - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) / static_cast<float>(C) + eps);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e = j * 512 + lane * 8;
    if (e >= C) continue;
    float w[8], b[8], sc[8], sh[8];
    if (weight) load8(weight + e, w);
    if (bias) load8(bias + e, b);
    if (scale) load8(scale + e, sc);
    if (shift) load8(shift + e, sh);
    uint32_t packed[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float y2[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma clang fp contract(off)
        float y = (to_f32(u16_at(v[j], i + t), dtype) - mean) * rstd;
        if (weight) y = y * w[i + t];
        if (bias) y = y + b[i + t];
        if (scale) y = y * (1.0f + sc[i + t]);
        if (shift) y = y + sh[i + t];
        y2[t] = y;
      }
      packed[i / 2] = from_f32(y2[0], dtype) | (from_f32(y2[1], dtype) << 16);
    }
    *reinterpret_cast<uint4*>(out + row * C + e) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
}

// out = float(x) + float(y) * gate[c], eight channels per thread.
// x and out may alias (each thread reads its eight elements before writing them).
__global__ void __launch_bounds__(256) gated_residual_kernel(const uint16_t* x, const uint16_t* __restrict__ y,
                                                             const float* __restrict__ gate, int64_t n8, int C,
                                                             int dtype, uint16_t* out) {
  const int64_t i8 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i8 >= n8) return;
  const int64_t e = i8 * 8;
  const int c = static_cast<int>(e % C);
  const uint4 xv = *reinterpret_cast<const uint4*>(x + e);
  const uint4 yv = *reinterpret_cast<const uint4*>(y + e);
  float g[8];
  load8(gate + c, g);
  uint32_t packed[4];
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float r[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma clang fp contract(off)
      r[t] = to_f32(u16_at(xv, i + t), dtype) + to_f32(u16_at(yv, i + t), dtype) * g[i + t];
    }
    packed[i / 2] = from_f32(r[0], dtype) | (from_f32(r[1], dtype) << 16);
  }
  *reinterpret_cast<uint4*>(out + e) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace dfs

extern "C" int dfs_adaln_modulate(const void* x, int64_t rows, int64_t channels, int dtype, const float* weight,
                                  const float* bias, const float* scale, const float* shift, float eps, void* out,
                                  dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "adaln_modulate";
  DFS_REQUIRE(x && out, "%s: x and out must be non-NULL", name);
  DFS_REQUIRE(rows > 0 && channels > 0 && channels % 8 == 0 && channels <= 512 * kMaxChunks,
              "%s: channels=%lld must be a positive multiple of 8 up to %d", name, (long long)channels,
              512 * kMaxChunks);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16, "%s: dtype must be bf16 or f16", name);
  DFS_REQUIRE(eps >= 0.f, "%s: eps must be non-negative", name);
  const void* ptrs[6] = {x, out, weight, bias, scale, shift};
  for (const void* q : ptrs) DFS_REQUIRE(q == nullptr || aligned16(q), "%s: operands must be 16-byte aligned", name);
  const int64_t blocks = (rows + 3) / 4;
  DFS_REQUIRE(blocks < (int64_t(1) << 31), "%s: too many rows", name);
  const int nch = static_cast<int>((channels + 511) / 512);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint16_t* op = static_cast<uint16_t*>(out);
  const int C = static_cast<int>(channels);
  switch ((nch + 1) / 2) {  // smallest even chunk count that covers the row
#define DFS_ADALN_CASE(HALF)                                                                                  \
  case HALF:                                                                                                  \
    hipLaunchKernelGGL(adaln_kernel<2 * HALF>, grid, block, 0, st, xp, rows, C, dtype, weight, bias, scale, shift, \
                       eps, op);                                                                              \
    break;
    DFS_ADALN_CASE(1)
    DFS_ADALN_CASE(2)
    DFS_ADALN_CASE(3)
    DFS_ADALN_CASE(4)
    DFS_ADALN_CASE(5)
    DFS_ADALN_CASE(6)
    DFS_ADALN_CASE(7)
    DFS_ADALN_CASE(8)
#undef DFS_ADALN_CASE
    default:
      set_error("%s: internal chunk count %d", name, nch);
      return 1;
  }
  return check_launch(name);
}

extern "C" int dfs_gated_residual(const void* x, const void* y, const float* gate, int64_t rows, int64_t channels,
                                  int dtype, void* out, dfs_stream_t stream) {
  using namespace dfs;
  const char* name = "gated_residual";
  DFS_REQUIRE(x && y && gate && out, "%s: NULL operand", name);
  DFS_REQUIRE(rows > 0 && channels > 0 && channels % 8 == 0, "%s: channels=%lld must be a positive multiple of 8",
              name, (long long)channels);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16, "%s: dtype must be bf16 or f16", name);
  DFS_REQUIRE(aligned16(x) && aligned16(y) && aligned16(gate) && aligned16(out),
              "%s: operands must be 16-byte aligned", name);
  DFS_REQUIRE(channels < (int64_t(1) << 31), "%s: too many channels", name);
  const int64_t n8 = rows * channels / 8;
  const int64_t blocks = (n8 + 255) / 256;
  DFS_REQUIRE(blocks < (int64_t(1) << 31), "%s: too many elements", name);
  hipLaunchKernelGGL(gated_residual_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                     static_cast<const uint16_t*>(y), gate, n8, static_cast<int>(channels), dtype,
                     static_cast<uint16_t*>(out));
  return check_launch(name);
}

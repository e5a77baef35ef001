// Fused QK RMSNorm + complex RoPE + head split for the DiT attention inputs.
//
// One wave owns one token row of C = H*D channels: it loads the row (16-byte
// chunks, 512 channels per wave step, C <= 8192 held in registers), reduces
// the sum of squares across the wave, normalises and scales by the weight,
// rounds to the storage dtype, rotates adjacent (even, odd) channel pairs of
// each head by the token's (cos, sin) in float64, and writes the row into any
// [B][H][L][D]-strided destination (so the head split / transpose of the
// reference's unflatten(2, (H, -1)).transpose(1, 2) costs nothing extra).
//
// Reference semantics followed:
//   - RMSNorm: dfsattn/kernels/triton/rmsnorm.py:9-48 — x in fp32,
//     var = sum(x*x) / C, rstd = 1 / sqrt(var + eps), y = (x * rstd) * w,
//     rounded to the input dtype.
//   - RoPE: dfsattn/kernels/include/rope/rope_enc_complex.cuh (the kernel
//     behind apply_qk_rope_inplace_cossin_complex, kernels/csrc/ops.h:207-261)
//     — out[2i] = x[2i] c - x[2i+1] s, out[2i+1] = x[2i+1] c + x[2i] s in
//     float64 with fp32 cos/sin [L - skip][D/2]; the first `skip` rows are
//     left as they are. The float64 result is rounded to float32 and then to
//     the storage dtype, which is torch's float64 -> bf16/f16 conversion
//     (the reference's fallback at replace_wan.py:209-213).
#include "common.h"

namespace dfs {
namespace {

constexpr int kMaxChunks = 16;  // at most 16 x 512 channels per row

struct NormRopeParams {
  int64_t x_sb, x_sl, x_sh;  // element strides of x (channel stride 1)
  int64_t o_sb, o_sl, o_sh;  // element strides of out
  int64_t rows;              // B * L
  int L, H, D, C, nch;
  int dtype;                 // DFS_DTYPE_BF16 / F16
  int w_dtype;               // weight dtype, -1 = no norm
  float eps;
  int rope_skip;             // rows l < rope_skip are not rotated
};

__device__ __forceinline__ float to_f32(uint32_t bits, int dtype) {
  return dtype == DFS_DTYPE_BF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits);
}

__device__ __forceinline__ uint32_t from_f32(float v, int dtype) {
  return dtype == DFS_DTYPE_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

__device__ __forceinline__ float wave_sum(float v) {
  // xor butterfly: every lane adds the same pairs (a + b == b + a), so all
  // lanes end with the same bits
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// NCH: 512-channel chunks held per lane (the smallest even count that covers
// the row: 10 for 5,120 channels). The weights and the RoPE table row are fetched together
// with x, before the reduction, so no second memory round trip sits
// between the reduction and the stores.
template <int NCH>
__global__ void __launch_bounds__(256) norm_rope_kernel(const uint16_t* x, uint16_t* out,  // may alias (in place)
                                                        const void* __restrict__ weight,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, NormRopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int64_t b = row / p.L;
  const int l = static_cast<int>(row - b * p.L);
  const uint16_t* xr = x + b * p.x_sb + static_cast<int64_t>(l) * p.x_sl;
  uint16_t* orow = out + b * p.o_sb + static_cast<int64_t>(l) * p.o_sl;
  const bool norm = p.w_dtype >= 0;
  const int lr = l - p.rope_skip;
  const bool rope = cos_t != nullptr && lr >= 0;
  const int half = p.D >> 1;
  // 512 % D == 0 (D = 64, 128, ...): every chunk of a lane has the same
  // channel d, so one (cos, sin) row slice serves all of them
  const bool same_d = (512 % p.D) == 0;

  uint4 v[NCH];
  uint4 wv[NCH];  // bf16/f16 weights
  float4 cs_same = make_float4(0.f, 0.f, 0.f, 0.f), sn_same = cs_same;
  if (rope && same_d) {
    const int d0 = (lane * 8) % p.D;
    cs_same = *reinterpret_cast<const float4*>(cos_t + static_cast<int64_t>(lr) * half + (d0 >> 1));
    sn_same = *reinterpret_cast<const float4*>(sin_t + static_cast<int64_t>(lr) * half + (d0 >> 1));
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e = j * 512 + lane * 8;
    if (e < p.C) {
      const int h = e / p.D, d = e - h * p.D;
      v[j] = *reinterpret_cast<const uint4*>(xr + h * p.x_sh + d);
      if (norm && p.w_dtype != DFS_DTYPE_F32) wv[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(weight) + e);
    }
  }
  float rstd = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j * 512 + lane * 8 < p.C) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float f = to_f32(u16_at(v[j], i), p.dtype);
          ss += f * f;
        }
      }
    }
    const float var = wave_sum(ss) / static_cast<float>(p.C);
    rstd = 1.0f / sqrtf(var + p.eps);
  }

#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e = j * 512 + lane * 8;
    if (e >= p.C) continue;
    const int h = e / p.D, d = e - h * p.D;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = to_f32(u16_at(v[j], i), p.dtype);
    if (norm) {
      float w[8];
      if (p.w_dtype == DFS_DTYPE_F32) {
        const float4 w0 = *reinterpret_cast<const float4*>(static_cast<const float*>(weight) + e);
        const float4 w1 = *reinterpret_cast<const float4*>(static_cast<const float*>(weight) + e + 4);
        w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
        w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = to_f32(u16_at(wv[j], i), p.w_dtype);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xh = y[i] * rstd;  // two roundings, as x_hat = x * rstd; y = x_hat * w
        y[i] = to_f32(from_f32(xh * w[i], p.dtype), p.dtype);
      }
    }
    if (rope) {
      float4 c4 = cs_same, s4 = sn_same;
      if (!same_d) {
        c4 = *reinterpret_cast<const float4*>(cos_t + static_cast<int64_t>(lr) * half + (d >> 1));
        s4 = *reinterpret_cast<const float4*>(sin_t + static_cast<int64_t>(lr) * half + (d >> 1));
      }
      const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double xe = y[2 * i], xo = y[2 * i + 1];
        // products of a 16-bit float and an fp32 are exact in float64, so
        // only the sums round
        const double re = xe * static_cast<double>(cs[i]) - xo * static_cast<double>(sn[i]);
        const double im = xo * static_cast<double>(cs[i]) + xe * static_cast<double>(sn[i]);
        y[2 * i] = static_cast<float>(re);
        y[2 * i + 1] = static_cast<float>(im);
      }
    }
    uint32_t packed[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      packed[i] = from_f32(y[2 * i], p.dtype) | (from_f32(y[2 * i + 1], p.dtype) << 16);
    *reinterpret_cast<uint4*>(orow + h * p.o_sh + d) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
}

}  // namespace
}  // namespace dfs

extern "C" int dfs_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int64_t x_sh, void* out, int64_t o_sb,
                             int64_t o_sl, int64_t o_sh, int64_t batch, int64_t seq_len, int64_t heads,
                             int64_t head_dim, int dtype, const void* weight, int weight_dtype, float eps,
                             const float* cos_table, const float* sin_table, int64_t rope_skip,
                             dfs_stream_t stream) {
  using namespace dfs;
  DFS_REQUIRE(x != nullptr && out != nullptr, "norm_rope: x and out must be non-NULL");
  DFS_REQUIRE(batch > 0 && seq_len > 0 && heads > 0, "norm_rope: batch, seq_len and heads must be positive");
  DFS_REQUIRE(head_dim > 0 && head_dim % 8 == 0, "norm_rope: head_dim %lld must be a positive multiple of 8",
              (long long)head_dim);
  const int64_t C = heads * head_dim;
  DFS_REQUIRE(C <= 512 * kMaxChunks, "norm_rope: heads*head_dim = %lld exceeds %d", (long long)C, 512 * kMaxChunks);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16, "norm_rope: dtype must be bf16 or f16");
  DFS_REQUIRE(weight == nullptr || weight_dtype == DFS_DTYPE_BF16 || weight_dtype == DFS_DTYPE_F16 ||
                  weight_dtype == DFS_DTYPE_F32,
              "norm_rope: weight dtype code %d is not supported", weight_dtype);
  DFS_REQUIRE(weight == nullptr || eps >= 0.f, "norm_rope: eps must be non-negative");
  DFS_REQUIRE((cos_table == nullptr) == (sin_table == nullptr), "norm_rope: pass both cos and sin tables or neither");
  DFS_REQUIRE(rope_skip >= 0 && rope_skip < seq_len, "norm_rope: rope_skip %lld must lie in [0, seq_len)",
              (long long)rope_skip);
  const int64_t strides[6] = {x_sb, x_sl, x_sh, o_sb, o_sl, o_sh};
  for (int i = 0; i < 6; ++i)
    DFS_REQUIRE(strides[i] >= 0 && strides[i] % 8 == 0,
                "norm_rope: strides must be non-negative multiples of 8 elements (16-byte rows)");
  DFS_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
              "norm_rope: x and out must be 16-byte aligned");
  DFS_REQUIRE(weight == nullptr || reinterpret_cast<uintptr_t>(weight) % 16 == 0,
              "norm_rope: weight must be 16-byte aligned");
  DFS_REQUIRE(cos_table == nullptr ||
                  (reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table)) % 16 == 0,
              "norm_rope: cos and sin tables must be 16-byte aligned");
  NormRopeParams p;
  p.x_sb = x_sb; p.x_sl = x_sl; p.x_sh = x_sh;
  p.o_sb = o_sb; p.o_sl = o_sl; p.o_sh = o_sh;
  p.rows = batch * seq_len;
  p.L = static_cast<int>(seq_len);
  p.H = static_cast<int>(heads);
  p.D = static_cast<int>(head_dim);
  p.C = static_cast<int>(C);
  p.nch = static_cast<int>((C + 511) / 512);
  p.dtype = dtype;
  p.w_dtype = weight ? weight_dtype : -1;
  p.eps = eps;
  p.rope_skip = static_cast<int>(rope_skip);
  DFS_REQUIRE(seq_len < (int64_t(1) << 31), "norm_rope: seq_len too large");
  const int64_t blocks = (p.rows + 3) / 4;
  DFS_REQUIRE(blocks < (int64_t(1) << 31), "norm_rope: too many rows");
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint16_t* xs = static_cast<const uint16_t*>(x);
  uint16_t* os = static_cast<uint16_t*>(out);
  switch ((p.nch + 1) / 2) {  // smallest even chunk count that covers the row
#define DFS_NORM_ROPE_CASE(HALF)                                                                        \
  case HALF:                                                                                           \
    hipLaunchKernelGGL(norm_rope_kernel<2 * HALF>, grid, block, 0, st, xs, os, weight, cos_table, sin_table, \
                       p);                                                                             \
    break;
    DFS_NORM_ROPE_CASE(1)
    DFS_NORM_ROPE_CASE(2)
    DFS_NORM_ROPE_CASE(3)
    DFS_NORM_ROPE_CASE(4)
    DFS_NORM_ROPE_CASE(5)
    DFS_NORM_ROPE_CASE(6)
    DFS_NORM_ROPE_CASE(7)
    DFS_NORM_ROPE_CASE(8)
#undef DFS_NORM_ROPE_CASE
    default:
      set_error("norm_rope: internal chunk count %d", p.nch);
      return 1;
  }
  return check_launch("norm_rope");
}

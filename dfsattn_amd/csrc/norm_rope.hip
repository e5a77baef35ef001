// Fused QK RMSNorm + RoPE + head split for the DiT attention inputs.
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
//   - Per-head variant (HunyuanVideo): RMSNorm of each head's D channels as
//     the reference's narrow RMSNorm kernel (kernels/include/norm/
//     narrow_rms_norm.cuh, called through kernels/__init__.py apply_qk_norm)
//     and real RoPE on the video rows with fp32 tables [rows][D]
//     (rope_enc_txtlast.cuh, apply_qk_rope_single/double):
//     out[2i] = x[2i] cos[2i] - x[2i+1] sin[2i], out[2i+1] = x[2i+1] cos[2i+1]
//     + x[2i] sin[2i+1], each product and sum rounded in fp32 (the
//     reference's torch fallback, replace_hyvideo.py:271-290).
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
  int per_head;              // 0: norm over all H*D channels (weight [H*D]); 1: per head (weight [D])
  int rope_kind;             // 0 none; 1 complex, float64; 2 real, fp32
  int rope_skip;             // kind 1: rows l < rope_skip are not rotated, table row l - rope_skip
  int rope_rows;             // kind 2: rows l < rope_rows are rotated, table row l
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
// the row: 10 for 5,120 channels). The weights and the RoPE table row are
// fetched together with x, before the reduction, so no second memory round
// trip sits between the reduction and the stores.
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
  // kind 1: complex pairs, table [L - skip][D/2]; kind 2: real, table [rows][D]
  const bool rope1 = p.rope_kind == 1 && l >= p.rope_skip;
  const bool rope2 = p.rope_kind == 2 && l < p.rope_rows;
  const int64_t trow = rope1 ? static_cast<int64_t>(l - p.rope_skip) * (p.D >> 1) : static_cast<int64_t>(l) * p.D;
  // 512 % D == 0 (D = 64, 128, ...): every chunk of a lane has the same
  // channel d, so one slice of the table row serves all of them
  const bool same_d = (512 % p.D) == 0;

  uint4 v[NCH];
  uint4 wv[NCH];  // bf16/f16 weights
  float cs[8] = {}, sn[8] = {};
  auto load_table = [&](int d) {
    if (rope1) {
      const float4 c4 = *reinterpret_cast<const float4*>(cos_t + trow + (d >> 1));
      const float4 s4 = *reinterpret_cast<const float4*>(sin_t + trow + (d >> 1));
      cs[0] = c4.x; cs[1] = c4.y; cs[2] = c4.z; cs[3] = c4.w;
      sn[0] = s4.x; sn[1] = s4.y; sn[2] = s4.z; sn[3] = s4.w;
    } else if (rope2) {
      const float4 c0 = *reinterpret_cast<const float4*>(cos_t + trow + d);
      const float4 c1 = *reinterpret_cast<const float4*>(cos_t + trow + d + 4);
      const float4 s0 = *reinterpret_cast<const float4*>(sin_t + trow + d);
      const float4 s1 = *reinterpret_cast<const float4*>(sin_t + trow + d + 4);
      cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
      sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    }
  };
  if (same_d) load_table((lane * 8) % p.D);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int e = j * 512 + lane * 8;
    if (e < p.C) {
      const int h = e / p.D, d = e - h * p.D;
      v[j] = *reinterpret_cast<const uint4*>(xr + h * p.x_sh + d);
      if (norm && p.w_dtype != DFS_DTYPE_F32)
        wv[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(weight) + (p.per_head ? d : e));
    }
  }
  // 1/rms of the norm group of each chunk's channels (one value for all
  // chunks when the group is the whole row)
  float rstd[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) rstd[j] = 1.f;
  if (norm) {
    if (!p.per_head) {
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
      const float r = 1.0f / sqrtf(wave_sum(ss) / static_cast<float>(p.C) + p.eps);
#pragma unroll
      for (int j = 0; j < NCH; ++j) rstd[j] = r;
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        float ss = 0.f;
        if (j * 512 + lane * 8 < p.C) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float f = to_f32(u16_at(v[j], i), p.dtype);
            ss += f * f;
          }
        }
        // the D/8 lanes of a head (aligned groups, as 512 % D == 0): a xor
        // butterfly leaves the same bits in all of them
        for (int off = p.D >> 4; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
        rstd[j] = 1.0f / sqrtf(ss / static_cast<float>(p.D) + p.eps);
      }
    }
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
        const float* wp = static_cast<const float*>(weight) + (p.per_head ? d : e);
        const float4 w0 = *reinterpret_cast<const float4*>(wp);
        const float4 w1 = *reinterpret_cast<const float4*>(wp + 4);
        w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w;
        w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = to_f32(u16_at(wv[j], i), p.w_dtype);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xh = y[i] * rstd[j];  // two roundings, as x_hat = x * rstd; y = x_hat * w
        y[i] = to_f32(from_f32(xh * w[i], p.dtype), p.dtype);
      }
    }
    if (!same_d) load_table(d);
    if (rope1) {
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
    } else if (rope2) {
#pragma clang fp contract(off)
      // x * cos + rotate(x) * sin with every product and sum rounded (no fusion)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float xe = y[2 * i], xo = y[2 * i + 1];
        y[2 * i] = xe * cs[2 * i] + (-xo) * sn[2 * i];
        y[2 * i + 1] = xo * cs[2 * i + 1] + xe * sn[2 * i + 1];
      }
    }
    uint32_t packed[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      packed[i] = from_f32(y[2 * i], p.dtype) | (from_f32(y[2 * i + 1], p.dtype) << 16);
    *reinterpret_cast<uint4*>(orow + h * p.o_sh + d) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
}

// Checks shared by both entry points, then the launch. per_head selects the
// norm group (a head of D channels, weight [D]) and the RoPE form (real
// tables [rope_rows][D] for rows l < rope_rows); otherwise the group is the
// whole row (weight [H*D]) and the RoPE complex (tables [L - rope_skip][D/2]
// for rows l >= rope_skip).
int launch_norm_rope(const char* name, const void* x, const int64_t* xs3, void* out, const int64_t* os3,
                     int64_t batch, int64_t seq_len, int64_t heads, int64_t head_dim, int dtype, const void* weight,
                     int weight_dtype, float eps, const float* cos_table, const float* sin_table, int per_head,
                     int64_t rope_param, hipStream_t st) {
  DFS_REQUIRE(x != nullptr && out != nullptr, "%s: x and out must be non-NULL", name);
  DFS_REQUIRE(batch > 0 && seq_len > 0 && heads > 0, "%s: batch, seq_len and heads must be positive", name);
  DFS_REQUIRE(head_dim > 0 && head_dim % 8 == 0, "%s: head_dim %lld must be a positive multiple of 8", name,
              (long long)head_dim);
  DFS_REQUIRE(!per_head || (head_dim <= 512 && (head_dim & (head_dim - 1)) == 0),
              "%s: head_dim %lld must be a power of two <= 512 for the per-head norm", name, (long long)head_dim);
  const int64_t C = heads * head_dim;
  DFS_REQUIRE(C <= 512 * kMaxChunks, "%s: heads*head_dim = %lld exceeds %d", name, (long long)C, 512 * kMaxChunks);
  DFS_REQUIRE(dtype == DFS_DTYPE_BF16 || dtype == DFS_DTYPE_F16, "%s: dtype must be bf16 or f16", name);
  DFS_REQUIRE(weight == nullptr || weight_dtype == DFS_DTYPE_BF16 || weight_dtype == DFS_DTYPE_F16 ||
                  weight_dtype == DFS_DTYPE_F32,
              "%s: weight dtype code %d is not supported", name, weight_dtype);
  DFS_REQUIRE(weight == nullptr || eps >= 0.f, "%s: eps must be non-negative", name);
  DFS_REQUIRE((cos_table == nullptr) == (sin_table == nullptr), "%s: pass both cos and sin tables or neither", name);
  if (per_head)
    DFS_REQUIRE(rope_param >= 0 && rope_param <= seq_len, "%s: rope_rows %lld must lie in [0, seq_len]", name,
                (long long)rope_param);
  else
    DFS_REQUIRE(rope_param >= 0 && rope_param < seq_len, "%s: rope_skip %lld must lie in [0, seq_len)", name,
                (long long)rope_param);
  for (int i = 0; i < 3; ++i)
    DFS_REQUIRE(xs3[i] >= 0 && xs3[i] % 8 == 0 && os3[i] >= 0 && os3[i] % 8 == 0,
                "%s: strides must be non-negative multiples of 8 elements (16-byte rows)", name);
  DFS_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
              "%s: x and out must be 16-byte aligned", name);
  DFS_REQUIRE(weight == nullptr || reinterpret_cast<uintptr_t>(weight) % 16 == 0, "%s: weight must be 16-byte aligned",
              name);
  DFS_REQUIRE(cos_table == nullptr ||
                  (reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table)) % 16 == 0,
              "%s: cos and sin tables must be 16-byte aligned", name);
  DFS_REQUIRE(seq_len < (int64_t(1) << 31), "%s: seq_len too large", name);
  NormRopeParams p;
  p.x_sb = xs3[0]; p.x_sl = xs3[1]; p.x_sh = xs3[2];
  p.o_sb = os3[0]; p.o_sl = os3[1]; p.o_sh = os3[2];
  p.rows = batch * seq_len;
  p.L = static_cast<int>(seq_len);
  p.H = static_cast<int>(heads);
  p.D = static_cast<int>(head_dim);
  p.C = static_cast<int>(C);
  p.nch = static_cast<int>((C + 511) / 512);
  p.dtype = dtype;
  p.w_dtype = weight ? weight_dtype : -1;
  p.eps = eps;
  p.per_head = per_head;
  p.rope_kind = cos_table == nullptr ? 0 : (per_head ? 2 : 1);
  p.rope_skip = per_head ? 0 : static_cast<int>(rope_param);
  p.rope_rows = per_head ? static_cast<int>(rope_param) : 0;
  const int64_t blocks = (p.rows + 3) / 4;
  DFS_REQUIRE(blocks < (int64_t(1) << 31), "%s: too many rows", name);
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  uint16_t* op = static_cast<uint16_t*>(out);
  switch ((p.nch + 1) / 2) {  // smallest even chunk count that covers the row
#define DFS_NORM_ROPE_CASE(HALF)                                                                        \
  case HALF:                                                                                           \
    hipLaunchKernelGGL(norm_rope_kernel<2 * HALF>, grid, block, 0, st, xp, op, weight, cos_table, sin_table, \
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
      set_error("%s: internal chunk count %d", name, p.nch);
      return 1;
  }
  return check_launch(name);
}

}  // namespace
}  // namespace dfs

extern "C" int dfs_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int64_t x_sh, void* out, int64_t o_sb,
                             int64_t o_sl, int64_t o_sh, int64_t batch, int64_t seq_len, int64_t heads,
                             int64_t head_dim, int dtype, const void* weight, int weight_dtype, float eps,
                             const float* cos_table, const float* sin_table, int64_t rope_skip,
                             dfs_stream_t stream) {
  const int64_t xs3[3] = {x_sb, x_sl, x_sh}, os3[3] = {o_sb, o_sl, o_sh};
  return dfs::launch_norm_rope("norm_rope", x, xs3, out, os3, batch, seq_len, heads, head_dim, dtype, weight,
                               weight_dtype, eps, cos_table, sin_table, 0, rope_skip,
                               reinterpret_cast<hipStream_t>(stream));
}

extern "C" int dfs_head_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int64_t x_sh, void* out,
                                  int64_t o_sb, int64_t o_sl, int64_t o_sh, int64_t batch, int64_t seq_len,
                                  int64_t heads, int64_t head_dim, int dtype, const void* weight, int weight_dtype,
                                  float eps, const float* cos_table, const float* sin_table, int64_t rope_rows,
                                  dfs_stream_t stream) {
  const int64_t xs3[3] = {x_sb, x_sl, x_sh}, os3[3] = {o_sb, o_sl, o_sh};
  return dfs::launch_norm_rope("head_norm_rope", x, xs3, out, os3, batch, seq_len, heads, head_dim, dtype, weight,
                               weight_dtype, eps, cos_table, sin_table, 1, rope_rows,
                               reinterpret_cast<hipStream_t>(stream));
}

// Attention prologue of the decider's softmax-attention layers for gfx950:
// per-head RMSNorm of q and k over head_dim, then the partial rotary embedding,
// written token-major for the GQA kernel.
//
// Replaces the eager sequence of the reference's patched attention forward
// (ref: experiments/native_gqa/bench_native_gqa_model.py:47-53): chunk of the
// q_proj output into query / gate, q_norm, k_norm (transformers Qwen3_5RMSNorm:
// x * rsqrt(mean(x^2) + eps) * (1 + w), computed in fp32, one bf16 rounding),
// and apply_rotary_pos_emb on the first rotary_dim features, where every bf16
// product and sum is rounded as the eager bf16 ops round it:
//   r_i = bf16(bf16(y_i * cos_i) + bf16(rot_i * sin_i)),  rot = (-y[R/2:R], y[0:R/2])
// The features past rotary_dim pass through.
//
// HBM-bound: a 16-lane group owns one (token, head) row of 128 features, 8 per
// lane (one 16-byte load and store); the sum of squares is reduced with an xor
// butterfly inside the group and the rotation partner is one lane-xor away.
// fp32 sequence of the norm, the order PyTorch's GPU row mean uses at width 128
// (so the normed rows equal eager Qwen3_5RMSNorm bit for bit; the CPU
// restatement reproduces it):
//   lane: a = ((x0^2 + x1^2) + x2^2) + x3^2, b = the same over x4..x7, s = a + b
//   group: s += shfl_xor(s, 1, 2, 4, 8)
//   inv = fp32(1 / sqrt(s / 128 + eps)) from the fp64 root and quotient;  y = bf16((x * inv) * g),  g = 1 + w or w
#include <type_traits>

#include "fd_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kD = 128;

struct PrologueArgs {
  const uint16_t* q_in;
  const uint16_t* k_in;
  int64_t q_ts, q_hs, k_ts, k_hs;  // token / head strides of the inputs (elements)
  const void* q_w;
  const void* k_w;
  const uint16_t* cos;
  const uint16_t* sin;
  uint16_t* q_out;
  uint16_t* k_out;
  int64_t rows;  // tokens * (q_heads + kv_heads)
  int hq, hkv, rot, w_f32, gain_offset;
  int w_vec;  // both gain vectors 16-byte aligned: each lane loads its 8 gains as vectors
  float eps;
};

// round to bf16 and back (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ float bf16r(float x) { return fd_lo(fd_pack2(x, 0.0f)); }

__global__ __launch_bounds__(kThreads) void attn_prologue_kernel(PrologueArgs a) {
  const int64_t grp = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 4;
  const int ln = threadIdx.x & 15;
  const bool valid = grp < a.rows;   // uniform over the 16 lanes of a group
  const int heads = a.hq + a.hkv;
  const int64_t row = valid ? grp : 0;
  const int64_t t = static_cast<int>(row) / heads;  // rows < 2^31 (checked by the host)
  const int hh = static_cast<int>(row - t * heads);
  const bool isq = hh < a.hq;
  const uint16_t* src = isq ? a.q_in + t * a.q_ts + hh * a.q_hs : a.k_in + t * a.k_ts + (hh - a.hq) * a.k_hs;
  const uint4 raw = *reinterpret_cast<const uint4*>(src + ln * 8);
  // The gains and the rotary tables do not depend on the row's values: their
  // loads go out with the row's, so the norm waits for one round of latency.
  const bool rot_lane = a.rot > 0 && ln < (a.rot >> 3);
  uint4 cr = make_uint4(0u, 0u, 0u, 0u), sr = cr;
  if (rot_lane) {
    cr = *reinterpret_cast<const uint4*>(a.cos + t * a.rot + ln * 8);
    sr = *reinterpret_cast<const uint4*>(a.sin + t * a.rot + ln * 8);
  }
  // Both gain vectors are loaded and the lane's is selected by value: a per-lane
  // choice of pointer would become the address of a kernel-argument field and
  // cost a dependent load round trip.
  uint4 gr0 = make_uint4(0u, 0u, 0u, 0u), gr1 = gr0;
  if (a.w_vec) {
    const int gstep = a.w_f32 ? 32 : 16;  // bytes of 8 gains
    const unsigned char* qw = static_cast<const unsigned char*>(a.q_w) + ln * gstep;
    const unsigned char* kw = static_cast<const unsigned char*>(a.k_w) + ln * gstep;
    const uint4 q0 = *reinterpret_cast<const uint4*>(qw), k0 = *reinterpret_cast<const uint4*>(kw);
    gr0 = isq ? q0 : k0;
    if (a.w_f32) {
      const uint4 q1 = *reinterpret_cast<const uint4*>(qw + 16), k1 = *reinterpret_cast<const uint4*>(kw + 16);
      gr1 = isq ? q1 : k1;
    }
  }
  const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = fd_lo(wd[i]);
    x[2 * i + 1] = fd_hi(wd[i]);
  }
  // PyTorch's order for a row mean of width 128: 32 slots of 4 features, each
  // ((x0^2 + x1^2) + x2^2) + x3^2, then a pairwise tree over the slots; a lane
  // holds slots 2 ln and 2 ln + 1, so the tree's first level is inside the lane
  float sa = x[0] * x[0], sb = x[4] * x[4];
#pragma unroll
  for (int e = 1; e < 4; ++e) {
    sa = sa + x[e] * x[e];
    sb = sb + x[4 + e] * x[4 + e];
  }
  float s = sa + sb;
  s = fd_xor_sum_up<16>(s);
  // 1 / sqrt in fp64 (root and quotient), rounded to fp32: torch.rsqrt's value on every input measured
  const float inv =
      static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(s * (1.0f / static_cast<float>(kD)) + a.eps)));
  float gw[8];
  if (a.w_vec) {
    if (a.w_f32) {
      gw[0] = __uint_as_float(gr0.x); gw[1] = __uint_as_float(gr0.y);
      gw[2] = __uint_as_float(gr0.z); gw[3] = __uint_as_float(gr0.w);
      gw[4] = __uint_as_float(gr1.x); gw[5] = __uint_as_float(gr1.y);
      gw[6] = __uint_as_float(gr1.z); gw[7] = __uint_as_float(gr1.w);
    } else {
      const uint32_t gd[4] = {gr0.x, gr0.y, gr0.z, gr0.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        gw[2 * i] = fd_lo(gd[i]);
        gw[2 * i + 1] = fd_hi(gd[i]);
      }
    }
  } else {
    const void* w = isq ? a.q_w : a.k_w;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      gw[e] = a.w_f32 ? static_cast<const float*>(w)[ln * 8 + e]
                      : fd_bf16_to_f32(static_cast<const uint16_t*>(w)[ln * 8 + e]);
  }
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = a.gain_offset ? 1.0f + gw[e] : gw[e];
    y[e] = bf16r((x[e] * inv) * g);
  }
  if (a.rot > 0) {
    // partner lane holds the other half of the rotated features (rot/16 lanes apart)
    const int half_lanes = a.rot >> 4;  // 1, 2, 4 or 8: inside the 16-lane row, on DPP
    float p[8];
    auto partners = [&](auto mc) {
      constexpr int kM = decltype(mc)::value;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float own;
        fd_xor_pair<kM>(y[e], own, p[e]);
      }
    };
    if (half_lanes == 1)
      partners(std::integral_constant<int, 1>{});
    else if (half_lanes == 2)
      partners(std::integral_constant<int, 2>{});
    else if (half_lanes == 4)
      partners(std::integral_constant<int, 4>{});
    else
      partners(std::integral_constant<int, 8>{});
    if (rot_lane) {
      const bool first_half = ln < half_lanes;
      const uint32_t cw[4] = {cr.x, cr.y, cr.z, cr.w};
      const uint32_t sw[4] = {sr.x, sr.y, sr.z, sr.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = (e & 1) ? fd_hi(cw[e >> 1]) : fd_lo(cw[e >> 1]);
        const float sn = (e & 1) ? fd_hi(sw[e >> 1]) : fd_lo(sw[e >> 1]);
        const float rot = first_half ? -p[e] : p[e];
        y[e] = bf16r(bf16r(y[e] * c) + bf16r(rot * sn));
      }
    }
  }
  if (valid) {
    uint16_t* dst = isq ? a.q_out + (t * a.hq + hh) * kD : a.k_out + (t * a.hkv + (hh - a.hq)) * kD;
    uint4 out;
    out.x = fd_pack2(y[0], y[1]);
    out.y = fd_pack2(y[2], y[3]);
    out.z = fd_pack2(y[4], y[5]);
    out.w = fd_pack2(y[6], y[7]);
    *reinterpret_cast<uint4*>(dst + ln * 8) = out;
  }
}

}  // namespace

extern "C" FD_API int fd_attn_prologue_fwd(const void* q_in, int64_t q_token_stride, int64_t q_head_stride,
                                           const void* k_in, int64_t k_token_stride, int64_t k_head_stride,
                                           const void* q_weight, const void* k_weight, int weight_dtype,
                                           int gain_offset, float eps, const void* cos, const void* sin,
                                           int rotary_dim, void* q_out, void* k_out, int64_t tokens, int q_heads,
                                           int kv_heads, int head_dim, void* stream) {
  FD_REQUIRE(q_in && k_in && q_weight && k_weight && q_out && k_out, FD_ERR_INVALID_ARGUMENT,
             "fd_attn_prologue_fwd: tensor pointers must be non-null");
  FD_REQUIRE(head_dim == kD, FD_ERR_UNSUPPORTED, "fd_attn_prologue_fwd: head_dim must be 128 (got %d)", head_dim);
  FD_REQUIRE(tokens >= 0 && q_heads >= 1 && kv_heads >= 1, FD_ERR_INVALID_ARGUMENT,
             "fd_attn_prologue_fwd: tokens >= 0 and at least one q and one kv head");
  FD_REQUIRE(rotary_dim == 0 || rotary_dim == 16 || rotary_dim == 32 || rotary_dim == 64 || rotary_dim == 128,
             FD_ERR_UNSUPPORTED, "fd_attn_prologue_fwd: rotary_dim must be 0, 16, 32, 64 or 128 (got %d)",
             rotary_dim);
  FD_REQUIRE(rotary_dim == 0 || (cos && sin), FD_ERR_INVALID_ARGUMENT,
             "fd_attn_prologue_fwd: cos and sin are required when rotary_dim > 0");
  FD_REQUIRE(rotary_dim == 0 || (fd_aligned16(cos) && fd_aligned16(sin)), FD_ERR_ALIGNMENT,
             "fd_attn_prologue_fwd: cos and sin must be 16-byte aligned");
  FD_REQUIRE(weight_dtype == FD_DTYPE_BF16 || weight_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_attn_prologue_fwd: weight_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  FD_REQUIRE(eps >= 0.0f, FD_ERR_INVALID_ARGUMENT, "fd_attn_prologue_fwd: eps must be >= 0");
  FD_REQUIRE(fd_aligned16(q_in) && fd_aligned16(k_in) && fd_aligned16(q_out) && fd_aligned16(k_out) &&
                 q_token_stride % 8 == 0 && q_head_stride % 8 == 0 && k_token_stride % 8 == 0 &&
                 k_head_stride % 8 == 0,
             FD_ERR_ALIGNMENT, "fd_attn_prologue_fwd: inputs, outputs and strides must keep 16-byte alignment");
  const int64_t rows = tokens * (q_heads + kv_heads);
  if (rows == 0) return FD_OK;
  const int64_t blocks = (rows * 16 + kThreads - 1) / kThreads;
  FD_REQUIRE(blocks < (1LL << 31) && rows < (1LL << 31), FD_ERR_INVALID_ARGUMENT,
             "fd_attn_prologue_fwd: problem too large");
  PrologueArgs a;
  a.q_in = static_cast<const uint16_t*>(q_in);
  a.k_in = static_cast<const uint16_t*>(k_in);
  a.q_ts = q_token_stride;
  a.q_hs = q_head_stride;
  a.k_ts = k_token_stride;
  a.k_hs = k_head_stride;
  a.q_w = q_weight;
  a.k_w = k_weight;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_out = static_cast<uint16_t*>(k_out);
  a.rows = rows;
  a.hq = q_heads;
  a.hkv = kv_heads;
  a.rot = rotary_dim;
  a.w_f32 = weight_dtype == FD_DTYPE_F32;
  a.gain_offset = gain_offset != 0;
  a.w_vec = fd_aligned16(q_weight) && fd_aligned16(k_weight);
  a.eps = eps;
  hipLaunchKernelGGL(attn_prologue_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return fd_check_launch("fd_attn_prologue_fwd");
}

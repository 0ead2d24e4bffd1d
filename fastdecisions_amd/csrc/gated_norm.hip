// Gated RMSNorm of the Gated-DeltaNet layers and the MLP's SiLU gate, for gfx950.
//
// fd_gated_rmsnorm_fwd replaces transformers' Qwen3_5RMSNormGated applied to the
// delta rule's output (the call after ref: src/decider/packed_conv.py:55-59:
// ``self.norm(core_attn_out, z)``), evaluated exactly as the eager ops round:
//   y  = bf16(x * (1 / sqrt(mean(x^2) + eps)))      (x.to(input dtype))
//   y2 = bf16(w * y)                                (bf16 weight times bf16 row)
//   out = bf16(y2 * silu(z)),  silu(z) = z / (1 + exp(-z)) in fp32 on the bf16 gate
// (with an fp32 weight the product w * y stays fp32, as the eager promotion does).
// With a bf16 weight the last product runs on the hardware exp2 and reciprocal
// (fd_gated_silu_bf16: the exact expression where the bf16 rounding could
// differ; fd_gated_silu_check verifies every (y2, z) pair of bf16 values).
// A 16-lane group owns one row of 128 (8 features per lane, 16-byte accesses);
// rows of 64 or 256 use 8 or 32 lanes.  The mean of squares sums in the order
// PyTorch's GPU row mean uses for these widths (slots of 4 features, each
// summed in feature order, then a pairwise tree over the slots) and the inverse
// root is evaluated in fp64, so at widths 64, 128 and 256 the rows equal eager
// Qwen3_5RMSNormGated bit for bit.
//
// fd_silu_mul_fwd replaces the MLP's ``act_fn(gate_proj(x)) * up_proj(x)``
// (transformers Qwen3_5MLP) on a combined [rows, 2*width] gate|up projection:
//   out = bf16(bf16(silu(gate)) * up)
// with bf16(silu(gate)) from fd_silu_bf16 (the hardware exp2 and reciprocal,
// the exact expression near bf16 ties; the same bf16 for every fp32 input).
// HBM-bound, 16-byte loads and stores, one thread per 8 features.
// fd_silu_mul_split_fwd does the same when the features come from two
// gate|up projections (features [0, width1) from the first, the rest from the
// second), writing one [rows, width1 + width2] output.
#include "fd_common.h"

namespace {

constexpr int kThreads = 256;

// round to bf16 and back (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ float bf16r(float x) { return fd_lo(fd_pack2(x, 0.0f)); }

__device__ __forceinline__ void unpack8(uint4 raw, float* x) {
  const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = fd_lo(wd[i]);
    x[2 * i + 1] = fd_hi(wd[i]);
  }
}

__device__ __forceinline__ uint4 pack8(const float* x) {
  return make_uint4(fd_pack2(x[0], x[1]), fd_pack2(x[2], x[3]), fd_pack2(x[4], x[5]), fd_pack2(x[6], x[7]));
}

// LANES lanes per row (LANES * 8 == width); W_VEC: the weight is 16-byte aligned
// and a lane loads its 8 weights as vectors.  The weights are loaded before the
// per-element work: loaded inside it, each waited out its own memory round trip
// between the exact-SiLU branches.
template <int LANES, bool W_F32, bool W_VEC>
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ z, int64_t z_ts,
                                                                 int64_t z_hs, int heads,
                                                                 const void* __restrict__ w,
                                                                 uint16_t* __restrict__ out, int64_t rows,
                                                                 float eps) {
  constexpr int kWidth = LANES * 8;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / LANES;
  const int ln = threadIdx.x % LANES;
  const bool valid = row < rows;  // uniform over the lanes of a row
  const int64_t r = valid ? row : 0;
  float xv[8], zv[8];
  unpack8(*reinterpret_cast<const uint4*>(x + r * kWidth + ln * 8), xv);
  const int tok = static_cast<int>(r) / heads;  // rows < 2^31 (checked by the host)
  const int hd = static_cast<int>(r) - tok * heads;
  unpack8(*reinterpret_cast<const uint4*>(z + tok * z_ts + hd * z_hs + ln * 8), zv);
  float wv[8];
  if constexpr (W_VEC && W_F32) {
    const float4 w0 = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + ln * 8);
    const float4 w1 = *reinterpret_cast<const float4*>(static_cast<const float*>(w) + ln * 8 + 4);
    wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
    wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
  } else if constexpr (W_VEC) {
    unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + ln * 8), wv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      wv[e] = W_F32 ? static_cast<const float*>(w)[ln * 8 + e]
                    : fd_bf16_to_f32(static_cast<const uint16_t*>(w)[ln * 8 + e]);
  }
  // PyTorch's order for a row mean of this width: width/4 slots of 4 features,
  // each ((x0^2 + x1^2) + x2^2) + x3^2, then a pairwise tree over the slots; a
  // lane holds slots 2 ln and 2 ln + 1, so the tree's first level is inside it
  float sa = xv[0] * xv[0], sb = xv[4] * xv[4];
#pragma unroll
  for (int e = 1; e < 4; ++e) {
    sa = sa + xv[e] * xv[e];
    sb = sb + xv[4 + e] * xv[4 + e];
  }
  float s = sa + sb;
  s = fd_xor_sum_up<LANES>(s);
  // 1 / sqrt in fp64 (root and quotient), rounded to fp32: torch.rsqrt's value on every input measured
  const float inv = static_cast<float>(
      1.0 / __builtin_sqrt(static_cast<double>(s * (1.0f / static_cast<float>(kWidth)) + eps)));
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float yn = bf16r(xv[e] * inv);
    float g;
    if constexpr (W_F32) {
      g = wv[e] * yn;
    } else {
      g = bf16r(wv[e] * yn);
    }
    if constexpr (W_F32) {
      const float act = zv[e] / (1.0f + expf(-zv[e]));
      y[e] = g * act;
    } else {
      y[e] = fd_gated_silu_bf16(g, zv[e]);  // g is a bf16 value
    }
  }
  if (valid) *reinterpret_cast<uint4*>(out + r * kWidth + ln * 8) = pack8(y);
}

// one 8-feature piece per thread; blockIdx.y is the row, so no index division.
// Output features [0, w1) come from gu1 (gate at column f, up at w1 + f), the
// rest from gu2 (gate at f - w1, up at w2 + f - w1).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ gu1, int64_t stride1, int w1,
                                                            const uint16_t* __restrict__ gu2, int64_t stride2, int w2,
                                                            uint16_t* __restrict__ out) {
  const int c = blockIdx.x * kThreads + threadIdx.x;  // piece within the row
  const int width = w1 + w2;
  if (c * 8 >= width) return;
  const int64_t r = blockIdx.y;
  const bool first = c * 8 < w1;
  const uint16_t* src = first ? gu1 + r * stride1 + c * 8 : gu2 + r * stride2 + (c * 8 - w1);
  const int up = first ? w1 : w2;
  float g[8], u[8], s[8], y[8];
  unpack8(*reinterpret_cast<const uint4*>(src), g);
  unpack8(*reinterpret_cast<const uint4*>(src + up), u);
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = fd_silu_bf16(g[e]);  // rounds to bf16 as g / (1 + expf(-g)) does
  unpack8(pack8(s), s);  // act_fn's bf16 output
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = s[e] * u[e];
  *reinterpret_cast<uint4*>(out + r * width + c * 8) = pack8(y);
}

// bf16(fd_gated_silu_bf16(g, z)) against bf16(g * fd_silu(z)) for the pairs
// (g, z) = (bf16 bits i >> 16, bf16 bits i & 0xffff), i in [begin, begin + count);
// both NaN counts as equal.  One atomic per wavefront.
__global__ __launch_bounds__(256) void gated_silu_check_kernel(uint32_t begin, uint32_t count,
                                                               unsigned long long* mismatches) {
  unsigned n = 0;
  // 64-bit index: a 32-bit one would wrap past 2^32 - stride and never reach count
  for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += gridDim.x * 256ull) {
    const uint32_t bits = begin + static_cast<uint32_t>(i);
    const float g = __uint_as_float(bits & 0xffff0000u);
    const float z = __uint_as_float(bits << 16);
    const uint32_t a = fd_pack2(fd_gated_silu_bf16(g, z), 0.0f) & 0xffffu;
    const uint32_t b = fd_pack2(g * fd_silu(z), 0.0f) & 0xffffu;
    const bool a_nan = (a & 0x7f80u) == 0x7f80u && (a & 0x7fu) != 0;
    const bool b_nan = (b & 0x7f80u) == 0x7f80u && (b & 0x7fu) != 0;
    if (a != b && !(a_nan && b_nan)) ++n;
  }
  for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off, 64);
  if ((threadIdx.x & 63) == 0 && n != 0) atomicAdd(mismatches, static_cast<unsigned long long>(n));
}

}  // namespace

extern "C" FD_API int fd_gated_silu_check(uint32_t begin, uint32_t count, unsigned long long* mismatches,
                                          void* stream) {
  FD_REQUIRE(mismatches != nullptr, FD_ERR_INVALID_ARGUMENT, "fd_gated_silu_check: mismatches must be non-null");
  FD_REQUIRE(static_cast<uint64_t>(begin) + count <= (1ULL << 32), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_silu_check: [begin, begin + count) must lie within the 2^32 (g, z) bf16 pairs");
  if (count == 0) return FD_OK;
  hipLaunchKernelGGL(gated_silu_check_kernel, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream), begin,
                     count, mismatches);
  return fd_check_launch("fd_gated_silu_check");
}

extern "C" FD_API int fd_gated_rmsnorm_fwd(const void* x, const void* gate, int64_t gate_token_stride,
                                           int64_t gate_head_stride, int heads, const void* weight, int weight_dtype,
                                           void* out, int64_t rows, int width, float eps, void* stream) {
  FD_REQUIRE(x && gate && weight && out, FD_ERR_INVALID_ARGUMENT, "fd_gated_rmsnorm_fwd: pointers must be non-null");
  FD_REQUIRE(width == 64 || width == 128 || width == 256, FD_ERR_UNSUPPORTED,
             "fd_gated_rmsnorm_fwd: width must be 64, 128 or 256 (got %d)", width);
  FD_REQUIRE(rows >= 0 && heads >= 1 && rows % heads == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_rmsnorm_fwd: rows must be a non-negative multiple of heads >= 1");
  FD_REQUIRE(gate_token_stride % 8 == 0 && gate_head_stride % 8 == 0 && gate_head_stride >= width &&
                 gate_token_stride >= static_cast<int64_t>(heads) * gate_head_stride,
             FD_ERR_ALIGNMENT, "fd_gated_rmsnorm_fwd: gate strides must be multiples of 8 covering [heads, width]");
  FD_REQUIRE(weight_dtype == FD_DTYPE_BF16 || weight_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_rmsnorm_fwd: weight_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  FD_REQUIRE(eps >= 0.0f, FD_ERR_INVALID_ARGUMENT, "fd_gated_rmsnorm_fwd: eps must be >= 0");
  FD_REQUIRE(fd_aligned16(x) && fd_aligned16(gate) && fd_aligned16(out), FD_ERR_ALIGNMENT,
             "fd_gated_rmsnorm_fwd: x, gate and out must be 16-byte aligned");
  if (rows == 0) return FD_OK;
  const int lanes = width / 8;
  const int64_t blocks = (rows * lanes + kThreads - 1) / kThreads;
  FD_REQUIRE(blocks < (1LL << 31) && rows < (1LL << 31), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_rmsnorm_fwd: problem too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* zp = static_cast<const uint16_t*>(gate);
  uint16_t* op = static_cast<uint16_t*>(out);
  const dim3 grid(static_cast<unsigned>(blocks));
  const bool wvec = fd_aligned16(weight);
#define FD_GN2(L, F, V)                                                                                       \
  hipLaunchKernelGGL((gated_rmsnorm_kernel<L, F, V>), grid, dim3(kThreads), 0, s, xp, zp, gate_token_stride,  \
                     gate_head_stride, heads, weight, op, rows, eps)
#define FD_GN(L)                                                                                              \
  do {                                                                                                        \
    if (weight_dtype == FD_DTYPE_F32) {                                                                       \
      if (wvec) FD_GN2(L, true, true); else FD_GN2(L, true, false);                                           \
    } else {                                                                                                  \
      if (wvec) FD_GN2(L, false, true); else FD_GN2(L, false, false);                                         \
    }                                                                                                         \
  } while (0)
  if (lanes == 8) FD_GN(8); else if (lanes == 16) FD_GN(16); else FD_GN(32);
#undef FD_GN
#undef FD_GN2
  return fd_check_launch("fd_gated_rmsnorm_fwd");
}

namespace {

int silu_mul_entry(const char* who, const void* gate_up1, int64_t row_stride1, int width1, const void* gate_up2,
                   int64_t row_stride2, int width2, void* out, int64_t rows, void* stream) {
  FD_REQUIRE(gate_up1 && out && (width2 == 0 || gate_up2), FD_ERR_INVALID_ARGUMENT,
             "%s: pointers must be non-null", who);
  FD_REQUIRE(rows >= 0 && width1 > 0 && width1 % 8 == 0 && row_stride1 >= 2LL * width1 && row_stride1 % 8 == 0,
             FD_ERR_INVALID_ARGUMENT,
             "%s: width a positive multiple of 8 and row_stride a multiple of 8 >= 2*width", who);
  FD_REQUIRE(width2 >= 0 && width2 % 8 == 0 && (width2 == 0 || (row_stride2 >= 2LL * width2 && row_stride2 % 8 == 0)),
             FD_ERR_INVALID_ARGUMENT,
             "%s: width2 a multiple of 8 >= 0 and row_stride2 a multiple of 8 >= 2*width2", who);
  FD_REQUIRE(fd_aligned16(gate_up1) && fd_aligned16(out) && (width2 == 0 || fd_aligned16(gate_up2)),
             FD_ERR_ALIGNMENT, "%s: gate_up and out must be 16-byte aligned", who);
  if (rows == 0) return FD_OK;
  const int64_t width = static_cast<int64_t>(width1) + width2;
  FD_REQUIRE(rows <= 65535 * 1024LL && width <= (1 << 28), FD_ERR_INVALID_ARGUMENT,
             "%s: problem too large", who);
  const int64_t pieces = width / 8;
  const unsigned bx = static_cast<unsigned>((pieces + kThreads - 1) / kThreads);
  const uint16_t* g1 = static_cast<const uint16_t*>(gate_up1);
  const uint16_t* g2 = static_cast<const uint16_t*>(gate_up2);
  // rows beyond the grid's y limit run in slabs of 65535
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const unsigned by = static_cast<unsigned>(rows - r0 < 65535 ? rows - r0 : 65535);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(bx, by), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       g1 + r0 * row_stride1, row_stride1, width1, width2 ? g2 + r0 * row_stride2 : g2, row_stride2,
                       width2, static_cast<uint16_t*>(out) + r0 * width);
  }
  return fd_check_launch(who);
}

}  // namespace

extern "C" FD_API int fd_silu_mul_fwd(const void* gate_up, int64_t row_stride, void* out, int64_t rows, int width,
                                      void* stream) {
  return silu_mul_entry("fd_silu_mul_fwd", gate_up, row_stride, width, nullptr, 0, 0, out, rows, stream);
}

extern "C" FD_API int fd_silu_mul_split_fwd(const void* gate_up1, int64_t row_stride1, int width1,
                                            const void* gate_up2, int64_t row_stride2, int width2, void* out,
                                            int64_t rows, void* stream) {
  return silu_mul_entry("fd_silu_mul_split_fwd", gate_up1, row_stride1, width1, gate_up2, row_stride2, width2, out,
                        rows, stream);
}

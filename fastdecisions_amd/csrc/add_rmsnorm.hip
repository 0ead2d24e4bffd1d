// Fused residual add + RMSNorm for gfx950.
//
// Replaces the reference's persistent Triton reduction
// (ref: src/decider/persistent_residual_rms_kernel.py:49-72) with corrected
// numerics: eps inside the rsqrt (ref: src/decider/residual_rms_baseline.py:75-78),
// the residual rounded to bf16 before it is normalised, and the updated
// residual emitted as a second output, as the eager decoder layer does
// (transformers Qwen3_5DecoderLayer residual add, Qwen3_5RMSNorm).
//
// HBM-bound: the row stays in registers between the reduction and the store,
// so x and residual are read from HBM exactly once.
//   - Widths that are a multiple of 1024: two wavefronts per row (a
//     128-thread workgroup), summing the squares in the order PyTorch's GPU
//     row reduction uses for such a width (x.float().pow(2).mean(-1)): lane l
//     owns the 4-feature groups at 256 k + 4 l (k = 0 .. width/256 - 1), one
//     accumulator per position in the group summed over k in order, then
//     ((a0 + a1) + a2) + a3, then a pairwise tree over the 64 lanes (xor
//     butterfly with offsets 1, 2, .., 32).  Wavefront 0 holds the first half
//     of the k and hands its accumulators to wavefront 1 through LDS.  Each
//     wavefront load reads 512 B contiguous.  With the inverse square root
//     rounded as torch.rsqrt rounds it, the normed output equals eager
//     Qwen3_5RMSNorm bit for bit at the decider's [2048, 2048] and config 3's
//     [8192, 2048] (PyTorch picks this reduction for a few hundred rows and
//     more; very short inputs may reduce otherwise).
//   - Other widths: one wavefront per row, lane l owns the 8-feature chunks
//     l, l+64, l+128, ...; the sum in chunk order per lane, then an xor
//     butterfly with offsets 32, 16, .., 1 (no LDS, no barrier).
//
// fp32 sequence (the CPU restatement reproduces it bit for bit):
//   h_i    = bf16(f32(x_i) + f32(r_i))
//   s      = the sum of h_i * h_i in the order above (each product and sum rounded)
//   inv    = fp32(1 / sqrt(s * fl(1 / width) + eps)), the root and quotient in fp64
//   out_i  = bf16((h_i * inv) * g_i),  g_i = 1 + w_i  or  w_i
#include "fd_common.h"

namespace {

constexpr int kRowsPerBlock = 4;  // one row per wavefront, 256 threads

// 1 / sqrt(v) evaluated in fp64 (IEEE root and quotient, together within
// 2^-52 relative of the exact value) and rounded to fp32.  It equals
// torch.rsqrt on this platform on every input measured (4M fp32 values; the
// hardware v_rsq_f32 differs on 11 % of them, 1 / sqrtf, which rounds twice in
// fp32, on 28 %).  Once per row, so the fp64 work costs nothing.
__device__ __forceinline__ float inv_rms(float v) {
  return static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(v)));
}

template <typename WT>
__device__ __forceinline__ void load_gain8(const WT* w, int chunk, int gain_offset, float g[8]);

template <>
__device__ __forceinline__ void load_gain8<uint16_t>(const uint16_t* w, int chunk, int gain_offset,
                                                     float g[8]) {
  uint4 raw = *reinterpret_cast<const uint4*>(w + chunk * 8);
  uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    g[2 * i] = fd_lo(wd[i]);
    g[2 * i + 1] = fd_hi(wd[i]);
  }
  if (gain_offset) {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = 1.0f + g[e];
  }
}

template <>
__device__ __forceinline__ void load_gain8<float>(const float* w, int chunk, int gain_offset, float g[8]) {
  float4 a = *reinterpret_cast<const float4*>(w + chunk * 8);
  float4 b = *reinterpret_cast<const float4*>(w + chunk * 8 + 4);
  g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
  g[4] = b.x; g[5] = b.y; g[6] = b.z; g[7] = b.w;
  if (gain_offset) {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = 1.0f + g[e];
  }
}

// NCH = chunks of 8 features per lane (width <= 512 * NCH).  One row per
// wavefront, for widths that are not a multiple of 1024.  (At [2048, 2048],
// which now runs two wavefronts per row, two or four rows per wavefront -- the
// loads of all rows first, the rows finished in turn -- measured 20 % and 54 %
// slower than one row per wavefront, for fewer wavefronts in flight.)
template <int NCH, typename WT, bool HAS_RES>
__global__ __launch_bounds__(64 * kRowsPerBlock) void add_rmsnorm_kernel(
    const uint16_t* x, const uint16_t* res, const WT* __restrict__ w,
    uint16_t* out, uint16_t* res_out, int64_t rows, int width, float eps, int gain_offset) {
  const int lane = threadIdx.x & 63;
  constexpr int RPW = 1;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row0 >= rows) return;  // whole wavefront exits together
  const int nchunks = width >> 3;

  // Every load of the rows is issued before any store: residual_out may alias
  // residual, so a store between two loads would make the compiler wait for
  // each load round in turn.
  uint4 xv[RPW][NCH], rv[RPW][NCH];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int64_t base = (row0 + rr) * width;
    const bool live = row0 + rr < rows;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int chunk = lane + 64 * i;
      xv[rr][i] = make_uint4(0u, 0u, 0u, 0u);
      rv[rr][i] = xv[rr][i];
      if (live && chunk < nchunks) {
        xv[rr][i] = *reinterpret_cast<const uint4*>(x + base + chunk * 8);
        if (HAS_RES) rv[rr][i] = *reinterpret_cast<const uint4*>(res + base + chunk * 8);
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    if (row0 + rr >= rows) break;
    const int64_t base = (row0 + rr) * width;
    float h[NCH][8];
    uint32_t hw[NCH][4];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const uint32_t xw[4] = {xv[rr][i].x, xv[rr][i].y, xv[rr][i].z, xv[rr][i].w};
      if (HAS_RES) {
        const uint32_t rw[4] = {rv[rr][i].x, rv[rr][i].y, rv[rr][i].z, rv[rr][i].w};
#pragma unroll
        for (int p = 0; p < 4; ++p)
          hw[i][p] = fd_pack2(fd_lo(xw[p]) + fd_lo(rw[p]), fd_hi(xw[p]) + fd_hi(rw[p]));
      } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) hw[i][p] = xw[p];
      }
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        h[i][2 * p] = fd_lo(hw[i][p]);
        h[i][2 * p + 1] = fd_hi(hw[i][p]);
      }
      // chunks past the row end hold zeros: they add +0 to the sum of squares
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sq = h[i][e] * h[i][e];
        s = s + sq;
      }
    }
    if (HAS_RES && res_out != nullptr) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int chunk = lane + 64 * i;
        if (chunk < nchunks)
          *reinterpret_cast<uint4*>(res_out + base + chunk * 8) =
              make_uint4(hw[i][0], hw[i][1], hw[i][2], hw[i][3]);
      }
    }
    s = fd_xor_sum_down<64>(s);

    const float mean = s * (1.0f / static_cast<float>(width));
    const float inv = inv_rms(mean + eps);

#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int chunk = lane + 64 * i;
      if (chunk < nchunks) {
        float g[8];
        load_gain8<WT>(w, chunk, gain_offset, g);
        uint32_t o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          float a = (h[i][2 * p] * inv) * g[2 * p];
          float b = (h[i][2 * p + 1] * inv) * g[2 * p + 1];
          o[p] = fd_pack2(a, b);
        }
        *reinterpret_cast<uint4*>(out + base + chunk * 8) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// Two wavefronts per row (width == 1024 * CPL), one row per 128-thread
// workgroup, summing the squares in PyTorch's order for a row reduction of
// this width: lane l owns the 4-feature groups 256 k + 4 l .. +3 (k = 0 .. K-1,
// K = width / 256), with one accumulator per group position summed over k in
// order, then ((a0 + a1) + a2) + a3, then a pairwise tree over the 64 lanes.
// Wavefront 0 holds k < K/2 and hands its accumulators to wavefront 1, which
// continues with the rest.
template <typename WT>
__device__ __forceinline__ void load_gain4(const WT* w, int f, int gain_offset, float g[4]);

template <>
__device__ __forceinline__ void load_gain4<uint16_t>(const uint16_t* w, int f, int gain_offset, float g[4]) {
  const uint2 raw = *reinterpret_cast<const uint2*>(w + f);
  g[0] = fd_lo(raw.x); g[1] = fd_hi(raw.x); g[2] = fd_lo(raw.y); g[3] = fd_hi(raw.y);
  if (gain_offset) {
#pragma unroll
    for (int e = 0; e < 4; ++e) g[e] = 1.0f + g[e];
  }
}

template <>
__device__ __forceinline__ void load_gain4<float>(const float* w, int f, int gain_offset, float g[4]) {
  const float4 a = *reinterpret_cast<const float4*>(w + f);
  g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
  if (gain_offset) {
#pragma unroll
    for (int e = 0; e < 4; ++e) g[e] = 1.0f + g[e];
  }
}

template <int CPL, typename WT, bool HAS_RES>
__global__ __launch_bounds__(128) void add_rmsnorm_pair_kernel(
    const uint16_t* x, const uint16_t* res, const WT* __restrict__ w,
    uint16_t* out, uint16_t* res_out, int width, float eps, int gain_offset) {
  constexpr int KH = 2 * CPL;  // 4-feature groups per lane of each wavefront
  __shared__ float part[4 * 64];
  __shared__ float inv_s;
  const int lane = threadIdx.x & 63;
  const int q = threadIdx.x >> 6;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * width;
  // every load before any store (residual_out may alias residual)
  uint2 xv[KH], rv[KH];
#pragma unroll
  for (int j = 0; j < KH; ++j) {
    const int f = 256 * (q * KH + j) + 4 * lane;
    xv[j] = *reinterpret_cast<const uint2*>(x + base + f);
    rv[j] = make_uint2(0u, 0u);
    if (HAS_RES) rv[j] = *reinterpret_cast<const uint2*>(res + base + f);
  }
  uint32_t hw[KH][2];
  float h[KH][4];
#pragma unroll
  for (int j = 0; j < KH; ++j) {
    const uint32_t xw[2] = {xv[j].x, xv[j].y};
    const uint32_t rw[2] = {rv[j].x, rv[j].y};
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      hw[j][p] = HAS_RES ? fd_pack2(fd_lo(xw[p]) + fd_lo(rw[p]), fd_hi(xw[p]) + fd_hi(rw[p])) : xw[p];
      h[j][2 * p] = fd_lo(hw[j][p]);
      h[j][2 * p + 1] = fd_hi(hw[j][p]);
    }
  }
  if (HAS_RES && res_out != nullptr) {
#pragma unroll
    for (int j = 0; j < KH; ++j)
      *reinterpret_cast<uint2*>(res_out + base + 256 * (q * KH + j) + 4 * lane) = make_uint2(hw[j][0], hw[j][1]);
  }
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (q == 0) {
#pragma unroll
    for (int j = 0; j < KH; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + h[j][i] * h[j][i];
#pragma unroll
    for (int i = 0; i < 4; ++i) part[i * 64 + lane] = acc[i];
  }
  __syncthreads();
  if (q == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = part[i * 64 + lane];
#pragma unroll
    for (int j = 0; j < KH; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + h[j][i] * h[j][i];
    float s = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    s = fd_xor_sum_up<64>(s);
    const float mean = s * (1.0f / static_cast<float>(width));  // PyTorch's mean: the sum times fl(1 / width)
    const float inv = inv_rms(mean + eps);
    if (lane == 0) inv_s = inv;
  }
  __syncthreads();
  const float inv = inv_s;
#pragma unroll
  for (int j = 0; j < KH; ++j) {
    const int f = 256 * (q * KH + j) + 4 * lane;
    float g[4];
    load_gain4<WT>(w, f, gain_offset, g);
    const float a0 = (h[j][0] * inv) * g[0], a1 = (h[j][1] * inv) * g[1];
    const float a2 = (h[j][2] * inv) * g[2], a3 = (h[j][3] * inv) * g[3];
    *reinterpret_cast<uint2*>(out + base + f) = make_uint2(fd_pack2(a0, a1), fd_pack2(a2, a3));
  }
}

template <int CPL, typename WT>
int launch_pair(const void* x, const void* res, const void* w, void* out, void* res_out, int64_t rows,
                int width, float eps, int gain_offset, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(rows)), block(128);
  if (res != nullptr) {
    hipLaunchKernelGGL((add_rmsnorm_pair_kernel<CPL, WT, true>), grid, block, 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res),
                       static_cast<const WT*>(w), static_cast<uint16_t*>(out), static_cast<uint16_t*>(res_out),
                       width, eps, gain_offset);
  } else {
    hipLaunchKernelGGL((add_rmsnorm_pair_kernel<CPL, WT, false>), grid, block, 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(nullptr),
                       static_cast<const WT*>(w), static_cast<uint16_t*>(out), static_cast<uint16_t*>(nullptr),
                       width, eps, gain_offset);
  }
  return fd_check_launch("fd_add_rmsnorm_fwd");
}

template <int NCH, typename WT>
int launch_nch(const void* x, const void* res, const void* w, void* out, void* res_out, int64_t rows,
               int width, float eps, int gain_offset, hipStream_t stream) {
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  dim3 grid(static_cast<unsigned>(blocks)), block(64 * kRowsPerBlock);
  if (res != nullptr) {
    hipLaunchKernelGGL((add_rmsnorm_kernel<NCH, WT, true>), grid, block, 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(res),
                       static_cast<const WT*>(w), static_cast<uint16_t*>(out), static_cast<uint16_t*>(res_out),
                       rows, width, eps, gain_offset);
  } else {
    hipLaunchKernelGGL((add_rmsnorm_kernel<NCH, WT, false>), grid, block, 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(nullptr),
                       static_cast<const WT*>(w), static_cast<uint16_t*>(out), static_cast<uint16_t*>(nullptr),
                       rows, width, eps, gain_offset);
  }
  return fd_check_launch("fd_add_rmsnorm_fwd");
}

template <typename WT>
int launch_wt(const void* x, const void* res, const void* w, void* out, void* res_out, int64_t rows,
              int width, float eps, int gain_offset, hipStream_t stream) {
  if (width % 1024 == 0 && rows < 2147483647LL) {
    switch (width / 1024) {
      case 1: return launch_pair<1, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 2: return launch_pair<2, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 3: return launch_pair<3, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 4: return launch_pair<4, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 5: return launch_pair<5, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 6: return launch_pair<6, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      case 7: return launch_pair<7, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
      default: return launch_pair<8, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
    }
  }
  const int nch = (width / 8 + 63) / 64;
  if (nch <= 1) return launch_nch<1, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
  if (nch <= 2) return launch_nch<2, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
  if (nch <= 4) return launch_nch<4, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
  if (nch <= 8) return launch_nch<8, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
  return launch_nch<16, WT>(x, res, w, out, res_out, rows, width, eps, gain_offset, stream);
}

}  // namespace

extern "C" int fd_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight, void* out,
                                  void* residual_out, int64_t rows, int width, float eps, int weight_dtype,
                                  int gain_offset, void* stream) {
  FD_REQUIRE(x != nullptr && weight != nullptr && out != nullptr, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: x, weight and out must be non-null");
  FD_REQUIRE(rows >= 0, FD_ERR_INVALID_ARGUMENT, "fd_add_rmsnorm_fwd: rows must be >= 0 (got %lld)",
             static_cast<long long>(rows));
  FD_REQUIRE(width >= 8 && width <= 8192 && width % 8 == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: width must be a multiple of 8 in [8, 8192] (got %d)", width);
  FD_REQUIRE(weight_dtype == FD_DTYPE_BF16 || weight_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: weight_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32 (got %d)", weight_dtype);
  FD_REQUIRE(gain_offset == 0 || gain_offset == 1, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: gain_offset must be 0 or 1 (got %d)", gain_offset);
  FD_REQUIRE(!(eps < 0.0f) && eps == eps, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: eps must be a non-negative number");
  FD_REQUIRE(rows / 4 < 2147483647LL, FD_ERR_INVALID_ARGUMENT, "fd_add_rmsnorm_fwd: too many rows");
  FD_REQUIRE(fd_aligned16(x) && fd_aligned16(weight) && fd_aligned16(out) &&
                 (residual == nullptr || fd_aligned16(residual)) &&
                 (residual_out == nullptr || fd_aligned16(residual_out)),
             FD_ERR_ALIGNMENT, "fd_add_rmsnorm_fwd: every pointer must be 16-byte aligned");
  FD_REQUIRE(residual_out == nullptr || residual_out != out, FD_ERR_INVALID_ARGUMENT,
             "fd_add_rmsnorm_fwd: out and residual_out must be distinct buffers");
  if (rows == 0) return FD_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (weight_dtype == FD_DTYPE_BF16)
    return launch_wt<uint16_t>(x, residual, weight, out, residual_out, rows, width, eps, gain_offset, s);
  return launch_wt<float>(x, residual, weight, out, residual_out, rows, width, eps, gain_offset, s);
}

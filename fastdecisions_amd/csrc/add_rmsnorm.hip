// Fused residual add + RMSNorm for gfx950.
//
// Replaces the reference's persistent Triton reduction
// (ref: src/decider/persistent_residual_rms_kernel.py:49-72) with corrected
// numerics: eps inside the rsqrt (ref: src/decider/residual_rms_baseline.py:75-78),
// the residual rounded to bf16 before it is normalised, and the updated
// residual emitted as a second output, as the eager decoder layer does
// (transformers Qwen3_5DecoderLayer residual add, Qwen3_5RMSNorm).
//
// HBM-bound: each 16-byte chunk (8 bf16) of a row belongs to one lane, and
// each wavefront load instruction reads 1 KiB contiguous; the row stays in
// registers between the reduction and the store, so x and residual are read
// from HBM exactly once.
//   - Widths that are a multiple of 1024: two wavefronts per row (a
//     128-thread workgroup).  Wavefront q owns chunks (q * CPL + c) * 64 + lane,
//     c = 0 .. CPL - 1 (CPL = width / 1024).  At the decider's [2048, 2048]
//     call that is 4 wavefronts per SIMD instead of 2: the call went from
//     8.7 to 7.8 us (6.8 to 5.6 us with the inputs in L2), config 3
//     ([4, 2048, 2048]) from 23.5 to 22.4 us.
//   - Other widths: one wavefront per row, lane l owns chunks l, l+64, l+128, ...
//     (no LDS, no barrier).
//
// fp32 sequence (the CPU restatement reproduces it bit for bit):
//   h_i    = bf16(f32(x_i) + f32(r_i))
//   lane   : s = 0; for each owned chunk in order, for e = 0..7: s = s + h*h (two roundings)
//   wave   : for off = 32,16,8,4,2,1: s = s + shfl_xor(s, off)
//   row    : the wavefront's s, or with two wavefronts s(q = 0) + s(q = 1)
//   inv    = 1 / sqrt(s / width + eps)       (correctly rounded sqrt and division)
//   out_i  = bf16((h_i * inv) * g_i),  g_i = 1 + w_i  or  w_i
#include "fd_common.h"

namespace {

constexpr int kRowsPerBlock = 4;  // one row per wavefront, 256 threads

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
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, 64);

    // Plain '/' and __builtin_sqrtf are IEEE correctly rounded in HIP device code
    // (correctly rounded fp32 divide/sqrt is the HIP default).
    const float mean = s / static_cast<float>(width);
    const float inv = 1.0f / __builtin_sqrtf(mean + eps);

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
// workgroup; the order of the fp32 operations is the file header's.
template <int CPL, typename WT, bool HAS_RES>
__global__ __launch_bounds__(128) void add_rmsnorm_pair_kernel(
    const uint16_t* x, const uint16_t* res, const WT* __restrict__ w,
    uint16_t* out, uint16_t* res_out, int width, float eps, int gain_offset) {
  __shared__ float part[2];
  const int lane = threadIdx.x & 63;
  const int q = threadIdx.x >> 6;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * width;
  // every load before any store (residual_out may alias residual)
  uint4 xv[CPL], rv[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = (q * CPL + c) * 64 + lane;
    xv[c] = *reinterpret_cast<const uint4*>(x + base + chunk * 8);
    rv[c] = make_uint4(0u, 0u, 0u, 0u);
    if (HAS_RES) rv[c] = *reinterpret_cast<const uint4*>(res + base + chunk * 8);
  }
  uint32_t hw[CPL][4];
  float h[CPL][8];
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    const uint32_t rw[4] = {rv[c].x, rv[c].y, rv[c].z, rv[c].w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      hw[c][p] = HAS_RES ? fd_pack2(fd_lo(xw[p]) + fd_lo(rw[p]), fd_hi(xw[p]) + fd_hi(rw[p])) : xw[p];
      h[c][2 * p] = fd_lo(hw[c][p]);
      h[c][2 * p + 1] = fd_hi(hw[c][p]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float sq = h[c][e] * h[c][e];
      s = s + sq;
    }
  }
  if (HAS_RES && res_out != nullptr) {
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      *reinterpret_cast<uint4*>(res_out + base + ((q * CPL + c) * 64 + lane) * 8) =
          make_uint4(hw[c][0], hw[c][1], hw[c][2], hw[c][3]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, 64);
  if (lane == 0) part[q] = s;
  __syncthreads();
  const float mean = (part[0] + part[1]) / static_cast<float>(width);
  const float inv = 1.0f / __builtin_sqrtf(mean + eps);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = (q * CPL + c) * 64 + lane;
    float g[8];
    load_gain8<WT>(w, chunk, gain_offset, g);
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float a = (h[c][2 * p] * inv) * g[2 * p];
      float b = (h[c][2 * p + 1] * inv) * g[2 * p + 1];
      o[p] = fd_pack2(a, b);
    }
    *reinterpret_cast<uint4*>(out + base + chunk * 8) = make_uint4(o[0], o[1], o[2], o[3]);
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

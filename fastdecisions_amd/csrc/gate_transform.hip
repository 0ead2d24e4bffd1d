// Gate transform of the Gated-DeltaNet layers for gfx950: from the a / b gate
// projections to the delta rule's log decay g (fp32) and write strength beta (bf16).
//
// Replaces the reference's unpack_gate_transform kernel
// (ref: src/decider/unpack_gate_transform_kernel.py:51-91) and the eager
// expressions it stands for (ref: src/decider/packed_conv.py:49-53):
//   g    = -exp(A_log) * softplus(a + dt_bias),  softplus(x) = x > 20 ? x : log1p(exp(x))
//   beta = bf16(sigmoid(b)),                     sigmoid(x) = 1 / (1 + exp(-x))
// in fp32 with the same library exp / log1p as PyTorch's elementwise kernels,
// one thread per (token, head).  a and b may be two views of one combined
// projection output (row stride 2*heads), as the reference's combined gate
// projection produces (ref: src/decider/combined_gates.py:19-43).
#include "fd_common.h"

namespace {

constexpr int kThreads = 256;

template <typename PT>
__device__ __forceinline__ float load_param(const void* p, int i);
template <>
__device__ __forceinline__ float load_param<uint16_t>(const void* p, int i) {
  return fd_bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <>
__device__ __forceinline__ float load_param<float>(const void* p, int i) {
  return static_cast<const float*>(p)[i];
}

template <typename LT, typename BT>
__global__ __launch_bounds__(kThreads) void gate_transform_kernel(const uint16_t* __restrict__ a,
                                                                  const uint16_t* __restrict__ b, int64_t a_stride,
                                                                  int64_t b_stride, const void* a_log,
                                                                  const void* dt_bias, float* __restrict__ g,
                                                                  uint16_t* __restrict__ beta, int64_t n, int heads) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / heads;
  const int h = static_cast<int>(i - row * heads);
  const float x = fd_bf16_to_f32(a[row * a_stride + h]) + load_param<BT>(dt_bias, h);
  const float sp = x > 20.0f ? x : log1pf(expf(x));
  g[i] = -expf(load_param<LT>(a_log, h)) * sp;
  const float y = fd_bf16_to_f32(b[row * b_stride + h]);
  beta[i] = static_cast<uint16_t>(fd_f32_to_bf16(1.0f / (1.0f + expf(-y))));
}

// ---------------------------------------------------------------------------
// a|b projection fused with the transform (fd_gate_proj_fwd).
//
// One workgroup per 16 tokens, 8 wavefronts; wavefront wv accumulates the
// hidden-dimension part [wv*hidden/8, (wv+1)*hidden/8) of all 2*heads outputs
// on v_mfma_f32_16x16x32_bf16 (exact bf16 products, fp32 sums).  Lane l
// supplies A = x[row0 + l%16][k + 8(l/16) .. +7] and B = W[n0 + l%16][same k]
// (16-byte loads); D[4(l/16)+r][l%16] is (token, output).  The 8 partial sums
// are added in wavefront order through LDS and rounded to bf16, the value a
// bf16 GEMM (F.linear) stores, then transformed as gate_transform_kernel does.
constexpr int kProjRows = 16;
constexpr int kProjWaves = 8;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename LT, typename BT, int NB>
__global__ __launch_bounds__(64 * kProjWaves) void gate_proj_kernel(
    const uint16_t* __restrict__ x, int64_t xs, const uint16_t* __restrict__ w, int hidden, const void* a_log,
    const void* dt_bias, float* __restrict__ g, uint16_t* __restrict__ beta, uint16_t* __restrict__ ab,
    int64_t rows) {
  constexpr int heads = 8 * NB;  // 2 * heads = NB blocks of 16 outputs
  __shared__ float part[kProjWaves][NB * 16][kProjRows + 1];
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int l = tid & 63;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kProjRows;
  const int64_t xrow = min(row0 + (l & 15), rows - 1);  // rows past the end re-read the last one
  const int kq = hidden / kProjWaves;
  const uint16_t* xp = x + xrow * xs + wv * kq + 8 * (l >> 4);
  const uint16_t* wp = w + static_cast<int64_t>(l & 15) * hidden + wv * kq + 8 * (l >> 4);
  f32x4_t acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4_t{};
  for (int k = 0; k < kq; k += 128) {
    bf16x8_t av[4], bv[4][NB];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      av[s] = *reinterpret_cast<const bf16x8_t*>(xp + k + 32 * s);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bv[s][nb] = *reinterpret_cast<const bf16x8_t*>(wp + static_cast<int64_t>(16 * nb) * hidden + k + 32 * s);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[s], bv[s][nb], acc[nb], 0, 0, 0);
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wv][16 * nb + (l & 15)][4 * (l >> 4) + r] = acc[nb][r];
  __syncthreads();
  if (tid >= kProjRows * heads) return;
  const int rr = tid / heads;
  const int h = tid - rr * heads;
  const int64_t row = row0 + rr;
  if (row >= rows) return;
  float sa = part[0][h][rr];
  float sb = part[0][heads + h][rr];
#pragma unroll
  for (int p = 1; p < kProjWaves; ++p) {
    sa = sa + part[p][h][rr];
    sb = sb + part[p][heads + h][rr];
  }
  const uint32_t abits = fd_f32_to_bf16(sa);
  const uint32_t bbits = fd_f32_to_bf16(sb);
  if (ab != nullptr) {
    ab[row * 2 * heads + h] = static_cast<uint16_t>(abits);
    ab[row * 2 * heads + heads + h] = static_cast<uint16_t>(bbits);
  }
  const float xa = fd_bf16_to_f32(abits) + load_param<BT>(dt_bias, h);
  const float sp = xa > 20.0f ? xa : log1pf(expf(xa));
  g[row * heads + h] = -expf(load_param<LT>(a_log, h)) * sp;
  const float y = fd_bf16_to_f32(bbits);
  beta[row * heads + h] = static_cast<uint16_t>(fd_f32_to_bf16(1.0f / (1.0f + expf(-y))));
}

}  // namespace

extern "C" FD_API int fd_gate_proj_fwd(const void* x, int64_t x_row_stride, const void* weight, int hidden,
                                       const void* a_log, int a_log_dtype, const void* dt_bias, int dt_bias_dtype,
                                       float* g, void* beta, void* ab, int64_t rows, int heads, void* stream) {
  FD_REQUIRE(x && weight && a_log && dt_bias && g && beta, FD_ERR_INVALID_ARGUMENT,
             "fd_gate_proj_fwd: pointers must be non-null");
  FD_REQUIRE(rows >= 0, FD_ERR_INVALID_ARGUMENT, "fd_gate_proj_fwd: rows must be >= 0");
  FD_REQUIRE(heads == 8 || heads == 16 || heads == 24 || heads == 32, FD_ERR_UNSUPPORTED,
             "fd_gate_proj_fwd: heads must be 8, 16, 24 or 32 (got %d)", heads);
  FD_REQUIRE(hidden > 0 && hidden % (kProjWaves * 128) == 0, FD_ERR_UNSUPPORTED,
             "fd_gate_proj_fwd: hidden must be a positive multiple of %d (got %d)", kProjWaves * 128, hidden);
  FD_REQUIRE(x_row_stride >= hidden && x_row_stride % 8 == 0 && fd_aligned16(x) && fd_aligned16(weight),
             FD_ERR_ALIGNMENT, "fd_gate_proj_fwd: x rows and weight must be 16-byte aligned, row stride >= hidden");
  FD_REQUIRE((a_log_dtype == FD_DTYPE_BF16 || a_log_dtype == FD_DTYPE_F32) &&
                 (dt_bias_dtype == FD_DTYPE_BF16 || dt_bias_dtype == FD_DTYPE_F32),
             FD_ERR_INVALID_ARGUMENT, "fd_gate_proj_fwd: parameter dtypes must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  if (rows == 0) return FD_OK;
  const int64_t blocks = (rows + kProjRows - 1) / kProjRows;
  FD_REQUIRE(blocks < (1LL << 31), FD_ERR_INVALID_ARGUMENT, "fd_gate_proj_fwd: problem too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(weight);
  uint16_t* betap = static_cast<uint16_t*>(beta);
  uint16_t* abp = static_cast<uint16_t*>(ab);
#define FD_PROJ_LAUNCH(LT, BT, NB)                                                                           \
  hipLaunchKernelGGL((gate_proj_kernel<LT, BT, NB>), grid, dim3(64 * kProjWaves), 0, s, xp, x_row_stride, wp, \
                     hidden, a_log, dt_bias, g, betap, abp, rows)
#define FD_PROJ_HEADS(LT, BT)                 \
  switch (heads) {                            \
    case 8: FD_PROJ_LAUNCH(LT, BT, 1); break;  \
    case 16: FD_PROJ_LAUNCH(LT, BT, 2); break; \
    case 24: FD_PROJ_LAUNCH(LT, BT, 3); break; \
    default: FD_PROJ_LAUNCH(LT, BT, 4); break; \
  }
  if (a_log_dtype == FD_DTYPE_F32) {
    if (dt_bias_dtype == FD_DTYPE_F32) FD_PROJ_HEADS(float, float) else FD_PROJ_HEADS(float, uint16_t)
  } else {
    if (dt_bias_dtype == FD_DTYPE_F32) FD_PROJ_HEADS(uint16_t, float) else FD_PROJ_HEADS(uint16_t, uint16_t)
  }
#undef FD_PROJ_HEADS
#undef FD_PROJ_LAUNCH
  return fd_check_launch("fd_gate_proj_fwd");
}

extern "C" FD_API int fd_gate_transform_fwd(const void* a, const void* b, int64_t a_row_stride,
                                            int64_t b_row_stride, const void* a_log, int a_log_dtype,
                                            const void* dt_bias, int dt_bias_dtype, float* g, void* beta,
                                            int64_t rows, int heads, void* stream) {
  FD_REQUIRE(a && b && a_log && dt_bias && g && beta, FD_ERR_INVALID_ARGUMENT,
             "fd_gate_transform_fwd: pointers must be non-null");
  FD_REQUIRE(rows >= 0 && heads > 0, FD_ERR_INVALID_ARGUMENT, "fd_gate_transform_fwd: rows >= 0 and heads > 0");
  FD_REQUIRE(a_row_stride >= heads && b_row_stride >= heads, FD_ERR_INVALID_ARGUMENT,
             "fd_gate_transform_fwd: row strides must be >= heads");
  FD_REQUIRE((a_log_dtype == FD_DTYPE_BF16 || a_log_dtype == FD_DTYPE_F32) &&
                 (dt_bias_dtype == FD_DTYPE_BF16 || dt_bias_dtype == FD_DTYPE_F32),
             FD_ERR_INVALID_ARGUMENT, "fd_gate_transform_fwd: parameter dtypes must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  const int64_t n = rows * heads;
  if (n == 0) return FD_OK;
  FD_REQUIRE(n / kThreads < (1LL << 31), FD_ERR_INVALID_ARGUMENT, "fd_gate_transform_fwd: problem too large");
  const dim3 grid(static_cast<unsigned>((n + kThreads - 1) / kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* ap = static_cast<const uint16_t*>(a);
  const uint16_t* bp = static_cast<const uint16_t*>(b);
  uint16_t* betap = static_cast<uint16_t*>(beta);
#define FD_GATE_LAUNCH(LT, BT)                                                                              \
  hipLaunchKernelGGL((gate_transform_kernel<LT, BT>), grid, dim3(kThreads), 0, s, ap, bp, a_row_stride,      \
                     b_row_stride, a_log, dt_bias, g, betap, n, heads)
  if (a_log_dtype == FD_DTYPE_F32) {
    if (dt_bias_dtype == FD_DTYPE_F32) FD_GATE_LAUNCH(float, float); else FD_GATE_LAUNCH(float, uint16_t);
  } else {
    if (dt_bias_dtype == FD_DTYPE_F32) FD_GATE_LAUNCH(uint16_t, float); else FD_GATE_LAUNCH(uint16_t, uint16_t);
  }
#undef FD_GATE_LAUNCH
  return fd_check_launch("fd_gate_transform_fwd");
}

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
#include "gate_proj_body.h"

namespace {

constexpr int kThreads = 256;

using fd_gate::load_param;

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
// a|b projection fused with the transform (fd_gate_proj_fwd): one workgroup per
// 16 tokens, 8 wavefronts, one hidden-dimension part each (gate_proj_body.h).
template <typename LT, typename BT, int NB>
__global__ __launch_bounds__(64 * fd_gate::kProjParts) void gate_proj_kernel(fd_gate::GateProjArgs args) {
  __shared__ fd_gate::PartSmem<NB> part;
  fd_gate::gate_proj_rows<LT, BT, NB, fd_gate::kProjParts>(blockIdx.x, args, part);
}

}  // namespace

extern "C" FD_API int fd_gate_proj_fwd(const void* x, int64_t x_row_stride, const void* weight, int hidden,
                                       const void* a_log, int a_log_dtype, const void* dt_bias, int dt_bias_dtype,
                                       float* g, void* beta, void* ab, int64_t rows, int heads, void* stream) {
  const int rc = fd_gate::gate_proj_check("fd_gate_proj_fwd", x, x_row_stride, weight, hidden, a_log, a_log_dtype,
                                          dt_bias, dt_bias_dtype, g, beta, rows, heads);
  if (rc != FD_OK) return rc;
  if (rows == 0) return FD_OK;
  const dim3 grid(static_cast<unsigned>((rows + fd_gate::kProjRows - 1) / fd_gate::kProjRows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const fd_gate::GateProjArgs args{static_cast<const uint16_t*>(x), x_row_stride, static_cast<const uint16_t*>(weight),
                                   hidden, a_log, dt_bias, g, static_cast<uint16_t*>(beta),
                                   static_cast<uint16_t*>(ab), rows};
#define FD_PROJ_LAUNCH(LT, BT, NB) \
  hipLaunchKernelGGL((gate_proj_kernel<LT, BT, NB>), grid, dim3(64 * fd_gate::kProjParts), 0, s, args)
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

// a|b gate projection fused with the gate transform, for gfx950: the body that
// fd_gate_proj_fwd (gate_transform.hip) and fd_packed_conv_gate_fwd
// (packed_conv.hip) share.
//
// One workgroup owns 16 tokens.  Each output sums its hidden dimension in the
// order hipBLASLt's bf16 GEMM uses for the eager in_proj_a / in_proj_b
// projections (16 outputs, measured equal bit for bit on the MI355X at 1,024
// to 5,008 tokens): kProjParts = 4 parts, part p taking the 32-wide slice
// [128 j + 32 p, 128 j + 32 p + 32) of every 128-deep block j in turn, each
// slice one v_mfma_f32_16x16x32_bf16 into the part's accumulator (exact bf16
// products, fp32 sums); then ((p0 + p1) + p2) + p3.  Lane l supplies
// A = x[row0 + l%16][k + 8(l/16) .. +7] and B = W[n0 + l%16][same k] (16-byte
// loads); D[4(l/16)+r][l%16] is (token, output).  A workgroup of WAVES
// wavefronts gives wavefront wv the parts wv, wv + WAVES, ...; the arithmetic of
// every part is the same whatever WAVES is, so both launches produce the same
// bits, and no order depends on the token count.  The sum is rounded to bf16,
// the value a bf16 GEMM (F.linear) stores, then transformed:
//   g    = -exp(A_log) * softplus(a + dt_bias),  softplus(x) = x > 20 ? x : log1p(exp(x))
//   beta = bf16(sigmoid(b)),                     sigmoid(x) = 1 / (1 + exp(-x))
// in fp32 with the same library exp / log1p as PyTorch's elementwise kernels
// (ref: src/decider/unpack_gate_transform_kernel.py:51-91,
//  ref: src/decider/packed_conv.py:49-53).
#pragma once

#include "fd_common.h"

namespace fd_gate {

constexpr int kProjRows = 16;
constexpr int kProjParts = 4;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

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

// The LDS a workgroup needs for the partial sums of NB blocks of 16 outputs.
template <int NB>
using PartSmem = float[kProjParts][NB * 16][kProjRows + 1];

struct GateProjArgs {
  const uint16_t* x;  // [rows, hidden] bf16, row stride xs elements
  int64_t xs;
  const uint16_t* w;  // [2*heads, hidden] bf16 contiguous
  int hidden;
  const void* a_log;    // [heads] bf16 or fp32
  const void* dt_bias;  // [heads] bf16 or fp32
  float* g;             // [rows, heads] fp32
  uint16_t* beta;       // [rows, heads] bf16
  uint16_t* ab;         // [rows, 2*heads] bf16 or null
  int64_t rows;
};

// Workgroup `block` computes tokens [16*block, 16*block + 16).  Every thread of
// the workgroup must call it (it holds one barrier); blocks past the last token
// return before the barrier, as a whole.
template <typename LT, typename BT, int NB, int WAVES>
__device__ __forceinline__ void gate_proj_rows(int64_t block, const GateProjArgs& a, PartSmem<NB>& part) {
  static_assert(kProjParts % WAVES == 0, "each wavefront takes whole parts");
  constexpr int heads = 8 * NB;  // 2 * heads = NB blocks of 16 outputs
  const int64_t row0 = block * kProjRows;
  if (row0 >= a.rows) return;
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int l = tid & 63;
  const int64_t xrow = min(row0 + (l & 15), a.rows - 1);  // rows past the end re-read the last one
  const int nblk = a.hidden / 128;
#pragma unroll
  for (int pp = 0; pp < kProjParts / WAVES; ++pp) {
    const int p = wv + pp * WAVES;
    const uint16_t* xp = a.x + xrow * a.xs + 32 * p + 8 * (l >> 4);
    const uint16_t* wp = a.w + static_cast<int64_t>(l & 15) * a.hidden + 32 * p + 8 * (l >> 4);
    f32x4_t acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4_t{};
    for (int j0 = 0; j0 < nblk; j0 += 4) {
      // the operands of four blocks are loaded before their MFMAs
      bf16x8_t av[4], bv[4][NB];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int j = j0 + s < nblk ? j0 + s : nblk - 1;
        av[s] = *reinterpret_cast<const bf16x8_t*>(xp + 128 * j);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          bv[s][nb] = *reinterpret_cast<const bf16x8_t*>(wp + static_cast<int64_t>(16 * nb) * a.hidden + 128 * j);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (j0 + s < nblk) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[s], bv[s][nb], acc[nb], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[p][16 * nb + (l & 15)][4 * (l >> 4) + r] = acc[nb][r];
  }
  __syncthreads();
  for (int idx = tid; idx < kProjRows * heads; idx += 64 * WAVES) {
    const int rr = idx / heads;
    const int h = idx - rr * heads;
    const int64_t row = row0 + rr;
    if (row >= a.rows) break;
    float sa = part[0][h][rr];
    float sb = part[0][heads + h][rr];
#pragma unroll
    for (int p = 1; p < kProjParts; ++p) {
      sa = sa + part[p][h][rr];
      sb = sb + part[p][heads + h][rr];
    }
    const uint32_t abits = fd_f32_to_bf16(sa);
    const uint32_t bbits = fd_f32_to_bf16(sb);
    if (a.ab != nullptr) {
      a.ab[row * 2 * heads + h] = static_cast<uint16_t>(abits);
      a.ab[row * 2 * heads + heads + h] = static_cast<uint16_t>(bbits);
    }
    const float xa = fd_bf16_to_f32(abits) + load_param<BT>(a.dt_bias, h);
    const float sp = xa > 20.0f ? xa : log1pf(expf(xa));
    a.g[row * heads + h] = -expf(load_param<LT>(a.a_log, h)) * sp;
    const float y = fd_bf16_to_f32(bbits);
    a.beta[row * heads + h] = static_cast<uint16_t>(fd_f32_to_bf16(1.0f / (1.0f + expf(-y))));
  }
}

// Argument checks shared by both entry points; `who` names the entry point in
// the error text.
inline int gate_proj_check(const char* who, const void* x, int64_t x_row_stride, const void* weight, int hidden,
                           const void* a_log, int a_log_dtype, const void* dt_bias, int dt_bias_dtype,
                           const float* g, const void* beta, int64_t rows, int heads) {
  FD_REQUIRE(x && weight && a_log && dt_bias && g && beta, FD_ERR_INVALID_ARGUMENT,
             "%s: gate pointers must be non-null", who);
  FD_REQUIRE(rows >= 0, FD_ERR_INVALID_ARGUMENT, "%s: rows must be >= 0", who);
  FD_REQUIRE(heads == 8 || heads == 16 || heads == 24 || heads == 32, FD_ERR_UNSUPPORTED,
             "%s: heads must be 8, 16, 24 or 32 (got %d)", who, heads);
  FD_REQUIRE(hidden > 0 && hidden % 128 == 0, FD_ERR_UNSUPPORTED,
             "%s: hidden must be a positive multiple of 128 (got %d)", who, hidden);
  FD_REQUIRE(x_row_stride >= hidden && x_row_stride % 8 == 0 && fd_aligned16(x) && fd_aligned16(weight),
             FD_ERR_ALIGNMENT, "%s: x rows and weight must be 16-byte aligned, row stride >= hidden", who);
  FD_REQUIRE((a_log_dtype == FD_DTYPE_BF16 || a_log_dtype == FD_DTYPE_F32) &&
                 (dt_bias_dtype == FD_DTYPE_BF16 || dt_bias_dtype == FD_DTYPE_F32),
             FD_ERR_INVALID_ARGUMENT, "%s: parameter dtypes must be FD_DTYPE_BF16 or FD_DTYPE_F32", who);
  FD_REQUIRE((rows + kProjRows - 1) / kProjRows < (1LL << 30), FD_ERR_INVALID_ARGUMENT, "%s: problem too large",
             who);
  return FD_OK;
}

}  // namespace fd_gate

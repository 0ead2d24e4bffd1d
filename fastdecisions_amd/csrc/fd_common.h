// Shared device helpers and host error plumbing for the gfx950 kernels.
//
// Every kernel file is compiled with -ffp-contract=off: each fp32 operation
// below rounds exactly once, in the order written, so the CPU restatement of a
// kernel (compiled with the same flag) reproduces it bit for bit.  Fused
// multiply-adds are written explicitly (__builtin_fmaf) where they are meant.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fd_kernels.h"

// ---------------------------------------------------------------- host side

// Record a message for fd_last_error() and return `code`.
int fd_set_error(int code, const char* fmt, ...);
// Map the last HIP launch status of this thread to FD_OK / FD_ERR_LAUNCH.
int fd_check_launch(const char* what);

#define FD_REQUIRE(cond, code, ...)                 \
  do {                                              \
    if (!(cond)) return fd_set_error((code), __VA_ARGS__); \
  } while (0)

static inline bool fd_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// -------------------------------------------------------------- device side

// bf16 <-> fp32, round-to-nearest-even, NaN -> canonical quiet NaN: the same
// rule torch applies when it casts fp32 to bfloat16.
__device__ __forceinline__ float fd_bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t fd_f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two bf16 packed in one 32-bit word (low half = lower address).
__device__ __forceinline__ float fd_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float fd_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// v_cvt_pk_bf16_f32: round-to-nearest-even, identical to fd_f32_to_bf16 for
// every non-NaN input (checked exhaustively over all 2^32 fp32 patterns on
// gfx950); a NaN input gives a quiet NaN.
__device__ __forceinline__ uint32_t fd_pack2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The value of lane i and of lane i ^ M (M = 1 .. 32, a power of two) as a pair,
// with no LDS round trip: DPP inside each row of 16 lanes for M <= 8 (row_ror:n
// gives lane i the value of lane (i - n) mod 16, so ror 8 is i ^ 8, and i ^ 4 is
// ror 4 where bit 2 of i is set and ror 12 elsewhere), v_permlane16_swap /
// v_permlane32_swap across rows (with the value in both operands each lane
// receives its own value and its partner's, in an order that depends on the
// lane).  The sum and max below are symmetric in the pair, so they equal
// s + __shfl_xor(s, M) and fmaxf(s, __shfl_xor(s, M)) bit for bit.  Every lane of
// the wavefront must take part, in a 1-D workgroup whose size is a multiple of 64
// (the lane index is threadIdx.x % 64).
template <int M>
__device__ __forceinline__ void fd_xor_pair(float s, float& a, float& b) {
  const uint32_t u = __float_as_uint(s);
  if constexpr (M == 32 || M == 16) {
    auto r = M == 32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                     : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    int p;
    if constexpr (M == 1) {
      p = __builtin_amdgcn_mov_dpp(static_cast<int>(u), 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
      p = __builtin_amdgcn_mov_dpp(static_cast<int>(u), 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
      const int r4 = __builtin_amdgcn_mov_dpp(static_cast<int>(u), 0x124, 0xF, 0xF, false);   // row_ror:4
      const int r12 = __builtin_amdgcn_mov_dpp(static_cast<int>(u), 0x12C, 0xF, 0xF, false);  // row_ror:12
      p = (threadIdx.x & 4) ? r4 : r12;
    } else {
      static_assert(M == 8, "xor distance: a power of two below 64");
      p = __builtin_amdgcn_mov_dpp(static_cast<int>(u), 0x128, 0xF, 0xF, false);  // row_ror:8
    }
    a = s;
    b = __uint_as_float(static_cast<uint32_t>(p));
  }
}
template <int M>
__device__ __forceinline__ float fd_xor_sum(float s) {
  float a, b;
  fd_xor_pair<M>(s, a, b);
  return a + b;
}
template <int M>
__device__ __forceinline__ float fd_xor_max(float s) {
  float a, b;
  fd_xor_pair<M>(s, a, b);
  return fmaxf(a, b);
}

// s summed over each aligned group of N lanes (N = 2 .. 64) by an xor butterfly
// with distances 1, 2, .., N/2 (up) or N/2, .., 1 (down).
template <int N>
__device__ __forceinline__ float fd_xor_sum_up(float s) {
  if constexpr (N >= 2) s = fd_xor_sum<1>(s);
  if constexpr (N >= 4) s = fd_xor_sum<2>(s);
  if constexpr (N >= 8) s = fd_xor_sum<4>(s);
  if constexpr (N >= 16) s = fd_xor_sum<8>(s);
  if constexpr (N >= 32) s = fd_xor_sum<16>(s);
  if constexpr (N >= 64) s = fd_xor_sum<32>(s);
  return s;
}
template <int N>
__device__ __forceinline__ float fd_xor_sum_down(float s) {
  if constexpr (N >= 64) s = fd_xor_sum<32>(s);
  if constexpr (N >= 32) s = fd_xor_sum<16>(s);
  if constexpr (N >= 16) s = fd_xor_sum<8>(s);
  if constexpr (N >= 8) s = fd_xor_sum<4>(s);
  if constexpr (N >= 4) s = fd_xor_sum<2>(s);
  if constexpr (N >= 2) s = fd_xor_sum<1>(s);
  return s;
}

// SiLU exactly as PyTorch's GPU kernel evaluates it in fp32: y / (1 + expf(-y))
// with the device expf and the correctly rounded IEEE division (no fast-math).
// Measured on the MI355X: torch.nn.functional.silu on fp32 equals this
// expression bit for bit on every one of 25M conv outputs.
__device__ __forceinline__ float fd_silu(float y) { return y / (1.0f + expf(-y)); }

// A value whose bf16 rounding equals that of fd_silu(y), for every fp32 y
// (NaN in, NaN out).  It is y * rcp(1 + exp2(-y log2 e)) on the hardware exp2
// and reciprocal, about 5 instructions against about 22, and fd_silu itself
// where the two could round differently:
//  * results within kSiluTieWindow fp32 ulps of a bf16 rounding tie (low
//    half-word 0x8000);
//  * y < -16: there exp2 amplifies the rounding of y log2 e to tens of ulps.
// fd_silu_check counts the inputs where the two bf16 roundings differ; a GPU
// test runs it over all 2^32 fp32 bit patterns.  (Measured: a window of 16
// with the fast path down to y = -80 left 719 inputs rounding differently, no
// window 5590; windows 8-32 with cut-offs at -4 to -16 left none.)
constexpr uint32_t kSiluTieWindow = 32;
__device__ __forceinline__ float fd_silu_bf16(float y) {
  float f = y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y * -1.44269504088896341f));
  const uint32_t low = __float_as_uint(f) & 0xffffu;
  // bitwise |: both tests on every lane, one branch (|| would branch around the fast path too)
  if ((y < -16.0f) | (low + kSiluTieWindow - 0x8000u < 2u * kSiluTieWindow)) f = fd_silu(y);
  return f;
}

// A value whose bf16 rounding equals that of g * fd_silu(z), for bf16 values g
// and z (the gated RMSNorm's last product): g * (z * rcp(1 + exp2(-z log2 e)))
// on the hardware exp2 and reciprocal, and g * fd_silu(z) itself where the two
// could round differently (products within kSiluTieWindow fp32 ulps of a bf16
// rounding tie, and z < -16).  fd_gated_silu_check counts the pairs where the
// two bf16 roundings differ; a GPU test runs it over all 2^32 pairs of bf16
// bit patterns.
__device__ __forceinline__ float fd_gated_silu_bf16(float g, float z) {
  float p = g * (z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.44269504088896341f)));
  const uint32_t low = __float_as_uint(p) & 0xffffu;
  if ((z < -16.0f) | (low + kSiluTieWindow - 0x8000u < 2u * kSiluTieWindow)) p = g * fd_silu(z);
  return p;
}

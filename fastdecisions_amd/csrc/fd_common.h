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

// e^t for the SiLU, branch-free: t is first clamped to [-20, 89] (v_med3);
// Cody–Waite reduction t = k*ln2 + r with ln2 split into a head of 16
// significant bits (so k*head is exact) and a tail; degree-7 Taylor polynomial
// of e^r on |r| <= ln2/2 in Horner form; exact scaling by 2^k (v_ldexp, k in
// [-29, 129]: no subnormal result, overflow to +inf).  Error < 2 ulp on
// [-20, 88.7]; identical bits on CPU and GPU since every step is one IEEE op.
// The clamp changes nothing the SiLU can see: below -17.4, 1 + e^t == 1 in
// fp32, and above 88.73 e^t is +inf either way.
__device__ __forceinline__ float fd_exp_silu(float t) {
  const float kLog2e = 1.44269502162933349609375f;
  const float kLn2Hi = 0.693145751953125f;         // 0x3f317200
  const float kLn2Lo = 1.428606765330187045e-06f;  // ln2 - kLn2Hi
  t = __builtin_amdgcn_fmed3f(t, -20.0f, 89.0f);
  const float k = __builtin_rintf(t * kLog2e);
  float r = __builtin_fmaf(-k, kLn2Hi, t);
  r = __builtin_fmaf(-k, kLn2Lo, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(k));
}

// SiLU as the reference writes it: y / (1 + exp(-y)), correctly rounded division.
// A NaN y gives NaN whatever the clamped exponential returns.
__device__ __forceinline__ float fd_silu(float y) { return y / (1.0f + fd_exp_silu(-y)); }

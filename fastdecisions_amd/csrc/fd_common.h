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
__device__ __forceinline__ uint32_t fd_pack2(float lo, float hi) {
  return fd_f32_to_bf16(lo) | (fd_f32_to_bf16(hi) << 16);
}

// exp(x) in fp32: Cody–Waite reduction x = k*ln2 + r (ln2 split into a
// 16-significant-bit head and a tail so k*head is exact), degree-7 Taylor
// polynomial of e^r on |r| <= ln2/2 in Horner form, then an exact scaling by
// 2^k (two steps when the result is subnormal, so it rounds only once).
// Error < 2 ulp over the whole range; identical bits on CPU and GPU because
// every step is a single IEEE operation.
__device__ __forceinline__ float fd_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __uint_as_float(0x7f800000u);
  if (x < -103.972084045410156f) return 0.0f;
  const float kLog2e = 1.44269502162933349609375f;
  const float kLn2Hi = 0.693145751953125f;         // 0x3f317200
  const float kLn2Lo = 1.428606765330187045e-06f;  // ln2 - kLn2Hi
  float k = rintf(x * kLog2e);
  float r = __builtin_fmaf(-k, kLn2Hi, x);
  r = __builtin_fmaf(-k, kLn2Lo, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ki = static_cast<int>(k);
  if (ki > 127) return (p * 1.7014118346046923e38f) * __uint_as_float(static_cast<uint32_t>(ki - 127 + 127) << 23);
  if (ki < -126) return (p * __uint_as_float(static_cast<uint32_t>(ki + 64 + 127) << 23)) * 5.421010862427522e-20f;
  return p * __uint_as_float(static_cast<uint32_t>(ki + 127) << 23);
}

// SiLU as the reference writes it: y / (1 + exp(-y)), correctly rounded division.
__device__ __forceinline__ float fd_silu(float y) { return y / (1.0f + fd_expf(-y)); }

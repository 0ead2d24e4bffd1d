// A plain streaming device copy: the measured HBM ceiling that the bandwidth-bound
// kernels of this library are set against.  No counterpart in the reference.
//
// Each thread moves four 16-byte chunks a block apart (a wavefront reads and
// writes 1 KiB contiguous per instruction), all four loads issued before the
// first store.  Loads and stores carry the nontemporal hint, so the copied
// lines stream through the L2 instead of being kept for a reuse that never
// comes.  On an MI355X this moves 64 MiB + 64 MiB per launch at about
// 5.8 TB/s and 256 MiB + 256 MiB at about 6.3 TB/s, against about 4.8 TB/s
// for a device-to-device copy through PyTorch at 64 MiB.
#include "fd_common.h"

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void hbm_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                            int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n16;
       base += stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kThreads;
      if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kThreads;
      if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

}  // namespace

extern "C" FD_API int fd_hbm_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  FD_REQUIRE(src && dst, FD_ERR_INVALID_ARGUMENT, "fd_hbm_copy: pointers must be non-null");
  FD_REQUIRE(bytes >= 0 && bytes % 16 == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_hbm_copy: bytes must be a non-negative multiple of 16");
  FD_REQUIRE(fd_aligned16(src) && fd_aligned16(dst), FD_ERR_ALIGNMENT,
             "fd_hbm_copy: src and dst must be 16-byte aligned");
  if (bytes == 0) return FD_OK;
  const int64_t n16 = bytes / 16;
  const int64_t per_block = static_cast<int64_t>(kThreads) * kUnroll;
  const int64_t blocks = (n16 + per_block - 1) / per_block;
  const unsigned grid = static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20));
  hipLaunchKernelGGL(hbm_copy_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n16);
  return fd_check_launch("fd_hbm_copy");
}

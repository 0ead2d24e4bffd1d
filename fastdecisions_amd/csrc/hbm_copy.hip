// A plain streaming device copy: the measured HBM ceiling that the bandwidth-bound
// kernels of this library are set against.  No counterpart in the reference.
//
// Each thread moves `U` 16-byte chunks a block apart (a wavefront reads and
// writes 1 KiB contiguous per instruction), all of its loads issued before its
// first store.  Loads and stores carry the nontemporal hint, so the copied
// lines stream through the L2 instead of being kept for a reuse that never
// comes.  The best shape depends on the size: on an MI355X 25 MB + 25 MB per
// launch ran fastest with 4 chunks per thread in 512-thread blocks (5.4 TB/s),
// 67 MB + 67 MB with one chunk per thread in 256-thread blocks (5.8 TB/s),
// against about 4.8 TB/s for a device-to-device copy through PyTorch.  The
// caller picks the shape; a ceiling is the best of them.
#include "fd_common.h"

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int U, int BS>
__global__ __launch_bounds__(BS) void hbm_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                      int64_t n16) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * BS * U;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * BS * U + threadIdx.x; base < n16; base += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * BS;
      if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * BS;
      if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

template <int U, int BS>
void launch(const void* src, void* dst, int64_t n16, hipStream_t s) {
  const int64_t per_block = static_cast<int64_t>(BS) * U;
  const int64_t blocks = (n16 + per_block - 1) / per_block;
  const unsigned grid = static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20));
  hipLaunchKernelGGL((hbm_copy_kernel<U, BS>), dim3(grid), dim3(BS), 0, s, static_cast<const u32x4*>(src),
                     static_cast<u32x4*>(dst), n16);
}

}  // namespace

extern "C" FD_API int fd_hbm_copy(const void* src, void* dst, int64_t bytes, int chunks_per_thread, int block,
                                  void* stream) {
  FD_REQUIRE(src && dst, FD_ERR_INVALID_ARGUMENT, "fd_hbm_copy: pointers must be non-null");
  FD_REQUIRE(bytes >= 0 && bytes % 16 == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_hbm_copy: bytes must be a non-negative multiple of 16");
  FD_REQUIRE(fd_aligned16(src) && fd_aligned16(dst), FD_ERR_ALIGNMENT,
             "fd_hbm_copy: src and dst must be 16-byte aligned");
  FD_REQUIRE((chunks_per_thread == 1 || chunks_per_thread == 2 || chunks_per_thread == 4) &&
                 (block == 256 || block == 512),
             FD_ERR_UNSUPPORTED, "fd_hbm_copy: chunks_per_thread must be 1, 2 or 4 and block 256 or 512");
  if (bytes == 0) return FD_OK;
  const int64_t n16 = bytes / 16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (block == 256) {
    if (chunks_per_thread == 1) launch<1, 256>(src, dst, n16, s);
    else if (chunks_per_thread == 2) launch<2, 256>(src, dst, n16, s);
    else launch<4, 256>(src, dst, n16, s);
  } else {
    if (chunks_per_thread == 1) launch<1, 512>(src, dst, n16, s);
    else if (chunks_per_thread == 2) launch<2, 512>(src, dst, n16, s);
    else launch<4, 512>(src, dst, n16, s);
  }
  return fd_check_launch("fd_hbm_copy");
}

// Native GQA causal attention forward for gfx950 (bf16 MFMA, fp32 softmax).
//
// Computes what the reference's Triton kernel computes
// (ref: src/decider/native_gqa_kernel.py:6-113): per query head h, kv head
// h / (Hq/Hkv) (:39-41); S = Q K^T * scale; causal mask key <= query (:63-81);
// online softmax with running max / denominator and correction
// exp(m_old - m_new) (:84-104); P rounded to bf16 before P·V (:98-102);
// out = acc / denominator (:106-113).  The design is CDNA4's own:
//
// * One workgroup = 4 wavefronts = the query heads of one KV group (or, for
//   groups smaller than 4, several 32-query blocks of fewer heads).  A 64-key
//   K tile and the transposed V tile are staged once in LDS and read by all 4
//   wavefronts: K/V leave L2 once per group instead of once per query head.
// * The score tile is computed transposed, S^T = K · Q^T, with
//   v_mfma_f32_32x32x16_bf16.  In the 32x32 accumulator a lane owns one
//   column (= one query) and 16 rows (= keys), so the softmax row max and sum
//   are lane-local except for one xor-32 exchange between the two lane halves.
// * The K rows fed to the MFMA are permuted (sigma below) so that the 8 keys a
//   lane holds for each 16-key slice of P are exactly the 8 consecutive keys
//   it must supply as the B operand of O^T += V^T · P^T: P never leaves
//   registers.  V is transposed while it is staged (4 keys x 8 dims per
//   thread, 8-byte LDS stores) so the A operand is one 16-byte LDS read.
// * The output is accumulated transposed (O^T), so the per-query rescale by
//   exp(m_old - m_new) and the final 1/denominator are lane-local too.
// * Register double buffering: the next K/V tile is loaded from global memory
//   while the current one is consumed from LDS; one barrier per tile.
// * Work items are ordered longest-first (causal tiles near the end of the
//   sequence have the most keys) and mapped so that each XCD receives a
//   contiguous range of (head group, query tile) items, keeping a KV head's
//   tiles in one L2.
#include "fd_common.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlockM = 32;  // queries per wavefront
constexpr int kBlockN = 64;  // keys per LDS tile
constexpr int kNumXcd = 8;

struct GqaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t qs[4], ks[4], vs[4], os[4];
  int q_heads, kv_heads, seq_len;
  float scale_log2;
  const int32_t* cu;
  int n_seqs;
  int hpw;        // query heads per workgroup
  int qpw;        // 32-query blocks per workgroup (hpw * qpw == 4)
  int n_qtiles;   // query tiles per (sequence, head group)
  int n_hgroups;  // q_heads / hpw
  int n_items;    // n_qtiles * n_hgroups * sequences
};

template <int D>
struct Tile {
  static constexpr int kRow = D + 8;         // K tile row stride (bf16), 16-byte pad
  static constexpr int kVtRow = kBlockN + 8;  // V^T row stride (bf16), 16-byte pad
  static constexpr int kKElems = kBlockN * kRow;
  static constexpr int kVElems = D * kVtRow;
  static constexpr int kStage = kKElems + kVElems;
  static constexpr int kKChunks = kBlockN * D / 8 / kThreads;          // 16-B K chunks per thread
  static constexpr int kVTasks = (kBlockN / 4) * (D / 8);             // (4 keys x 8 dims) tasks
  static constexpr int kVPerThread = (kVTasks + kThreads - 1) / kThreads;
};

// Key (within a 32-key block) supplied by MFMA row m, chosen so that the
// accumulator registers 8j..8j+7 of lane half g hold keys 16j + 8g + 0..7.
__device__ __forceinline__ int sigma(int m) {
  return ((m >> 4) << 4) + (((m >> 2) & 1) << 3) + (((m >> 3) & 1) << 2) + (m & 3);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

template <int D>
__global__ __launch_bounds__(kThreads, 1) void gqa_fwd_kernel(GqaArgs a) {
  using T = Tile<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * T::kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query within the wavefront's block
  const int half = lane >> 5;

  // ---- work item: XCD-contiguous renumbering, longest tile first
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int item = (nb % kNumXcd == 0) ? (b % kNumXcd) * (nb / kNumXcd) + b / kNumXcd : b;
  if (item >= a.n_items) return;
  const int j = item % a.n_qtiles;
  const int hg = (item / a.n_qtiles) % a.n_hgroups;
  const int sidx = item / (a.n_qtiles * a.n_hgroups);
  const int qtile = a.n_qtiles - 1 - j;

  int seq_start, seq_end, bidx;
  if (a.cu != nullptr) {
    seq_start = a.cu[sidx];
    seq_end = a.cu[sidx + 1];
    bidx = 0;
  } else {
    seq_start = 0;
    seq_end = a.seq_len;
    bidx = sidx;
  }
  const int qspan = kBlockM * a.qpw;
  const int q0 = seq_start + qtile * qspan;
  if (q0 >= seq_end) return;  // uniform over the workgroup

  const int group = a.q_heads / a.kv_heads;
  const int hsub = wave % a.hpw;
  const int qb = wave / a.hpw;
  const int qhead = hg * a.hpw + hsub;
  const int kvhead = (hg * a.hpw) / group;

  const uint16_t* qbase = a.q + bidx * a.qs[0] + qhead * a.qs[1];
  const uint16_t* kbase = a.k + bidx * a.ks[0] + kvhead * a.ks[1];
  const uint16_t* vbase = a.v + bidx * a.vs[0] + kvhead * a.vs[1];
  uint16_t* obase = a.o + bidx * a.os[0] + qhead * a.os[1];

  const int qw0 = q0 + qb * kBlockM;  // first query of this wavefront
  const int qpos = qw0 + col;
  const bool qvalid = qpos < seq_end;

  // Q^T as MFMA B operand: lane supplies Q[qpos][16kk + 8*half + 0..7].
  bf16x8_t qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    uint4 u = make_uint4(0u, 0u, 0u, 0u);
    if (qvalid) u = *reinterpret_cast<const uint4*>(qbase + qpos * a.qs[2] + kk * 16 + half * 8);
    qf[kk] = as_bf16x8(u);
  }

  const int kend = min(q0 + qspan, seq_end);
  const int ntiles = (kend - seq_start + kBlockN - 1) / kBlockN;

  // ---- global -> register staging of one K/V tile
  uint4 kreg[T::kKChunks];
  uint4 vreg[T::kVPerThread][4];
  auto load_tile = [&](int t) {
    const int ks0 = seq_start + t * kBlockN;
#pragma unroll
    for (int i = 0; i < T::kKChunks; ++i) {
      const int c = tid + kThreads * i;
      const int row = c / (D / 8), c8 = c % (D / 8);
      const int key = ks0 + row;
      kreg[i] = key < seq_end ? *reinterpret_cast<const uint4*>(kbase + key * a.ks[2] + c8 * 8)
                              : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < T::kVPerThread; ++i) {
      const int c = tid + kThreads * i;
      if (c < T::kVTasks) {
        const int k4 = c % (kBlockN / 4), d8 = c / (kBlockN / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = ks0 + k4 * 4 + r;
          vreg[i][r] = key < seq_end ? *reinterpret_cast<const uint4*>(vbase + key * a.vs[2] + d8 * 8)
                                     : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  };
  auto store_tile = [&](int stage) {
    uint16_t* ks_l = smem + stage * T::kStage;
    uint16_t* vt_l = ks_l + T::kKElems;
#pragma unroll
    for (int i = 0; i < T::kKChunks; ++i) {
      const int c = tid + kThreads * i;
      const int row = c / (D / 8), c8 = c % (D / 8);
      *reinterpret_cast<uint4*>(ks_l + row * T::kRow + c8 * 8) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < T::kVPerThread; ++i) {
      const int c = tid + kThreads * i;
      if (c < T::kVTasks) {
        const int k4 = c % (kBlockN / 4), d8 = c / (kBlockN / 4);
        const uint32_t w0[4] = {vreg[i][0].x, vreg[i][0].y, vreg[i][0].z, vreg[i][0].w};
        const uint32_t w1[4] = {vreg[i][1].x, vreg[i][1].y, vreg[i][1].z, vreg[i][1].w};
        const uint32_t w2[4] = {vreg[i][2].x, vreg[i][2].y, vreg[i][2].z, vreg[i][2].w};
        const uint32_t w3[4] = {vreg[i][3].x, vreg[i][3].y, vreg[i][3].z, vreg[i][3].w};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // dims 2p (low halves) and 2p+1 (high halves) of keys 4*k4 + 0..3
          uint2 lo, hi;
          lo.x = (w0[p] & 0xffffu) | (w1[p] << 16);
          lo.y = (w2[p] & 0xffffu) | (w3[p] << 16);
          hi.x = (w0[p] >> 16) | (w1[p] & 0xffff0000u);
          hi.y = (w2[p] >> 16) | (w3[p] & 0xffff0000u);
          *reinterpret_cast<uint2*>(vt_l + (d8 * 8 + 2 * p) * T::kVtRow + k4 * 4) = lo;
          *reinterpret_cast<uint2*>(vt_l + (d8 * 8 + 2 * p + 1) * T::kVtRow + k4 * 4) = hi;
        }
      }
    }
  };

  f32x16_t o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = f32x16_t{};
  float m_run = -__builtin_inff();
  float l_run = 0.0f;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int krow_a = sigma(col);  // K row this lane supplies as MFMA A operand
  for (int t = 0; t < ntiles; ++t) {
    const int stage = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
    const int ks0 = seq_start + t * kBlockN;
    const uint16_t* ks_l = smem + stage * T::kStage;
    const uint16_t* vt_l = ks_l + T::kKElems;

    // Tiles entirely after this wavefront's last query carry no visible key.
    if (ks0 <= qw0 + kBlockM - 1) {
      // S^T for keys ks0 + [0,32) and ks0 + [32,64)
      f32x16_t s[2];
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        s[blk] = f32x16_t{};
        const uint16_t* kr = ks_l + (blk * 32 + krow_a) * T::kRow + half * 8;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(kr + kk * 16);
          s[blk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qf[kk], s[blk], 0, 0, 0);
        }
      }
      // scale (log2 domain) + causal / end-of-sequence mask
      const bool need_mask = (ks0 + kBlockN - 1 > qw0) || (ks0 + kBlockN > seq_end);
      float mx = -__builtin_inff();
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[blk][r] * a.scale_log2;
          if (need_mask) {
            const int key = ks0 + blk * 32 + (r >> 3) * 16 + half * 8 + (r & 7);
            if (key > qpos || key >= seq_end) x = -__builtin_inff();
          }
          s[blk][r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      // m_new is finite: the first tile always holds key seq_start <= qpos.
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      float psum = 0.0f;
      bf16x8_t pb[4];
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          f32x8_t pv;
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const float p = __builtin_amdgcn_exp2f(s[blk][h2 * 8 + r] - m_new);
            psum += p;
            pv[r] = p;
          }
          pb[blk * 2 + h2] = __builtin_convertvector(pv, bf16x8_t);
        }
      }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
      // O^T += V^T · P^T over four 16-key slices
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const uint16_t* vr = vt_l + (db * 32 + col) * T::kVtRow + half * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(vr + c * 16);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[c], o[db], 0, 0, 0);
        }
      }
    }
    if (t + 1 < ntiles) store_tile(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / denominator, 4 consecutive dims per 8-byte store
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / l_tot;
  if (qvalid) {
    uint16_t* orow = obase + qpos * a.os[2];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = db * 32 + r4 * 8 + half * 4;
        uint2 w;
        w.x = fd_pack2(o[db][r4 * 4 + 0] * inv, o[db][r4 * 4 + 1] * inv);
        w.y = fd_pack2(o[db][r4 * 4 + 2] * inv, o[db][r4 * 4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
    }
  }
}

int gcd_int(int x, int y) {
  while (y) {
    int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

bool stride_ok(const int64_t s[4]) {
  if (s[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8 != 0) return false;  // 16-byte rows
  return true;
}

}  // namespace

extern "C" int fd_gqa_fwd(const void* q, const void* k, const void* v, void* out, const int64_t q_strides[4],
                          const int64_t k_strides[4], const int64_t v_strides[4], const int64_t out_strides[4],
                          int batch, int q_heads, int kv_heads, int seq_len, int head_dim, float scale,
                          const int32_t* cu_seqlens, int n_seqs, int max_seqlen, void* stream) {
  FD_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: tensor and stride pointers must be non-null");
  FD_REQUIRE(batch >= 0 && seq_len >= 0 && q_heads >= 1 && kv_heads >= 1, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: batch/seq_len must be >= 0 and head counts >= 1");
  FD_REQUIRE(q_heads % kv_heads == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: q_heads (%d) must be divisible by kv_heads (%d)", q_heads, kv_heads);
  FD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, FD_ERR_UNSUPPORTED,
             "fd_gqa_fwd: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  FD_REQUIRE(scale > 0.0f && scale < 1e30f, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: scale must be positive");
  FD_REQUIRE(stride_ok(q_strides) && stride_ok(k_strides) && stride_ok(v_strides) && stride_ok(out_strides),
             FD_ERR_ALIGNMENT,
             "fd_gqa_fwd: innermost strides must be 1 and the others multiples of 8 elements (16 bytes)");
  FD_REQUIRE(fd_aligned16(q) && fd_aligned16(k) && fd_aligned16(v) && fd_aligned16(out), FD_ERR_ALIGNMENT,
             "fd_gqa_fwd: tensors must be 16-byte aligned");
  int n_slots;
  int span_len;
  if (cu_seqlens != nullptr) {
    FD_REQUIRE(batch == 1, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: cu_seqlens requires batch == 1 (got %d)", batch);
    FD_REQUIRE(n_seqs >= 1, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: n_seqs must be >= 1");
    FD_REQUIRE(max_seqlen >= 0 && max_seqlen <= seq_len, FD_ERR_INVALID_ARGUMENT,
               "fd_gqa_fwd: max_seqlen must be in [0, seq_len]");
    n_slots = n_seqs;
    span_len = max_seqlen;
  } else {
    n_slots = batch;
    span_len = seq_len;
  }
  if (n_slots == 0 || span_len == 0) return FD_OK;

  const int group = q_heads / kv_heads;
  GqaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(out);
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.os[i] = out_strides[i];
  }
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.seq_len = seq_len;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.cu = cu_seqlens;
  a.n_seqs = n_seqs;
  a.hpw = gcd_int(group, kWaves);
  a.qpw = kWaves / a.hpw;
  a.n_qtiles = (span_len + kBlockM * a.qpw - 1) / (kBlockM * a.qpw);
  a.n_hgroups = q_heads / a.hpw;
  const int64_t items = static_cast<int64_t>(a.n_qtiles) * a.n_hgroups * n_slots;
  FD_REQUIRE(items < 2147483647LL, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: problem too large");
  a.n_items = static_cast<int>(items);
  const int nblocks = static_cast<int>((items + kNumXcd - 1) / kNumXcd * kNumXcd);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(nblocks), block(kThreads);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(gqa_fwd_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(gqa_fwd_kernel<128>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(gqa_fwd_kernel<256>, grid, block, 0, s, a); break;
  }
  return fd_check_launch("fd_gqa_fwd");
}

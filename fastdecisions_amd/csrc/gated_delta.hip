// Chunked gated delta rule forward for gfx950 (fp32 arithmetic, MFMA).
//
// Computes what transformers' torch_chunk_gated_delta_rule computes for the
// decider's linear-attention layers (called at ref: src/decider/packed_conv.py:55-59
// with use_qk_l2norm_in_kernel=True; transformers modeling_qwen3_5.py:249-328),
// per value head h (key head h / (Hv/Hk), the repeat_interleave mapping):
//
//   q, k <- l2norm(q), l2norm(k) on the bf16 rows, each step rounded to bf16
//   q <- q * scale;  per 64-token chunk: gc = cumsum(g),  D_ij = e^{gc_i - gc_j} (j <= i)
//   L = strictly-lower(beta_i k_i.k_j D_ij),  T = (I + L)^-1
//   u = T (beta v),  w = T (beta e^{gc} k),   A = (q k^T) o D (j <= i)
//   across chunks, state S [dk, dv] (zero or the initial state):
//     v' = u - w S;  o = (q e^{gc}) S + A v';  S <- e^{gc_last} S + (k e^{gc_last - gc})^T v'
//
// Packed requests (cu_seqlens) are chunked per request and each request starts
// from its own state, so no state crosses a request boundary.
//
// Up to four launches, all on the caller's stream, intermediates in a
// caller-provided workspace (fd_gated_delta_workspace_bytes):
//   1. gd_chunk_table — packed requests only, one workgroup: chunk -> (first
//      row, length), request -> first chunk.  A padded batch needs no table.
//   2. gd_prep_kernel — one workgroup per (chunk, value head), chunk-parallel:
//      l2norm, cumsum, the Gram and q.k tiles on bf16 MFMA (the normalised q/k
//      are bf16 values, so these products are exact before fp32 accumulation),
//      then u and w as the solutions of (I + L) x = rhs by forward substitution,
//      one right-hand-side column per thread (256 columns: 128 of u, 128 of w),
//      in four 16-row blocks; each finished block is stored while the next runs.
//   3. gd_state_kernel — one workgroup per (request, value head, 16 value
//      columns): the only sequential part.  Each state column evolves on its
//      own, so the 128 value columns split over 8 workgroups.  Four wavefronts
//      run the chain: the state slice lives in their registers, and the
//      operands of the chunks two ahead are loaded straight into registers
//      (three register sets) while the current chunk runs; two barriers per
//      chunk.  Four more wavefronts, one per SIMD beside the chain's, compute
//      each chunk's output o = scale e^{gc} (q S_chunk) + A v' for the
//      slice's columns from the state and v' planes the chain leaves in LDS,
//      so neither the chunk-start states nor v' go through HBM.
//      All products run on bf16 MFMA over exact bf16 splits of the fp32 operands.
//   4. fd_gated_rmsnorm_fwd's kernel — with the layer's gated RMSNorm
//      (fd_gated_delta_norm_fwd) only: the output rows, written to the
//      workspace, normalised into the caller's output.
// The intermediates sit in the workspace in the order their consumer's MFMA
// operands are loaded (one wavefront load = 1-2 KiB contiguous).  The MFMA
// lane layout (v_mfma_f32_16x16x32_bf16): lane l supplies A[l%16][8(l/16)+j]
// and B[8(l/16)+j][l%16] for j = 0..7 of each 32-step; D[4(l/16)+r][l%16].
#include <mutex>
#include <type_traits>

#include "fd_common.h"

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

namespace {

constexpr int kC = 64;                 // tokens per chunk
constexpr int kD = 128;                // head_k_dim == head_v_dim
constexpr int kSlice = 16;             // value columns per state workgroup
constexpr int kSlices = kD / kSlice;   // state workgroups per (request, head)
constexpr int kThreads = 256;

struct GdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g;
  const void* beta;
  uint16_t* o;
  const float* s0;   // [N, Hv, Dk, Dv] or null
  float* sN;         // [N, Hv, Dk, Dv] or null
  int32_t* row0;     // [nc]  first packed row of each chunk
  int32_t* len;      // [nc]  valid rows of each chunk (0 = unused)
  int32_t* first;    // [N+1] first chunk of each request
  float* gc;         // [Hv, nc, 3, 64]: e^{gc_t}, e^{gl - gc_t}, then e^{gl} (gl = gc of the last row)
  // q and A are stored in the state pass's output-wavefront operand order
  // (lane = 16 * g4 + c16): every load there reads 1-2 KiB contiguous
  uint16_t* qn;      // [Hv, nc, rt 4, st 4, lane 64, 8] bf16: q[16rt + c16][32st + 8g4 + e]
  // w, k^T and u are stored in the state pass's operand order: every load of a
  // wavefront there reads 1 KiB contiguous (lane = 16 * g4 + c16, see gd_state_kernel)
  uint16_t* kn;      // [Hv, nc, wv 4, m 2, st 2, lane 64, 8] bf16: k^T[32wv + 16m + c16][32st + 8g4 + e]
  uint16_t* w;       // [Hv, nc, plane 3, wv 4, st 4, lane 64, 8] bf16: w_x[16wv + c16][32st + 8g4 + e],
                     // w split exactly into hi + mid + lo planes
  float* u;          // [Hv, nc, js 8, wv 4, lane 64, r 4]: u[16wv + 4g4 + r][16js + c16]
  float* aq;         // [Hv, nc, rt 4, st 2, lane 64, 8]: A[16rt + c16][32st + 8g4 + e]
  int hk, hv, nc, nseq;
  int varlen, seq_len, nct;  // packed requests (table) or a padded batch of nct chunks per sequence
  int beta_f32, l2norm;
  float scale;
};

// round to bf16 and back (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ float bf16r(float x) { return fd_lo(fd_pack2(x, 0.0f)); }

__device__ __forceinline__ f32x4_t mfma_f32(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// x == hi + mid + lo exactly (each a bf16; the two differences are exact in fp32),
// so a product with a bf16 value is three exact bf16 products accumulated in fp32.
// The conversions are v_cvt_pk_bf16_f32 (round to nearest even).
// four fp32 values -> three planes of four bf16 each (8 bytes per plane)
__device__ __forceinline__ void split3x4(const float* x, uint2& hi, uint2& mid, uint2& lo) {
  const uint32_t h01 = fd_pack2(x[0], x[1]), h23 = fd_pack2(x[2], x[3]);
  const float r[4] = {x[0] - fd_lo(h01), x[1] - fd_hi(h01), x[2] - fd_lo(h23), x[3] - fd_hi(h23)};
  const uint32_t m01 = fd_pack2(r[0], r[1]), m23 = fd_pack2(r[2], r[3]);
  const uint32_t l01 = fd_pack2(r[0] - fd_lo(m01), r[1] - fd_hi(m01));
  const uint32_t l23 = fd_pack2(r[2] - fd_lo(m23), r[3] - fd_hi(m23));
  hi = make_uint2(h01, h23);
  mid = make_uint2(m01, m23);
  lo = make_uint2(l01, l23);
}

__device__ __forceinline__ void unpack8(uint4 raw, float* x) {
  const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = fd_lo(wd[i]);
    x[2 * i + 1] = fd_hi(wd[i]);
  }
}

__device__ __forceinline__ uint4 pack8(const float* x) {
  uint4 r;
  r.x = fd_pack2(x[0], x[1]);
  r.y = fd_pack2(x[2], x[3]);
  r.z = fd_pack2(x[4], x[5]);
  r.w = fd_pack2(x[6], x[7]);
  return r;
}

// transformers' l2norm on a bf16 row of 128 held by 16 consecutive lanes (8
// values each): x*x rounded to bf16, summed in fp32 (lane chunk order, then an
// xor butterfly over the 16 lanes), the sum, sum + eps and 1/sqrt each rounded
// to bf16, then x * inv rounded to bf16.  Every lane of the wavefront must call it.
__device__ __forceinline__ uint4 l2norm_row8(uint4 raw) {
  float x[8];
  unpack8(raw, x);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = s + bf16r(x[e] * x[e]);
  s = fd_xor_sum_down<16>(s);
  const float e = bf16r(bf16r(s) + 1e-6f);
  const float inv = bf16r(1.0f / __builtin_sqrtf(e));
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = x[i] * inv;
  return pack8(y);
}

// ---------------------------------------------------------------------------
// 1. chunk table (one workgroup)
__global__ __launch_bounds__(kThreads) void gd_chunk_table(const int32_t* __restrict__ cu, int nseq, int seq_len,
                                                           int total, GdArgs a) {
  __shared__ int scan[kThreads];
  const int t = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < nseq; base += kThreads) {
    const int s = base + t;
    int start = 0, end = 0;
    if (s < nseq) {
      if (cu != nullptr) {
        start = min(max(cu[s], 0), total);
        end = min(max(cu[s + 1], start), total);
      } else {
        start = s * seq_len;
        end = start + seq_len;
      }
    }
    const int n = (end - start + kC - 1) / kC;
    scan[t] = n;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
      const int add = t >= off ? scan[t - off] : 0;
      __syncthreads();
      scan[t] += add;
      __syncthreads();
    }
    const int f = carry + scan[t] - n;
    const int block_total = scan[kThreads - 1];
    __syncthreads();
    if (s < nseq) {
      a.first[s] = f;
      for (int j = 0; j < n && f + j < a.nc; ++j) {
        a.row0[f + j] = start + j * kC;
        a.len[f + j] = min(kC, end - start - j * kC);
      }
    }
    carry += block_total;
  }
  if (t == 0) a.first[nseq] = carry;
  for (int c = carry + t; c < a.nc; c += kThreads) {
    a.row0[c] = 0;
    a.len[c] = 0;
  }
}

// ---------------------------------------------------------------------------
// chunk and request ranges: from the table for packed requests, by arithmetic
// for a padded batch (no table launch)
__device__ __forceinline__ void chunk_rows(const GdArgs& a, int c, int* r0, int* len) {
  if (a.varlen) {
    *r0 = a.row0[c];
    *len = a.len[c];
  } else {
    const int s = c / a.nct;
    const int j = c - s * a.nct;
    *r0 = s * a.seq_len + j * kC;
    *len = min(kC, a.seq_len - j * kC);
  }
}

__device__ __forceinline__ void request_chunks(const GdArgs& a, int s, int* first, int* last) {
  if (a.varlen) {
    *first = a.first[s];
    *last = min(a.first[s + 1], a.nc);
  } else {
    *first = s * a.nct;
    *last = (s + 1) * a.nct;
  }
}

// ---------------------------------------------------------------------------
// 2. per-chunk preparation
constexpr int kRowK = kD + 8;    // bf16 row stride of the row-major q/k/v tiles (272 B)
constexpr int kRowF = kC + 4;    // fp32 row stride of the 64x64 tiles (272 B)
constexpr int kPrepK = 0;                                   // bf16 [64][kRowK]
constexpr int kPrepQ = kPrepK + kC * kRowK * 2;             // bf16 [64][kRowK]
constexpr int kPrepV = kPrepQ + kC * kRowK * 2;             // bf16 [64][kRowK]
constexpr int kPrepL = kPrepV + kC * kRowK * 2;             // fp32 [64][kRowF]
constexpr int kPrepG = kPrepL + kC * kRowF * 4;             // fp32 [64]  gc
constexpr int kPrepB = kPrepG + kC * 4;                     // fp32 [64]  beta
constexpr int kPrepBG = kPrepB + kC * 4;                    // fp32 [64]  beta e^gc
constexpr int kPrepBytes = kPrepBG + kC * 4;

// position of A[i][j] in the state pass's output-wavefront operand order
__device__ __forceinline__ int aq_index(int i, int j) {
  return (((i >> 4) * 2 + (j >> 5)) * 64 + 16 * ((j & 31) >> 3) + (i & 15)) * 8 + (j & 7);
}

// Inside a 16-row block the solve reads row m of the transposed L tile in 4-wide
// pieces starting at (m + 1) & ~3, for m = 0..14: 36 reads, piece k at (tri_m(k), tri_i0(k)).
constexpr int kTriReads = 36;
constexpr int kTriWin = 8;
// rows 0-2 have 4 pieces, rows 3-6 three, rows 7-10 two, rows 11-14 one
constexpr int tri_m(int k) {
  return k < 12 ? k / 4 : k < 24 ? 3 + (k - 12) / 3 : k < 32 ? 7 + (k - 24) / 2 : 11 + (k - 32);
}
constexpr int tri_i0(int k) {
  return k < 12 ? 4 * (k % 4) : k < 24 ? 4 + 4 * ((k - 12) % 3) : k < 32 ? 8 + 4 * ((k - 24) % 2) : 12;
}
static_assert(tri_m(kTriReads - 1) == 14 && tri_i0(kTriReads - 1) == 12 && tri_m(11) == 2 && tri_i0(11) == 12 &&
                  tri_m(12) == 3 && tri_i0(12) == 4 && tri_m(24) == 7 && tri_i0(25) == 12 && tri_m(32) == 11,
              "36 pieces in the inner solve of a 16-row block");

// One workgroup per (chunk, value head).  u = T (beta v) and w = T (beta e^gc k)
// are the solutions of (I + L) x = rhs; thread j < 128 solves for column j of
// u, thread 128 + j for column j of w, by forward substitution with the rows of
// L read from LDS (every lane reads the same address: broadcast).
// BETA_F32: beta is fp32 (else bf16).
template <bool BETA_F32>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void gd_prep_kernel(GdArgs a) {
  const int h = blockIdx.x % a.hv;
  const int c = blockIdx.x / a.hv;
  int r0, L;
  chunk_rows(a, c, &r0, &L);
  if (L <= 0) return;
  const int hk = h / (a.hv / a.hk);
  const size_t hc = static_cast<size_t>(h) * a.nc + c;

  __shared__ __attribute__((aligned(16))) unsigned char smem[kPrepBytes];
  uint16_t* sK = reinterpret_cast<uint16_t*>(smem + kPrepK);
  uint16_t* sQ = reinterpret_cast<uint16_t*>(smem + kPrepQ);
  uint16_t* sV = reinterpret_cast<uint16_t*>(smem + kPrepV);
  float* sL = reinterpret_cast<float*>(smem + kPrepL);
  float* sG = reinterpret_cast<float*>(smem + kPrepG);
  float* sB = reinterpret_cast<float*>(smem + kPrepB);
  float* sBG = reinterpret_cast<float*>(smem + kPrepBG);

  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int l = tid & 63;
  const int g4 = l >> 4;
  const int c16 = l & 15;

  // q, k, v rows: 16 lanes per row, 8 values (16 bytes) per lane
  const size_t qk_row = static_cast<size_t>(a.hk) * kD;
  const size_t v_row = static_cast<size_t>(a.hv) * kD;
  uint16_t* gq = a.qn + hc * kC * kD;
  // g and beta of row l (padded rows carry g = beta = 0; wave 0 uses them), loaded
  // first and by every wave, with no branch to convert in: wave 0 runs the cumsum
  // below while the q, k, v rows are in flight
  const size_t gidx = static_cast<size_t>(r0 + (l < L ? l : 0)) * a.hv + h;
  const float graw = a.g[gidx];
  float braw;
  if constexpr (BETA_F32)
    braw = static_cast<const float*>(a.beta)[gidx];
  else
    braw = fd_bf16_to_f32(static_cast<const uint16_t*>(a.beta)[gidx]);
  __builtin_amdgcn_sched_barrier(0);
  // every load of the block is issued before any is used (rows past the chunk's
  // end re-read its first row and are zeroed below)
  uint4 rq[4], rk[4], rv[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = it * 16 + wv * 4 + g4;
    const size_t grow = static_cast<size_t>(r0 + (row < L ? row : 0));
    rq[it] = *reinterpret_cast<const uint4*>(a.q + grow * qk_row + hk * kD + c16 * 8);
    rk[it] = *reinterpret_cast<const uint4*>(a.k + grow * qk_row + hk * kD + c16 * 8);
    rv[it] = *reinterpret_cast<const uint4*>(a.v + grow * v_row + h * kD + c16 * 8);
  }
  // g (inclusive cumsum over the chunk) and beta
  if (wv == 0) {
    float gv = l < L ? graw : 0.0f;
    const float bv = l < L ? braw : 0.0f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float up = __shfl_up(gv, off);
      if (l >= off) gv = gv + up;
    }
    sG[l] = gv;
    sB[l] = bv;
    const float eg = expf(gv);
    sBG[l] = bv * eg;
    const float gl = __shfl(gv, kC - 1);
    float* gx = a.gc + hc * 3 * kC;
    gx[l] = eg;
    gx[kC + l] = expf(gl - gv);
    if (l == 0) gx[2 * kC] = expf(gl);
  }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = it * 16 + wv * 4 + g4;
    const uint4 zero = make_uint4(0, 0, 0, 0);
    uint4 q4 = row < L ? rq[it] : zero;
    uint4 k4 = row < L ? rk[it] : zero;
    const uint4 v4 = row < L ? rv[it] : zero;
    if (a.l2norm) {
      q4 = l2norm_row8(q4);
      k4 = l2norm_row8(k4);
    }
    *reinterpret_cast<uint4*>(sQ + row * kRowK + c16 * 8) = q4;
    *reinterpret_cast<uint4*>(sK + row * kRowK + c16 * 8) = k4;
    *reinterpret_cast<uint4*>(sV + row * kRowK + c16 * 8) = v4;
    *reinterpret_cast<uint4*>(gq + (((row >> 4) * 4 + (c16 >> 2)) * 64 + 16 * (c16 & 3) + (row & 15)) * 8) = q4;
  }
  __syncthreads();

  // Gram (k.k) and q.k lower 32x32 tiles on bf16 MFMA; wave 3 zeroes A's upper tile
  float* gaq = a.aq + hc * kC * kC;
  if (wv < 3) {
    const int I = wv == 0 ? 0 : 1;
    const int J = wv == 2 ? 1 : 0;
    f32x16_t accG = {};
    f32x16_t accA = {};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int kc = 16 * s + 8 * (l >> 5);
      const bf16x8_t ak = *reinterpret_cast<const bf16x8_t*>(sK + (32 * I + (l & 31)) * kRowK + kc);
      const bf16x8_t aq = *reinterpret_cast<const bf16x8_t*>(sQ + (32 * I + (l & 31)) * kRowK + kc);
      const bf16x8_t bk = *reinterpret_cast<const bf16x8_t*>(sK + (32 * J + (l & 31)) * kRowK + kc);
      accG = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, bk, accG, 0, 0, 0);
      accA = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, bk, accA, 0, 0, 0);
    }
    const int j = 32 * J + (l & 31);
    const float gj = sG[j];
    // gc and beta of the lane's 16 rows 32I + 8q + 4(l/32) + e, read before any is
    // used, and the decays computed for every row and then selected: a branch per
    // row would serialise the 16 LDS round trips
    f32x4_t gi[4], bi[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gi[q] = *reinterpret_cast<const f32x4_t*>(sG + 32 * I + 8 * q + 4 * (l >> 5));
      bi[q] = *reinterpret_cast<const f32x4_t*>(sB + 32 * I + 8 * q + 4 * (l >> 5));
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * I + (r >> 2) * 8 + (l >> 5) * 4 + (r & 3);
      const float e = expf(gi[r >> 2][r & 3] - gj);
      const float dec = i >= j ? e : 0.0f;
      sL[j * kRowF + i] = i > j ? (bi[r >> 2][r & 3] * accG[r]) * dec : 0.0f;  // transposed: sL[j][i] = L[i][j]
      gaq[aq_index(i, j)] = i >= j ? (a.scale * accA[r]) * dec : 0.0f;
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) gaq[aq_index(r * 2 + (l >> 5), 32 + (l & 31))] = 0.0f;
  }
  __syncthreads();

  // forward substitution (I + L) x = rhs, one column per thread (wave wv owns the 64
  // columns of its lanes), in four blocks of 16 rows:
  //  - inside a block, right-looking on the thread's column: once x_m is final every
  //    later row of the block takes -L[i][m] x_m (column m of L is row m of the
  //    transposed tile, read as broadcasts);
  //  - after a block, every remaining row takes -L[rest, block] X_block on fp32 MFMA
  //    (v_mfma_f32_16x16x4f32), the operands and results passing through a
  //    wave-private LDS area (the wave's own 64 columns: no barrier).
  const bool is_w = tid >= kD;   // waves 2, 3
  const int j = tid & (kD - 1);
  const uint16_t* src = is_w ? sK : sV;
  float x[kC];
  uint32_t kbits[kC / 2];
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const uint32_t bits = src[i * kRowK + j];
    if (i & 1)
      kbits[i >> 1] |= bits << 16;
    else
      kbits[i >> 1] = bits;
    x[i] = (is_w ? sBG[i] : sB[i]) * fd_bf16_to_f32(bits);
  }
  if (is_w) {
    // normalised k^T in the state pass's operand order: row dk = j, the 8 tokens
    // 32st + 8g4 .. +7 of lane 16g4 + (j % 16) (16 lanes write 256 B contiguous);
    // stored before the substitution so that its registers are free there
    uint16_t* kt = a.kn + hc * kC * kD;
    const int kwv = j >> 5, km = (j >> 4) & 1, kc16 = j & 15;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int i = 4 * (4 * st + g);  // kbits index of token 32st + 8g
        *reinterpret_cast<uint4*>(kt + ((((kwv * 2 + km) * 2 + st) * 64) + 16 * g + kc16) * 8) =
            make_uint4(kbits[i], kbits[i + 1], kbits[i + 2], kbits[i + 3]);
      }
  }
  __syncthreads();  // every wave has read its right-hand sides: the q/k/v tiles are free
  float* wl = reinterpret_cast<float*>(smem) + wv * (48 * 64);  // 12 KiB per wave
  uint16_t* gw = a.w + hc * 3 * kC * kD;
  float* gu = a.u + hc * kC * kD;
  // the four blocks, each with its block index a compile-time constant (a loop
  // this size is beyond the unroller's limit)
  auto block = [&](auto bc) __attribute__((always_inline)) {
    constexpr int b = decltype(bc)::value;
    constexpr int b0 = 16 * b;
    // the block's 36 reads of L pieces pass through a window of kTriWin registers,
    // each issued kTriWin steps before its FMAs, so the LDS latency is not paid per
    // read (x[i] still takes its updates in increasing m)
    f32x4_t lwin[kTriWin];
#pragma unroll
    for (int k = 0; k < kTriWin; ++k)
      lwin[k] = *reinterpret_cast<const f32x4_t*>(sL + (b0 + tri_m(k)) * kRowF + b0 + tri_i0(k));
#pragma unroll
    for (int k = 0; k < kTriReads; ++k) {
      const int m = b0 + tri_m(k), i0 = b0 + tri_i0(k);
      const f32x4_t lv = lwin[k % kTriWin];
      const float xm = x[m];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i0 + e > m) x[i0 + e] = fmaf(-lv[e], xm, x[i0 + e]);
      if (k + kTriWin < kTriReads)
        lwin[k % kTriWin] = *reinterpret_cast<const f32x4_t*>(sL + (b0 + tri_m(k + kTriWin)) * kRowF + b0 +
                                                               tri_i0(k + kTriWin));
      __builtin_amdgcn_sched_barrier(0);
    }
    // X_block (16 rows of the wave's 64 columns) -> LDS [16][64]
#pragma unroll
    for (int k = 0; k < 16; ++k) wl[k * 64 + l] = x[b0 + k];
    // These 16 rows of u or w are final: store them now, in the state pass's
    // operand order, so the writes drain while the later blocks run.
    if (is_w) {
      // w piece (row 16b + lane%16, columns 32c + 8(lane/16) .. +7) as three exact bf16 planes;
      // this wave holds the column groups c = 2(wv-2), 2(wv-2)+1
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const int q = (b << 8) | ((2 * (wv - 2) + ch) << 6) | l;
        const float* src_row = wl + (l & 15) * 64 + 32 * ch + 8 * (l >> 4);
        const f32x4_t v0 = *reinterpret_cast<const f32x4_t*>(src_row);
        const f32x4_t v1 = *reinterpret_cast<const f32x4_t*>(src_row + 4);
        const float va[4] = {v0[0], v0[1], v0[2], v0[3]};
        const float vb[4] = {v1[0], v1[1], v1[2], v1[3]};
        uint2 ha, ma, la, hb, mb, lb;
        split3x4(va, ha, ma, la);
        split3x4(vb, hb, mb, lb);
        *reinterpret_cast<uint4*>(gw + q * 8) = make_uint4(ha.x, ha.y, hb.x, hb.y);
        *reinterpret_cast<uint4*>(gw + kC * kD + q * 8) = make_uint4(ma.x, ma.y, mb.x, mb.y);
        *reinterpret_cast<uint4*>(gw + 2 * kC * kD + q * 8) = make_uint4(la.x, la.y, lb.x, lb.y);
      }
    } else {
      // u piece (rows 16b + 4(lane/16) .. +3, column 16g + lane%16) in fp32;
      // this wave holds the column groups g = 4wv .. 4wv+3
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        const int q = ((4 * wv + cg) << 8) | (b << 6) | l;
        const float* src_col = wl + 4 * (l >> 4) * 64 + 16 * cg + (l & 15);
        const f32x4_t v = {src_col[0], src_col[64], src_col[128], src_col[192]};
        *reinterpret_cast<f32x4_t*>(gu + q * 4) = v;
      }
    }
    if constexpr (b == 3) return;
    // C[rest rows][64 columns] = L[rest, block] X_block: rest row tile rt (16 rows), column tile t
    constexpr int kMaxRt = 3;
    const int nrt = 3 - b;
    float bx[4][4];  // B[k = 4s + l/16][n = 16t + l%16]
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int st = 0; st < 4; ++st) bx[t][st] = wl[(4 * st + (l >> 4)) * 64 + 16 * t + (l & 15)];
    f32x4_t acc[kMaxRt][4];
#pragma unroll
    for (int rt = 0; rt < kMaxRt; ++rt) {
      if (rt >= nrt) break;
      float al[4];  // A[i = l%16][k = l/16 + 4s] = L[b0 + 16 + 16rt + l%16][b0 + 4s + l/16]
#pragma unroll
      for (int st = 0; st < 4; ++st) al[st] = sL[(b0 + 4 * st + (l >> 4)) * kRowF + b0 + 16 + 16 * rt + (l & 15)];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc[rt][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; ++st) acc[rt][t] = mfma_f32(al[st], bx[t][st], acc[rt][t]);
      }
    }
    // C -> LDS [rest rows][64], then every lane subtracts its own column
#pragma unroll
    for (int rt = 0; rt < kMaxRt; ++rt) {
      if (rt >= nrt) break;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) wl[(16 * rt + 4 * (l >> 4) + r) * 64 + 16 * t + (l & 15)] = acc[rt][t][r];
    }
#pragma unroll
    for (int i = b0 + 16; i < kC; ++i) x[i] = x[i] - wl[(i - b0 - 16) * 64 + l];
  };
  block(std::integral_constant<int, 0>{});
  block(std::integral_constant<int, 1>{});
  block(std::integral_constant<int, 2>{});
  block(std::integral_constant<int, 3>{});
}

// ---------------------------------------------------------------------------
// 3. sequential state pass over the chunks of one request, with the chunks' outputs
//
// Both products of a chunk run on v_mfma_f32_16x16x32_bf16 with the fp32
// operands split exactly into bf16 planes (x = hi + mid + lo): w S keeps six of
// the nine plane products (hi.hi, hi.mid, mid.hi, hi.lo, mid.mid, lo.hi; the
// rest are below 2^-24 relative), k^T v' (k is a bf16 value) keeps all three.
// The lane layout is that of the fp32 MFMA (A[l%16][k], B[k][l%16],
// D[4(l/16)+r][l%16]) with the 8 consecutive reduction indices 8(l/16)..+7 of
// each 32-step in a lane.
constexpr int kRowSB = kD + 8;   // bf16 row stride of a transposed state plane (272 B)
constexpr int kRowVB = kC + 8;   // bf16 row stride of a transposed v' plane (144 B)

constexpr int kStateThreads = 512;

__global__ __launch_bounds__(kStateThreads) void gd_state_kernel(GdArgs a) {
  // XCD-aware order: block b runs on XCD b % 8; the logical index below gives
  // each XCD a contiguous range, so the 8 column slices of one head (which read
  // the same w / k / q / A tiles) share one L2.  The grid is a multiple of 8.
  const int nb = gridDim.x;
  const int lb = (blockIdx.x % 8) * (nb / 8) + blockIdx.x / 8;
  const int js = lb % kSlices;
  const int h = (lb / kSlices) % a.hv;
  const int sq = lb / (kSlices * a.hv);
  int first, last;
  request_chunks(a, sq, &first, &last);

  __shared__ __attribute__((aligned(16))) uint16_t sS[3][kSlice * kRowSB];   // state planes [col][dk]
  __shared__ __attribute__((aligned(16))) uint16_t sVd[3][kSlice * kRowVB];  // e^{gl - gc} v' planes [col][t]
  __shared__ __attribute__((aligned(16))) uint16_t sVp[3][kSlice * kRowVB];  // v' planes [col][t]

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int g4 = l >> 4;
  const int c16 = l & 15;
  const int col = kSlice * js + c16;  // value column owned in the C layout
  const size_t state_base = (static_cast<size_t>(sq) * a.hv + h) * kD * kD;

  if (wv < 4) {
    // ---- the state chain (wavefront wv: v' rows 16wv .. +15, state rows 32wv .. +31)
    // state slice in the C layout (fp32): S[m][r] = S[dk = 32wv + 16m + 4g4 + r][col]
    float S[2][4];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[m][r] = a.s0 ? a.s0[state_base + static_cast<size_t>(32 * wv + 16 * m + 4 * g4 + r) * kD + col] : 0.0f;

    // operands of one chunk, loaded straight into registers two chunks ahead;
    // three register sets rotate (the loop body is unrolled by three) and every
    // load is issued unconditionally (past the last chunk it re-reads the last one)
    struct ChunkRegs {
      uint4 w[3][4];  // plane x, step s: w_x[16wv + c16][32s + 8g4 .. +7]      (A of w S)
      uint4 k[2][2];  // tile m, step s: k^T[32wv + 16m + c16][32s + 8g4 .. +7]  (A of k^T v')
      float u[4];     // u[16wv + 4g4 + r][col]                                 (C layout)
      f32x4_t dec;    // e^{gl - gc_t}, t = 16wv + 4g4 .. +3
      float egl;      // e^{gl}
    };
    // Part `part` of the operand loads of chunk c: parts 0-2 are the w planes,
    // part 3 k^T, u and the exponentials; -1 loads all of them.
    auto load_chunk = [&](ChunkRegs& R, int c, int part = -1) {
      c = min(c, last - 1);
      const size_t hc = static_cast<size_t>(h) * a.nc + c;
      const uint16_t* w = a.w + hc * 3 * kC * kD + (wv * 4 * 64 + l) * 8;
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        if (part >= 0 && part != x) continue;
#pragma unroll
        for (int st = 0; st < 4; ++st) R.w[x][st] = *reinterpret_cast<const uint4*>(w + x * kC * kD + st * 64 * 8);
      }
      if (part >= 0 && part != 3) return;
      const uint16_t* kt = a.kn + hc * kC * kD + (wv * 4 * 64 + l) * 8;
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int st = 0; st < 2; ++st) R.k[m][st] = *reinterpret_cast<const uint4*>(kt + (m * 2 + st) * 64 * 8);
      const f32x4_t u4 = *reinterpret_cast<const f32x4_t*>(a.u + hc * kC * kD + ((js * 4 + wv) * 64 + l) * 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) R.u[r] = u4[r];
      const float* gx = a.gc + hc * 3 * kC;
      R.dec = *reinterpret_cast<const f32x4_t*>(gx + kC + 16 * wv + 4 * g4);
      R.egl = gx[2 * kC];
    };

    // One chunk.  The loads of chunk cp (two ahead) into P go out in four parts,
    // each where the wavefront waits anyway (before a barrier, behind an issued
    // MFMA group): the address unit takes about 16 cycles per 1 KiB load per CU,
    // and one burst of all 19 would stall the in-order wavefront for most of a
    // step.  sched_barrier keeps each part in place.
    auto step = [&](const ChunkRegs& R, int c, ChunkRegs& P, int cp) {
      // state at the chunk start: bf16 planes to LDS (B of w S and of the output's q S)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int dk = 32 * wv + 16 * m + 4 * g4;
        uint2 ph, pm, pl;
        split3x4(S[m], ph, pm, pl);
        *reinterpret_cast<uint2*>(sS[0] + c16 * kRowSB + dk) = ph;
        *reinterpret_cast<uint2*>(sS[1] + c16 * kRowSB + dk) = pm;
        *reinterpret_cast<uint2*>(sS[2] + c16 * kRowSB + dk) = pl;
      }
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(P, cp, 0);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();

      // v' = u - w S for rows 16wv..16wv+15 of this slice
      f32x4_t acc0 = {};
      f32x4_t acc1 = {};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int off = c16 * kRowSB + 32 * st + 8 * g4;
        const uint4 sh = *reinterpret_cast<const uint4*>(sS[0] + off);
        const uint4 sm = *reinterpret_cast<const uint4*>(sS[1] + off);
        const uint4 sl = *reinterpret_cast<const uint4*>(sS[2] + off);
        acc0 = mfma_bf16(R.w[0][st], sh, acc0);
        acc1 = mfma_bf16(R.w[0][st], sm, acc1);
        acc0 = mfma_bf16(R.w[1][st], sh, acc0);
        acc1 = mfma_bf16(R.w[0][st], sl, acc1);
        acc0 = mfma_bf16(R.w[1][st], sm, acc0);
        acc1 = mfma_bf16(R.w[2][st], sh, acc1);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(P, cp, 1);
      __builtin_amdgcn_sched_barrier(0);
      f32x4_t vnew;
      float vdec[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vnew[r] = R.u[r] - (acc0[r] + acc1[r]);
        vdec[r] = vnew[r] * R.dec[r];
      }
      {
        const int off = c16 * kRowVB + 16 * wv + 4 * g4;
        uint2 ph, pm, pl;
        split3x4(vdec, ph, pm, pl);
        *reinterpret_cast<uint2*>(sVd[0] + off) = ph;
        *reinterpret_cast<uint2*>(sVd[1] + off) = pm;
        *reinterpret_cast<uint2*>(sVd[2] + off) = pl;
        // v'[t][col] planes for the output wavefronts
        const float vv[4] = {vnew[0], vnew[1], vnew[2], vnew[3]};
        split3x4(vv, ph, pm, pl);
        *reinterpret_cast<uint2*>(sVp[0] + off) = ph;
        *reinterpret_cast<uint2*>(sVp[1] + off) = pm;
        *reinterpret_cast<uint2*>(sVp[2] + off) = pl;
      }
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(P, cp, 2);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();

      // S <- e^{gl} S + k^T (e^{gl - gc} v'), dk rows 32wv..32wv+31
      f32x4_t st0 = {S[0][0] * R.egl, S[0][1] * R.egl, S[0][2] * R.egl, S[0][3] * R.egl};
      f32x4_t st1 = {S[1][0] * R.egl, S[1][1] * R.egl, S[1][2] * R.egl, S[1][3] * R.egl};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int off = c16 * kRowVB + 32 * st + 8 * g4;
        const uint4 dh = *reinterpret_cast<const uint4*>(sVd[0] + off);
        const uint4 dm = *reinterpret_cast<const uint4*>(sVd[1] + off);
        const uint4 dl = *reinterpret_cast<const uint4*>(sVd[2] + off);
        st0 = mfma_bf16(R.k[0][st], dh, st0);
        st1 = mfma_bf16(R.k[1][st], dh, st1);
        st0 = mfma_bf16(R.k[0][st], dm, st0);
        st1 = mfma_bf16(R.k[1][st], dm, st1);
        st0 = mfma_bf16(R.k[0][st], dl, st0);
        st1 = mfma_bf16(R.k[1][st], dl, st1);
      }
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(P, cp, 3);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        S[0][r] = st0[r];
        S[1][r] = st1[r];
      }
      // no third barrier: the next writes of sS follow this step's second
      // barrier, and the next writes of sVd and sVp follow the next step's first
    };

    if (first < last) {
      ChunkRegs A, B, Cr;
      load_chunk(A, first);
      load_chunk(B, first + 1);
      for (int c = first; c < last; c += 3) {
        step(A, c, Cr, c + 2);
        if (c + 1 < last) step(B, c + 1, A, c + 3);
        if (c + 2 < last) step(Cr, c + 2, B, c + 4);
      }
    }

    if (a.sN != nullptr) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          a.sN[state_base + static_cast<size_t>(32 * wv + 16 * m + 4 * g4 + r) * kD + col] = S[m][r];
    }
  } else {
    // ---- the chunk outputs (wavefront wv: rows 16rt .. +15 of every chunk)
    //   o[t][col] = scale e^{gc_t} (q S_chunk)[t][col] + (A v')[t][col]
    // q S takes the three products of the bf16 q with the state planes the
    // chain wrote; A v' six of the nine plane products of exact three-plane
    // splits of the fp32 A and v'.
    const int rt = wv - 4;
    const size_t o_row = static_cast<size_t>(a.hv) * kD;
    struct OutRegs {
      uint4 q[4];       // q[16rt + c16][32st + 8g4 .. +7]
      f32x4_t av[2][2];  // A[16rt + c16][32st + 8g4 + 4i .. +3]
      f32x4_t eg;       // e^{gc_t}, t = 16rt + 4g4 .. +3
    };
    auto load_out = [&](OutRegs& R, int c) {
      c = min(c, last - 1);
      const size_t hc = static_cast<size_t>(h) * a.nc + c;
      const uint16_t* qp = a.qn + hc * kC * kD + (rt * 4 * 64 + l) * 8;
#pragma unroll
      for (int st = 0; st < 4; ++st) R.q[st] = *reinterpret_cast<const uint4*>(qp + st * 64 * 8);
      const float* ap = a.aq + hc * kC * kC + (rt * 2 * 64 + l) * 8;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        R.av[st][0] = *reinterpret_cast<const f32x4_t*>(ap + st * 64 * 8);
        R.av[st][1] = *reinterpret_cast<const f32x4_t*>(ap + st * 64 * 8 + 4);
      }
      R.eg = *reinterpret_cast<const f32x4_t*>(a.gc + hc * 3 * kC + 16 * rt + 4 * g4);
    };
    auto split8v = [](f32x4_t v0, f32x4_t v1, uint4& hi, uint4& mid, uint4& lo) {
      const float va[4] = {v0[0], v0[1], v0[2], v0[3]};
      const float vb[4] = {v1[0], v1[1], v1[2], v1[3]};
      uint2 ha, ma, la, hb, mb, lb;
      split3x4(va, ha, ma, la);
      split3x4(vb, hb, mb, lb);
      hi = make_uint4(ha.x, ha.y, hb.x, hb.y);
      mid = make_uint4(ma.x, ma.y, mb.x, mb.y);
      lo = make_uint4(la.x, la.y, lb.x, lb.y);
    };
    // the barriers match the chain's step: the first finds the chunk-start
    // state planes in sS, the second the v' planes in sVp
    auto out_step = [&](const OutRegs& R, int c, OutRegs& P, int cp) {
      __syncthreads();
      // the chain's operand reads of the state planes go first: the A split and
      // the next chunk's loads (no LDS) come before this wavefront's own reads
      uint4 ah[2], am[2], al[2];
      split8v(R.av[0][0], R.av[0][1], ah[0], am[0], al[0]);
      load_out(P, cp);
      __builtin_amdgcn_sched_barrier(0);
      f32x4_t acc1 = {};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int off = c16 * kRowSB + 32 * st + 8 * g4;
        const uint4 sh = *reinterpret_cast<const uint4*>(sS[0] + off);
        const uint4 sm = *reinterpret_cast<const uint4*>(sS[1] + off);
        const uint4 sl = *reinterpret_cast<const uint4*>(sS[2] + off);
        acc1 = mfma_bf16(R.q[st], sh, acc1);
        acc1 = mfma_bf16(R.q[st], sm, acc1);
        acc1 = mfma_bf16(R.q[st], sl, acc1);
      }
      __syncthreads();
      // likewise the chain's reads of the e^{gl - gc} v' planes go first
      split8v(R.av[1][0], R.av[1][1], ah[1], am[1], al[1]);
      __builtin_amdgcn_sched_barrier(0);
      f32x4_t acc2 = {};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int off = c16 * kRowVB + 32 * st + 8 * g4;
        const uint4 b0 = *reinterpret_cast<const uint4*>(sVp[0] + off);
        const uint4 b1 = *reinterpret_cast<const uint4*>(sVp[1] + off);
        const uint4 b2 = *reinterpret_cast<const uint4*>(sVp[2] + off);
        acc2 = mfma_bf16(ah[st], b0, acc2);
        acc2 = mfma_bf16(ah[st], b1, acc2);
        acc2 = mfma_bf16(am[st], b0, acc2);
        acc2 = mfma_bf16(ah[st], b2, acc2);
        acc2 = mfma_bf16(am[st], b1, acc2);
        acc2 = mfma_bf16(al[st], b0, acc2);
      }
      int r0, L;
      chunk_rows(a, c, &r0, &L);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * g4 + r;
        if (t < L) {
          const float val = (a.scale * R.eg[r]) * acc1[r] + acc2[r];
          a.o[static_cast<size_t>(r0 + t) * o_row + h * kD + col] = static_cast<uint16_t>(fd_pack2(val, 0.0f));
        }
      }
    };

    if (first < last) {
      OutRegs A, B, Cr;
      load_out(A, first);
      load_out(B, first + 1);
      for (int c = first; c < last; c += 3) {
        out_step(A, c, Cr, c + 2);
        if (c + 1 < last) out_step(B, c + 1, A, c + 3);
        if (c + 2 < last) out_step(Cr, c + 2, B, c + 4);
      }
    }
  }
}

// Byte offsets of the workspace regions: the chunk table, the per-(head, chunk)
// intermediates GdArgs describes, and `ob`, the raw bf16 output rows
// [tokens, Hv, 128] that the gated norm reads (fd_gated_delta_norm_fwd only).
struct GdLayout {
  size_t row0, len, first, gc, qn, kn, w, u, aq, ob, total;
};

GdLayout gd_layout(int64_t nc, int64_t hv, int64_t nseq, int64_t tokens) {
  auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  const size_t hc = static_cast<size_t>(hv) * static_cast<size_t>(nc);
  GdLayout L;
  size_t off = 0;
  L.row0 = off;
  off = al(off + static_cast<size_t>(nc) * 4);
  L.len = off;
  off = al(off + static_cast<size_t>(nc) * 4);
  L.first = off;
  off = al(off + static_cast<size_t>(nseq + 1) * 4);
  L.gc = off;
  off = al(off + hc * 3 * kC * 4);
  L.qn = off;
  off = al(off + hc * kC * kD * 2);
  L.kn = off;
  off = al(off + hc * kC * kD * 2);
  L.w = off;
  off = al(off + hc * 3 * kC * kD * 2);
  L.u = off;
  off = al(off + hc * kC * kD * 4);
  L.aq = off;
  off = al(off + hc * kC * kC * 4);
  L.ob = off;
  off = al(off + static_cast<size_t>(tokens) * hv * kD * 2);
  L.total = off;
  return L;
}

// chunks and requests of a launch; false if the sizes are out of range
bool gd_counts(int batch, int seq_len, int n_seqs, bool varlen, int64_t* nc, int64_t* nseq) {
  if (batch < 0 || seq_len < 0) return false;
  const int64_t total = static_cast<int64_t>(batch) * seq_len;
  if (total >= (1LL << 31)) return false;
  if (varlen) {
    if (n_seqs < 1 || batch != 1) return false;
    *nseq = n_seqs;
    *nc = (total + kC - 1) / kC + n_seqs;
  } else {
    *nseq = batch;
    *nc = static_cast<int64_t>(batch) * ((seq_len + kC - 1) / kC);
  }
  return true;
}

}  // namespace

extern "C" FD_API int64_t fd_gated_delta_workspace_bytes(int batch, int seq_len, int v_heads, int head_k_dim,
                                                         int head_v_dim, int n_seqs) {
  if (v_heads <= 0 || head_k_dim != kD || head_v_dim != kD) return FD_ERR_UNSUPPORTED;
  int64_t nc = 0, nseq = 0;
  if (!gd_counts(batch, seq_len, n_seqs, n_seqs > 0, &nc, &nseq)) return FD_ERR_INVALID_ARGUMENT;
  return static_cast<int64_t>(gd_layout(nc, v_heads, nseq, static_cast<int64_t>(batch) * seq_len).total);
}

namespace {

struct GdNorm {
  const void* z;
  int64_t z_ts, z_hs;
  const void* w;
  int w_dtype;
  float eps;
};

int gd_run(const void* q, const void* k, const void* v, const float* g, const void* beta, void* out,
           const float* initial_state, float* final_state, void* workspace, int64_t workspace_bytes, int batch,
           int seq_len, int k_heads, int v_heads, int head_k_dim, int head_v_dim, float scale, int beta_dtype,
           int l2norm_qk, const int32_t* cu_seqlens, int n_seqs, void* stream, const GdNorm* norm) {
  FD_REQUIRE(q && k && v && g && beta && out && workspace, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: q, k, v, g, beta, out and workspace must be non-null");
  FD_REQUIRE(k_heads > 0 && v_heads > 0 && v_heads % k_heads == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: v_heads (%d) must be a positive multiple of k_heads (%d)", v_heads, k_heads);
  FD_REQUIRE(head_k_dim == kD && head_v_dim == kD, FD_ERR_UNSUPPORTED,
             "fd_gated_delta_fwd: head_k_dim and head_v_dim must be 128 (got %d, %d)", head_k_dim, head_v_dim);
  FD_REQUIRE(beta_dtype == FD_DTYPE_BF16 || beta_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: beta_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  FD_REQUIRE(scale > 0.0f && scale < 1e30f, FD_ERR_INVALID_ARGUMENT, "fd_gated_delta_fwd: scale must be positive");
  FD_REQUIRE(fd_aligned16(q) && fd_aligned16(k) && fd_aligned16(v) && fd_aligned16(out) && fd_aligned16(workspace),
             FD_ERR_ALIGNMENT, "fd_gated_delta_fwd: q, k, v, out and workspace must be 16-byte aligned");
  FD_REQUIRE((reinterpret_cast<uintptr_t>(g) & 3u) == 0 && (reinterpret_cast<uintptr_t>(beta) & 1u) == 0 &&
                 (beta_dtype != FD_DTYPE_F32 || (reinterpret_cast<uintptr_t>(beta) & 3u) == 0),
             FD_ERR_ALIGNMENT, "fd_gated_delta_fwd: g and beta must be aligned to their element size");
  const bool varlen = cu_seqlens != nullptr;
  if (varlen) {
    FD_REQUIRE(batch == 1, FD_ERR_INVALID_ARGUMENT, "fd_gated_delta_fwd: cu_seqlens requires batch == 1 (got %d)",
               batch);
    FD_REQUIRE(n_seqs >= 1, FD_ERR_INVALID_ARGUMENT, "fd_gated_delta_fwd: n_seqs must be >= 1 with cu_seqlens");
  }
  int64_t nc = 0, nseq = 0;
  FD_REQUIRE(gd_counts(batch, seq_len, n_seqs, varlen, &nc, &nseq), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: batch and seq_len must be >= 0 with batch * seq_len < 2^31");
  FD_REQUIRE(nc * v_heads < (1LL << 31) && nseq * v_heads * kSlices < (1LL << 31), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: problem too large");
  if (nseq == 0) return FD_OK;  // empty batch: nothing to launch
  const int64_t total = static_cast<int64_t>(batch) * seq_len;
  // the gated norm runs over total * v_heads rows (checked here so nothing is launched if it cannot)
  FD_REQUIRE(norm == nullptr || total * v_heads < (1LL << 31), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_norm_fwd: problem too large (batch * seq_len * v_heads must be < 2^31)");
  const GdLayout lay = gd_layout(nc, v_heads, nseq, total);
  FD_REQUIRE(workspace_bytes >= static_cast<int64_t>(lay.total), FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_fwd: workspace too small (%lld bytes, need %lld)",
             static_cast<long long>(workspace_bytes), static_cast<long long>(lay.total));

  unsigned char* ws = static_cast<unsigned char*>(workspace);
  GdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.g = g;
  a.beta = beta;
  // with the gated norm the raw output rows go to the workspace and the norm writes `out`
  a.o = norm ? reinterpret_cast<uint16_t*>(ws + lay.ob) : static_cast<uint16_t*>(out);
  a.s0 = initial_state;
  a.sN = final_state;
  a.row0 = reinterpret_cast<int32_t*>(ws + lay.row0);
  a.len = reinterpret_cast<int32_t*>(ws + lay.len);
  a.first = reinterpret_cast<int32_t*>(ws + lay.first);
  a.gc = reinterpret_cast<float*>(ws + lay.gc);
  a.qn = reinterpret_cast<uint16_t*>(ws + lay.qn);
  a.kn = reinterpret_cast<uint16_t*>(ws + lay.kn);
  a.w = reinterpret_cast<uint16_t*>(ws + lay.w);
  a.u = reinterpret_cast<float*>(ws + lay.u);
  a.aq = reinterpret_cast<float*>(ws + lay.aq);
  a.hk = k_heads;
  a.hv = v_heads;
  a.nc = static_cast<int>(nc);
  a.nseq = static_cast<int>(nseq);
  a.varlen = varlen;
  a.seq_len = seq_len;
  a.nct = (seq_len + kC - 1) / kC;
  a.beta_f32 = beta_dtype == FD_DTYPE_F32;
  a.l2norm = l2norm_qk != 0;
  a.scale = scale;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (varlen)
    hipLaunchKernelGGL(gd_chunk_table, dim3(1), dim3(kThreads), 0, s, cu_seqlens, a.nseq, seq_len,
                       static_cast<int>(total), a);
  if (nc > 0) {
    if (a.beta_f32)
      hipLaunchKernelGGL(gd_prep_kernel<true>, dim3(static_cast<unsigned>(nc * v_heads)), dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL(gd_prep_kernel<false>, dim3(static_cast<unsigned>(nc * v_heads)), dim3(kThreads), 0, s, a);
  }
  hipLaunchKernelGGL(gd_state_kernel, dim3(static_cast<unsigned>(nseq * v_heads * kSlices)), dim3(kStateThreads), 0,
                     s, a);
  const int rc = fd_check_launch("fd_gated_delta_fwd");
  if (rc != FD_OK || norm == nullptr || total == 0) return rc;
  // the layer's gated RMSNorm over the raw output rows (one row per token and value head)
  return fd_gated_rmsnorm_fwd(a.o, norm->z, norm->z_ts, norm->z_hs, v_heads, norm->w, norm->w_dtype, out,
                              total * v_heads, kD, norm->eps, stream);
}

}  // namespace

// ---------------------------------------------------------------------------
// Static device scratch of fd_gated_delta_fwd_noalloc: the workspace of callers
// that cannot allocate (HIP graph capture, serving loops).  Every GPU the
// library runs on holds its own copy for the life of the process.  Host code
// never passes `scratch` itself to a kernel (in host code the name is a
// host-side stand-in, not a device address): it uses the address that
// hipGetSymbolAddress returns once per device.
static __device__ __align__(256) unsigned char scratch[FD_GD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current
// device for the null stream), looked up on that device's first call.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream != nullptr) {
    FD_REQUIRE(hipStreamGetDevice(stream, &dev) == hipSuccess, FD_ERR_LAUNCH,
               "fd_gated_delta_fwd_noalloc: cannot query the stream's device");
  } else {
    FD_REQUIRE(hipGetDevice(&dev) == hipSuccess, FD_ERR_LAUNCH, "fd_gated_delta_fwd_noalloc: no current device");
  }
  FD_REQUIRE(dev >= 0 && dev < kMaxDevices, FD_ERR_UNSUPPORTED, "fd_gated_delta_fwd_noalloc: device %d out of range",
             dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    FD_REQUIRE(hipGetDevice(&cur) == hipSuccess, FD_ERR_LAUNCH, "fd_gated_delta_fwd_noalloc: no current device");
    if (cur != dev) FD_REQUIRE(hipSetDevice(dev) == hipSuccess, FD_ERR_LAUNCH,
                               "fd_gated_delta_fwd_noalloc: cannot select device %d", dev);
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    FD_REQUIRE(err == hipSuccess && p != nullptr, FD_ERR_LAUNCH,
               "fd_gated_delta_fwd_noalloc: hipGetSymbolAddress of the scratch failed: %s", hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FD_OK;
}

}  // namespace

extern "C" FD_API int fd_gated_delta_fwd(const void* q, const void* k, const void* v, const float* g,
                                         const void* beta, void* out, const float* initial_state,
                                         float* final_state, void* workspace, int64_t workspace_bytes, int batch,
                                         int seq_len, int k_heads, int v_heads, int head_k_dim, int head_v_dim,
                                         float scale, int beta_dtype, int l2norm_qk, const int32_t* cu_seqlens,
                                         int n_seqs, void* stream) {
  return gd_run(q, k, v, g, beta, out, initial_state, final_state, workspace, workspace_bytes, batch, seq_len,
                k_heads, v_heads, head_k_dim, head_v_dim, scale, beta_dtype, l2norm_qk, cu_seqlens, n_seqs, stream,
                nullptr);
}

extern "C" FD_API int fd_gated_delta_norm_fwd(const void* q, const void* k, const void* v, const float* g,
                                              const void* beta, const void* z, int64_t z_token_stride,
                                              int64_t z_head_stride, const void* norm_weight, int norm_weight_dtype,
                                              float norm_eps, void* out, const float* initial_state,
                                              float* final_state, void* workspace, int64_t workspace_bytes,
                                              int batch, int seq_len, int k_heads, int v_heads, int head_k_dim,
                                              int head_v_dim, float scale, int beta_dtype, int l2norm_qk,
                                              const int32_t* cu_seqlens, int n_seqs, void* stream) {
  FD_REQUIRE(z && norm_weight, FD_ERR_INVALID_ARGUMENT, "fd_gated_delta_norm_fwd: z and norm_weight must be non-null");
  FD_REQUIRE(norm_weight_dtype == FD_DTYPE_BF16 || norm_weight_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_gated_delta_norm_fwd: norm_weight_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  FD_REQUIRE(norm_eps >= 0.0f, FD_ERR_INVALID_ARGUMENT, "fd_gated_delta_norm_fwd: norm_eps must be >= 0");
  FD_REQUIRE(fd_aligned16(z) && z_token_stride % 8 == 0 && z_head_stride % 8 == 0 && z_head_stride >= kD &&
                 z_token_stride >= static_cast<int64_t>(v_heads) * z_head_stride,
             FD_ERR_ALIGNMENT,
             "fd_gated_delta_norm_fwd: z must be 16-byte aligned with strides that are multiples of 8 covering "
             "[v_heads, 128]");
  FD_REQUIRE((reinterpret_cast<uintptr_t>(norm_weight) & (norm_weight_dtype == FD_DTYPE_F32 ? 3u : 1u)) == 0,
             FD_ERR_ALIGNMENT, "fd_gated_delta_norm_fwd: norm_weight must be aligned to its element size");
  const GdNorm norm{z, z_token_stride, z_head_stride, norm_weight, norm_weight_dtype, norm_eps};
  return gd_run(q, k, v, g, beta, out, initial_state, final_state, workspace, workspace_bytes, batch, seq_len,
                k_heads, v_heads, head_k_dim, head_v_dim, scale, beta_dtype, l2norm_qk, cu_seqlens, n_seqs, stream,
                &norm);
}

extern "C" FD_API int fd_gated_delta_fwd_noalloc(const void* q, const void* k, const void* v, const float* g,
                                                 const void* beta, void* out, const float* initial_state,
                                                 float* final_state, int batch, int seq_len, int k_heads,
                                                 int v_heads, int head_k_dim, int head_v_dim, float scale,
                                                 int beta_dtype, int l2norm_qk, const int32_t* cu_seqlens,
                                                 int n_seqs, void* stream) {
  const int64_t need = fd_gated_delta_workspace_bytes(batch, seq_len, v_heads, head_k_dim, head_v_dim,
                                                      cu_seqlens != nullptr ? n_seqs : 0);
  if (need < 0) {
    return fd_set_error(static_cast<int>(need), "fd_gated_delta_fwd_noalloc: unsupported sizes (batch %d, seq_len %d, "
                        "v_heads %d, head dims %d/%d, n_seqs %d)", batch, seq_len, v_heads, head_k_dim, head_v_dim,
                        n_seqs);
  }
  FD_REQUIRE(need <= FD_GD_SCRATCH_BYTES, FD_ERR_UNSUPPORTED,
             "fd_gated_delta_fwd_noalloc: these sizes need %lld bytes of workspace, more than the %lld-byte "
             "static scratch (call fd_gated_delta_fwd with a workspace instead)",
             static_cast<long long>(need), static_cast<long long>(FD_GD_SCRATCH_BYTES));
  void* ws = nullptr;
  const int rc = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (rc != FD_OK) return rc;
  return gd_run(q, k, v, g, beta, out, initial_state, final_state, ws, FD_GD_SCRATCH_BYTES, batch, seq_len, k_heads,
                v_heads, head_k_dim, head_v_dim, scale, beta_dtype, l2norm_qk, cu_seqlens, n_seqs, stream, nullptr);
}

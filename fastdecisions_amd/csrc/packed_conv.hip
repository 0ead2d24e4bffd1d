// Packed causal depthwise conv1d + SiLU with a head-split q/k/v store, gfx950.
//
// Replaces the reference's hand-edited Inductor pointwise kernel
// (ref: src/decider/packed_conv_kernel.py:115-191), which reads x [B*T, C]
// token-major and stores straight into q/k/v [B, T, H, D].
//
// HBM-bound, no MFMA.  A thread owns 2 contiguous channels (one 4-byte
// access) and a run of RUN consecutive tokens.  The causal window of the last
// WIDTH-1 inputs stays in registers, so each input vector is loaded from HBM
// once; only the WIDTH-1 halo rows in front of a run are read a second time
// (from L2: the neighbouring run is mapped to the same XCD, see below).  A
// wavefront covers 128 channels = 256 B contiguous per token row, for both the
// loads and the stores (2 full 128-byte lines).  Each input row is widened to
// fp64 once, into a ring of WIDTH rows, and serves the WIDTH outputs that use it.
//
// Occupancy, not the access width, sets how much of the arithmetic hides under
// the transfers (B=1, T=2048, C=6144; the loads and stores alone take about
// 10.7 us): 2 channels per thread need 51 VGPRs, so 8 wavefronts share a SIMD,
// and took 13.6 us; 4 channels (8-byte accesses, 89 VGPRs, 5 wavefronts per
// SIMD) took 14.7 us, 8 channels (16-byte, 152 VGPRs, 3 per SIMD) 15.8 us.
//
// XCD-aware block order: the hardware deals workgroups round-robin over the 8
// XCDs, so block b runs on XCD b % 8.  Token runs are renumbered so that each
// XCD receives one contiguous range of runs; the halo rows a run re-reads
// were loaded by its predecessor into the same XCD's L2.
//
// Arithmetic per output, chosen to equal PyTorch's fp32 GPU path
// (silu(conv1d(x.float(), w.float())) then one cast) bit for bit:
//   y = fp32(exact sum of the W products w[j]*x[t-W+1+j]): the products of two
//       bf16 values are exact, and their sum is accumulated in fp64 from +0 in
//       tap order, which is exact for any 4 such products short of an
//       exponent spread beyond 2^37; one rounding to fp32 (MIOpen's
//       depthwise conv accumulates in fp64 and rounds once: measured equal on
//       every output of the config-2 tensor, where every fp32 tap order
//       differs on 0.3 % of them);
//   (+ bias, one fp32 add), then y / (1 + expf(-y)) for SiLU, one bf16 rounding
//   (fd_silu_bf16: the hardware exp2 and reciprocal wherever they round to the
//   same bf16, which fd_silu_check confirms for every fp32 input).
// The taps are the reference's (ref: :139-177): w[W-1] multiplies x[t], w[j]
// multiplies x[t-W+1+j], taps before the sequence start are zero.
#include "fd_common.h"
#include "gate_proj_body.h"

namespace {

constexpr int kThreads = 256;
constexpr int kNumXcd = 8;
constexpr int kCh = 2;  // channels per thread: one 4-byte pair of bf16

__device__ __forceinline__ uint32_t load4(const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// The 2 bf16 of a 4-byte pair as doubles (exact), element e = channel c0 + e.
// The empty asm pins each widened value in registers: without it the compiler
// re-derives the conversions at every one of the WIDTH outputs that use a value.
__device__ __forceinline__ void widen2(const uint32_t raw, double (&d)[kCh]) {
  d[0] = static_cast<double>(fd_lo(raw));
  d[1] = static_cast<double>(fd_hi(raw));
#pragma unroll
  for (int e = 0; e < kCh; ++e) asm volatile("" : "+v"(d[e]));
}

// Grid: 1-D, n_col * n_runs_padded blocks (a multiple of 8).  Linear block b
// runs on XCD b % 8; logical block L = (b % 8) * (nblocks / 8) + b / 8, so the
// logical blocks of one XCD are contiguous: all channel columns of a run, then
// the next run.
struct ConvArgs {
  const uint16_t* x;     // [total_rows, C] bf16, row stride x_row elements
  const uint16_t* w;     // [C, WIDTH] bf16
  const uint16_t* bias;  // [C] bf16 or null
  uint16_t* q;           // [total_rows, key_dim]
  uint16_t* k;           // [total_rows, key_dim]
  uint16_t* v;           // [total_rows, value_dim]
  int64_t x_row;
  int total_rows, seq_len, key_dim, value_dim;
  const int32_t* cu_seqlens;  // [n_seqs + 1] or null
  int n_seqs, n_runs, n_col;
};

// The conv work of linear block `lin` of `nblocks` (a multiple of 8).
template <int WIDTH, int RUN, bool SILU, bool HAS_BIAS>
__device__ __forceinline__ void conv_block(int lin, int nblocks, const ConvArgs& a) {
  const uint16_t* __restrict__ x = a.x;
  const uint16_t* __restrict__ w = a.w;
  const uint16_t* __restrict__ bias = a.bias;
  uint16_t* __restrict__ q = a.q;
  uint16_t* __restrict__ k = a.k;
  uint16_t* __restrict__ v = a.v;
  const int64_t x_row = a.x_row;
  const int total_rows = a.total_rows, seq_len = a.seq_len, key_dim = a.key_dim, value_dim = a.value_dim;
  const int32_t* __restrict__ cu_seqlens = a.cu_seqlens;
  const int n_seqs = a.n_seqs, n_runs = a.n_runs, n_col = a.n_col;
  const int C = 2 * key_dim + value_dim;
  const int logical = (lin % kNumXcd) * (nblocks / kNumXcd) + lin / kNumXcd;
  const int run = logical / n_col;
  const int chunk = (logical % n_col) * kThreads + threadIdx.x;  // kCh-channel chunk
  if (run >= n_runs || chunk * kCh >= C) return;
  const int c0 = chunk * kCh;
  const int r0 = run * RUN;

  // Per-channel taps in fp64 (exact: every bf16 value is a double); tap
  // WIDTH-1 multiplies the current token.
  double wd[WIDTH][kCh];
  if (WIDTH == 4) {
    const uint4 t = *reinterpret_cast<const uint4*>(w + c0 * 4);  // 2 channels x 4 taps = 16 B
    const uint32_t u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < kCh; ++e) {
      wd[0][e] = fd_lo(u[2 * e]);
      wd[1][e] = fd_hi(u[2 * e]);
      wd[2][e] = fd_lo(u[2 * e + 1]);
      wd[3][e] = fd_hi(u[2 * e + 1]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kCh; ++e) {
#pragma unroll
      for (int j = 0; j < WIDTH; ++j) wd[j][e] = fd_bf16_to_f32(w[(c0 + e) * WIDTH + j]);
    }
  }
  float bs[kCh];
  if (HAS_BIAS) {
    const uint32_t b = load4(bias + c0);
    bs[0] = fd_lo(b);
    bs[1] = fd_hi(b);
  }

  // Sequence containing r0: [seg_start, seg_end).  For varlen, seg is the
  // largest index in [0, n_seqs) with cu_seqlens[seg] <= r0; the offsets are
  // clamped to [0, total_rows] so a malformed table cannot move an access
  // outside x or the outputs.
  int seg = 0, seg_start, seg_end;
  if (cu_seqlens != nullptr) {
    int lo = 0, hi = n_seqs;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu_seqlens[mid] <= r0) lo = mid; else hi = mid;
    }
    seg = lo;
    seg_start = min(max(cu_seqlens[seg], 0), total_rows);
    seg_end = min(max(cu_seqlens[seg + 1], 0), total_rows);
  } else {
    seg_start = (r0 / seq_len) * seq_len;
    seg_end = seg_start + seq_len;
  }

  uint16_t* dst;
  int dst_stride, dst_c;
  if (c0 < key_dim) {
    dst = q; dst_stride = key_dim; dst_c = c0;
  } else if (c0 < 2 * key_dim) {
    dst = k; dst_stride = key_dim; dst_c = c0 - key_dim;
  } else {
    dst = v; dst_stride = value_dim; dst_c = c0 - 2 * key_dim;
  }
  const uint16_t* __restrict__ xc = x + c0;

  // The outputs of one row from the window rows win[0..WIDTH-1] (oldest
  // first): exact tap sums rounded once to fp32, bias, activation, one
  // 4-byte store of the bf16 results.  The fast SiLU runs on every lane;
  // the exact expression only where fd_silu_bf16's test sends it.
  auto row_out = [&](const double* const (&win)[WIDTH], int r) {
    float y[kCh];
#pragma unroll
    for (int e = 0; e < kCh; ++e) {
      double acc = 0.0;  // from +0, so an exact zero sum is +0 whatever the signs of the products
#pragma unroll
      for (int j = 0; j < WIDTH; ++j) acc = __builtin_fma(wd[j][e], win[j][e], acc);
      float t = static_cast<float>(acc);
      if (HAS_BIAS) t = t + bs[e];
      y[e] = SILU ? fd_silu_bf16(t) : t;
    }
    *reinterpret_cast<uint32_t*>(dst + static_cast<int64_t>(r) * dst_stride + dst_c) = fd_pack2(y[0], y[1]);
  };

  if (r0 + RUN <= seg_end && r0 + RUN <= total_rows) {
    // The whole run lies in one sequence (the usual case).  Every load is
    // issued up front: WIDTH-1 halo rows (zero before the sequence start) +
    // RUN rows.  Each row is widened to fp64 once, into a ring of WIDTH rows
    // (row m in slot m % WIDTH); every index below is static after unrolling.
    uint32_t raw[WIDTH - 1 + RUN];
#pragma unroll
    for (int m = 0; m < WIDTH - 1 + RUN; ++m) {
      const int r = r0 - (WIDTH - 1) + m;
      raw[m] = (m >= WIDTH - 1 || r >= seg_start) ? load4(xc + static_cast<int64_t>(r) * x_row) : 0u;
    }
    double ring[WIDTH][kCh];
#pragma unroll
    for (int m = 0; m < WIDTH - 1; ++m) widen2(raw[m], ring[m % WIDTH]);
#pragma unroll
    for (int i = 0; i < RUN; ++i) {
      widen2(raw[i + WIDTH - 1], ring[(i + WIDTH - 1) % WIDTH]);
      const double* win[WIDTH];
#pragma unroll
      for (int j = 0; j < WIDTH; ++j) win[j] = ring[(i + j) % WIDTH];
      row_out(win, r0 + i);
    }
  } else {
    // A sequence starts inside the run, or the run passes the last row: one
    // row at a time, with the window re-read (from L1/L2).
    int start = seg_start;
#pragma unroll 1
    for (int r = r0; r < min(r0 + RUN, total_rows); ++r) {
      if (r >= seg_end) {  // first token of the next sequence
        if (cu_seqlens != nullptr) {
          while (seg + 1 < n_seqs && cu_seqlens[seg + 1] <= r) ++seg;
          start = min(max(cu_seqlens[seg], 0), total_rows);
          seg_end = min(max(cu_seqlens[seg + 1], 0), total_rows);
        } else {
          start = (r / seq_len) * seq_len;
          seg_end = start + seq_len;
        }
      }
      double xw[WIDTH][kCh];
#pragma unroll
      for (int j = 0; j < WIDTH; ++j) {
        const int src = r - (WIDTH - 1) + j;
        widen2(src >= start ? load4(xc + static_cast<int64_t>(src) * x_row) : 0u, xw[j]);
      }
      const double* win[WIDTH];
#pragma unroll
      for (int j = 0; j < WIDTH; ++j) win[j] = xw[j];
      row_out(win, r);
    }
  }
}

template <int WIDTH, int RUN, bool SILU, bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void packed_conv_kernel(ConvArgs args) {
  conv_block<WIDTH, RUN, SILU, HAS_BIAS>(blockIdx.x, gridDim.x, args);
}

// The conv (SiLU, no bias) and the a|b gate projection of the same layer in one
// launch.  The two are independent, and the projection alone is a small,
// latency-bound launch: its first `gate_blocks` workgroups (a multiple of 8,
// so every conv block keeps its XCD) run the projection of 16 tokens each with
// 4 wavefronts taking two hidden-dimension parts apiece, and the rest run
// exactly the conv's blocks.  The projection's bits equal fd_gate_proj_fwd's.
// The register budget asks for the conv kernel's own occupancy (8 wavefronts
// per SIMD), which the projection body would otherwise lower; with 24 or 32
// gate heads the body needs more registers and the launch runs 6 or 4.
template <int WIDTH, int RUN, typename LT, typename BT, int NB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void conv_gate_kernel(ConvArgs conv, fd_gate::GateProjArgs gate,
                                                             int gate_blocks) {
  __shared__ fd_gate::PartSmem<NB> part;
  const int b = blockIdx.x;
  if (b < gate_blocks) {
    fd_gate::gate_proj_rows<LT, BT, NB, kThreads / 64>(b, gate, part);
    return;
  }
  conv_block<WIDTH, RUN, true, false>(b - gate_blocks, gridDim.x - gate_blocks, conv);
}

// Gate projection launched with the conv (fd_packed_conv_gate_fwd), or none.
struct GateSpec {
  fd_gate::GateProjArgs args;
  int a_log_dtype, dt_bias_dtype, heads;
};

template <int WIDTH, int RUN, typename LT, typename BT>
void launch_conv_gate(const ConvArgs& conv, const GateSpec& gate, int conv_blocks, hipStream_t stream) {
  int gate_blocks = static_cast<int>((gate.args.rows + fd_gate::kProjRows - 1) / fd_gate::kProjRows);
  gate_blocks = (gate_blocks + kNumXcd - 1) / kNumXcd * kNumXcd;  // blocks past the last token exit at once
  const dim3 grid(static_cast<unsigned>(gate_blocks + conv_blocks)), block(kThreads);
  switch (gate.heads) {
    case 8: hipLaunchKernelGGL((conv_gate_kernel<WIDTH, RUN, LT, BT, 1>), grid, block, 0, stream, conv, gate.args, gate_blocks); break;
    case 16: hipLaunchKernelGGL((conv_gate_kernel<WIDTH, RUN, LT, BT, 2>), grid, block, 0, stream, conv, gate.args, gate_blocks); break;
    case 24: hipLaunchKernelGGL((conv_gate_kernel<WIDTH, RUN, LT, BT, 3>), grid, block, 0, stream, conv, gate.args, gate_blocks); break;
    default: hipLaunchKernelGGL((conv_gate_kernel<WIDTH, RUN, LT, BT, 4>), grid, block, 0, stream, conv, gate.args, gate_blocks); break;
  }
}

template <int WIDTH, int RUN>
int launch_run(const char* who, const void* x, int64_t x_row, const void* w, const void* bias, void* q, void* k,
               void* v, int total_rows, int seq_len, int key_dim, int value_dim, const int32_t* cu, int n_seqs,
               int act, const GateSpec* gate, hipStream_t stream) {
  const int C = 2 * key_dim + value_dim;
  const int chunks = C / kCh;
  const int n_runs = (total_rows + RUN - 1) / RUN;
  const int n_col = (chunks + kThreads - 1) / kThreads;
  int64_t nblocks = static_cast<int64_t>(n_col) * n_runs;
  nblocks = (nblocks + kNumXcd - 1) / kNumXcd * kNumXcd;  // padded blocks exit at once
  if (nblocks > (1LL << 30)) return fd_set_error(FD_ERR_INVALID_ARGUMENT, "%s: grid too large", who);
  dim3 grid(static_cast<unsigned>(nblocks)), block(kThreads);
  auto xs = static_cast<const uint16_t*>(x);
  auto ws = static_cast<const uint16_t*>(w);
  auto bsp = static_cast<const uint16_t*>(bias);
  auto qs = static_cast<uint16_t*>(q);
  auto ks = static_cast<uint16_t*>(k);
  auto vs = static_cast<uint16_t*>(v);
  const ConvArgs args{xs, ws, bsp, qs, ks, vs, x_row, total_rows, seq_len, key_dim, value_dim, cu, n_seqs, n_runs,
                      n_col};
  if (gate != nullptr) {
    const bool lf = gate->a_log_dtype == FD_DTYPE_F32, bf = gate->dt_bias_dtype == FD_DTYPE_F32;
    const int nb = static_cast<int>(nblocks);
    if (lf && bf) launch_conv_gate<WIDTH, RUN, float, float>(args, *gate, nb, stream);
    else if (lf) launch_conv_gate<WIDTH, RUN, float, uint16_t>(args, *gate, nb, stream);
    else if (bf) launch_conv_gate<WIDTH, RUN, uint16_t, float>(args, *gate, nb, stream);
    else launch_conv_gate<WIDTH, RUN, uint16_t, uint16_t>(args, *gate, nb, stream);
    return fd_check_launch(who);
  }
#define FD_CONV_LAUNCH(SILU, BIAS) \
  hipLaunchKernelGGL((packed_conv_kernel<WIDTH, RUN, SILU, BIAS>), grid, block, 0, stream, args)
  const bool silu = act == FD_ACT_SILU;
  if (silu && bsp == nullptr) FD_CONV_LAUNCH(true, false);
  else if (silu) FD_CONV_LAUNCH(true, true);
  else if (bsp == nullptr) FD_CONV_LAUNCH(false, false);
  else FD_CONV_LAUNCH(false, true);
#undef FD_CONV_LAUNCH
  return fd_check_launch(who);
}

// Tokens per thread: 8 measured fastest with 2 channels per thread (B=1,
// T=2048, C=6144: 13.6 us, 12,288 wavefronts at 8 per SIMD); 16 took 14.2 us
// (one round, 6 per SIMD), 4 and 32 15.8 us, 12 and 24 22 us.
// The fast path's arithmetic is about 17 VALU instructions per output: 4 fp64
// fmas, 2 for the input widening (once per row), the fp64 -> fp32 rounding, 5
// for the hardware SiLU and 4 for the tie-window test, one branch per output
// for the exact fallback.  SQ_INSTS_VALU counts 23.7 per output over a whole
// launch at B=1, T=2048, C=6144 (addresses, packing and the run setup included).
constexpr int kRun = 8;

int packed_conv_entry(const char* who, const void* x, int64_t x_row_stride, const void* weight, const void* bias,
                      void* q, void* k, void* v, int batch, int seq_len, int key_dim, int value_dim, int width,
                      const int32_t* cu_seqlens, int n_seqs, int activation, const GateSpec* gate, void* stream) {
  FD_REQUIRE(x != nullptr && weight != nullptr && q != nullptr && k != nullptr && v != nullptr,
             FD_ERR_INVALID_ARGUMENT, "%s: x, weight, q, k and v must be non-null", who);
  FD_REQUIRE(batch >= 0 && seq_len >= 0, FD_ERR_INVALID_ARGUMENT,
             "%s: batch and seq_len must be >= 0 (got %d, %d)", who, batch, seq_len);
  FD_REQUIRE(key_dim > 0 && value_dim > 0 && key_dim % 8 == 0 && value_dim % 8 == 0, FD_ERR_INVALID_ARGUMENT,
             "%s: key_dim and value_dim must be positive multiples of 8 (got %d, %d)", who, key_dim, value_dim);
  FD_REQUIRE(width >= 1 && width <= 4, FD_ERR_UNSUPPORTED, "%s: width must be in [1, 4] (got %d)", who, width);
  FD_REQUIRE(activation == FD_ACT_NONE || activation == FD_ACT_SILU, FD_ERR_INVALID_ARGUMENT,
             "%s: activation must be FD_ACT_NONE or FD_ACT_SILU (got %d)", who, activation);
  const int64_t total = static_cast<int64_t>(batch) * seq_len;
  const int64_t C = 2 * static_cast<int64_t>(key_dim) + value_dim;
  FD_REQUIRE(x_row_stride >= C && x_row_stride % 8 == 0, FD_ERR_ALIGNMENT,
             "%s: the row stride of x must be a multiple of 8 and >= C", who);
  FD_REQUIRE(total * x_row_stride < (static_cast<int64_t>(1) << 40) && total < 2147483647LL && C <= 1048576,
             FD_ERR_INVALID_ARGUMENT, "%s: problem too large", who);
  if (cu_seqlens != nullptr) {
    FD_REQUIRE(batch == 1, FD_ERR_INVALID_ARGUMENT, "%s: cu_seqlens requires batch == 1 (got %d)", who, batch);
    FD_REQUIRE(n_seqs >= 1, FD_ERR_INVALID_ARGUMENT, "%s: n_seqs must be >= 1 (got %d)", who, n_seqs);
  }
  FD_REQUIRE(fd_aligned16(x) && fd_aligned16(weight) && fd_aligned16(q) && fd_aligned16(k) && fd_aligned16(v) &&
                 (bias == nullptr || fd_aligned16(bias)),
             FD_ERR_ALIGNMENT, "%s: inputs must be aligned to 16 bytes", who);
  if (total == 0) return FD_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rows = static_cast<int>(total);
  switch (width) {
    case 1: return launch_run<1, kRun>(who, x, x_row_stride, weight, bias, q, k, v, rows, seq_len, key_dim, value_dim, cu_seqlens, n_seqs, activation, gate, s);
    case 2: return launch_run<2, kRun>(who, x, x_row_stride, weight, bias, q, k, v, rows, seq_len, key_dim, value_dim, cu_seqlens, n_seqs, activation, gate, s);
    case 3: return launch_run<3, kRun>(who, x, x_row_stride, weight, bias, q, k, v, rows, seq_len, key_dim, value_dim, cu_seqlens, n_seqs, activation, gate, s);
    default: return launch_run<4, kRun>(who, x, x_row_stride, weight, bias, q, k, v, rows, seq_len, key_dim, value_dim, cu_seqlens, n_seqs, activation, gate, s);
  }
}

}  // namespace

extern "C" int fd_packed_conv_fwd(const void* x, const void* weight, const void* bias, void* q, void* k, void* v,
                                  int batch, int seq_len, int key_dim, int value_dim, int width,
                                  const int32_t* cu_seqlens, int n_seqs, int activation, void* stream) {
  return packed_conv_entry("fd_packed_conv_fwd", x, 2 * static_cast<int64_t>(key_dim) + value_dim, weight, bias, q,
                           k, v, batch, seq_len, key_dim, value_dim, width, cu_seqlens, n_seqs, activation, nullptr,
                           stream);
}

extern "C" int fd_packed_conv_strided_fwd(const void* x, int64_t x_row_stride, const void* weight, const void* bias,
                                          void* q, void* k, void* v, int batch, int seq_len, int key_dim,
                                          int value_dim, int width, const int32_t* cu_seqlens, int n_seqs,
                                          int activation, void* stream) {
  return packed_conv_entry("fd_packed_conv_fwd", x, x_row_stride, weight, bias, q, k, v, batch, seq_len, key_dim,
                           value_dim, width, cu_seqlens, n_seqs, activation, nullptr, stream);
}

extern "C" int fd_packed_conv_gate_fwd(const void* x, int64_t x_row_stride, const void* weight, void* q, void* k,
                                       void* v, int batch, int seq_len, int key_dim, int value_dim, int width,
                                       const int32_t* cu_seqlens, int n_seqs, const void* hidden_states,
                                       int64_t hidden_row_stride, const void* gate_weight, int hidden,
                                       const void* a_log, int a_log_dtype, const void* dt_bias, int dt_bias_dtype,
                                       float* g, void* beta, int heads, void* stream) {
  const char* who = "fd_packed_conv_gate_fwd";
  const int64_t rows = static_cast<int64_t>(batch) * seq_len;
  const int rc = fd_gate::gate_proj_check(who, hidden_states, hidden_row_stride, gate_weight, hidden, a_log,
                                          a_log_dtype, dt_bias, dt_bias_dtype, g, beta, rows, heads);
  if (rc != FD_OK) return rc;
  const GateSpec gate{{static_cast<const uint16_t*>(hidden_states), hidden_row_stride,
                       static_cast<const uint16_t*>(gate_weight), hidden, a_log, dt_bias, g,
                       static_cast<uint16_t*>(beta), nullptr, rows},
                      a_log_dtype, dt_bias_dtype, heads};
  return packed_conv_entry(who, x, x_row_stride, weight, nullptr, q, k, v, batch, seq_len, key_dim, value_dim, width,
                           cu_seqlens, n_seqs, FD_ACT_SILU, &gate, stream);
}

namespace {
// bf16(fd_silu_bf16(y)) against bf16(fd_silu(y)) for the fp32 bit patterns
// [begin, begin + count); both NaN counts as equal.  One atomic per wavefront.
__global__ __launch_bounds__(256) void silu_check_kernel(uint32_t begin, uint32_t count,
                                                         unsigned long long* mismatches) {
  unsigned n = 0;
  // 64-bit index: a 32-bit one would wrap past 2^32 - stride and never reach count
  for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += gridDim.x * 256ull) {
    const float y = __uint_as_float(begin + static_cast<uint32_t>(i));
    const uint32_t a = fd_pack2(fd_silu_bf16(y), 0.0f) & 0xffffu;
    const uint32_t b = fd_pack2(fd_silu(y), 0.0f) & 0xffffu;
    const bool a_nan = (a & 0x7f80u) == 0x7f80u && (a & 0x7fu) != 0;
    const bool b_nan = (b & 0x7f80u) == 0x7f80u && (b & 0x7fu) != 0;
    if (a != b && !(a_nan && b_nan)) ++n;
  }
  for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off, 64);
  if ((threadIdx.x & 63) == 0 && n != 0) atomicAdd(mismatches, static_cast<unsigned long long>(n));
}
}  // namespace

extern "C" int fd_silu_check(uint32_t begin, uint32_t count, unsigned long long* mismatches, void* stream) {
  FD_REQUIRE(mismatches != nullptr, FD_ERR_INVALID_ARGUMENT, "fd_silu_check: mismatches must be non-null");
  FD_REQUIRE(static_cast<uint64_t>(begin) + count <= (1ULL << 32), FD_ERR_INVALID_ARGUMENT,
             "fd_silu_check: [begin, begin + count) must lie within the 2^32 fp32 bit patterns");
  if (count == 0) return 0;
  hipLaunchKernelGGL(silu_check_kernel, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream), begin, count,
                     mismatches);
  return fd_check_launch("fd_silu_check");
}

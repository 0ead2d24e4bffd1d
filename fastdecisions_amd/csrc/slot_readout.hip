// Slot-only readout of the decider for gfx950: final RMSNorm + option-letter
// projection + masked softmax, evaluated only at the requested (row, position)
// slots instead of at every token.
//
// Replaces the reference's opt-in slot projection
// (ref: src/decider/slot_projection.py:6-21: project the final hidden states only
// at the slots) and the readout after it (ref: src/decider/engine.py:48-56,
// src/decider/model.py:18-27, src/decider/temperature.py:136-144), and moves the
// model's final norm (transformers Qwen3_5RMSNorm, which is row-local) to the
// slot rows as well:
//   y        = bf16((x * (1 / sqrt(mean(x^2) + eps))) * g),   g = 1 + w or w
//   logit[k] = bf16(sum_d y_d * W[k, d])                        (F.linear on bf16)
//   prob     = softmax(logit[:nopts] / temperature), 0 past nopts
// One workgroup (256 threads) per slot: the row's sum of squares is formed in
// the order PyTorch's GPU row mean uses (for H a multiple of 256; then y equals
// eager's normed row bit for bit), the row normalised into LDS, then each
// wavefront takes every 4th letter row of W with a wavefront reduction per letter.
#include "fd_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxWidth = 8192;
constexpr int kMaxLetters = 1024;

struct SlotArgs {
  const uint16_t* hidden;  // [B, T, H]
  const void* norm_w;      // [H]
  const uint16_t* letters; // [K, H]
  const int32_t* rows;
  const int32_t* pos;
  const int32_t* nopts;    // [N] or null (all K letters)
  float* logits;           // [N, K]
  float* probs;            // [N, K] or null
  int B, T, H, K, w_f32, gain_offset;
  float eps, temp;
};

// round to bf16 and back (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ float bf16r(float x) { return fd_lo(fd_pack2(x, 0.0f)); }

__device__ __forceinline__ float wave_sum(float s) {
  s = fd_xor_sum_down<64>(s);
  return s;
}

__global__ __launch_bounds__(kThreads) void slot_readout_kernel(SlotArgs a) {
  __shared__ __attribute__((aligned(16))) float sy[kMaxWidth];
  __shared__ float sl[kMaxLetters];
  __shared__ float red[kThreads / 64];
  const int n = blockIdx.x;
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int l = tid & 63;
  // out-of-range slots read row 0, position 0 (as the reference's unused entries do)
  int b = a.rows[n], t = a.pos[n];
  if (b < 0 || b >= a.B || t < 0 || t >= a.T) b = t = 0;
  const uint16_t* x = a.hidden + (static_cast<int64_t>(b) * a.T + t) * a.H;
  const int nch = a.H / 8;

  // the row, widened to fp32 into LDS (16-byte loads); each thread later
  // normalises the same features in place
  for (int c = tid; c < nch; c += kThreads) {
    const uint4 raw = *reinterpret_cast<const uint4*>(x + 8 * c);
    *reinterpret_cast<float4*>(sy + 8 * c) = make_float4(fd_lo(raw.x), fd_hi(raw.x), fd_lo(raw.y), fd_hi(raw.y));
    *reinterpret_cast<float4*>(sy + 8 * c + 4) = make_float4(fd_lo(raw.z), fd_hi(raw.z), fd_lo(raw.w), fd_hi(raw.w));
  }
  __syncthreads();
  const bool torch_order = a.H % 256 == 0;
  if (torch_order) {
    // PyTorch's order for a row mean of this width (the model's final norm runs
    // over every row in eager): lane l owns the 4-feature groups at 256 k + 4 l,
    // one accumulator per group position summed over k in order, then
    // ((a0 + a1) + a2) + a3, then a pairwise tree over the 64 lanes.
    if (wv == 0) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k = 0; k < a.H / 256; ++k) {
        const float4 v = *reinterpret_cast<const float4*>(sy + 256 * k + 4 * l);
        acc[0] = acc[0] + v.x * v.x;
        acc[1] = acc[1] + v.y * v.y;
        acc[2] = acc[2] + v.z * v.z;
        acc[3] = acc[3] + v.w * v.w;
      }
      float s = ((acc[0] + acc[1]) + acc[2]) + acc[3];
      s = fd_xor_sum_up<64>(s);
      if (l == 0) red[0] = s;
    }
  } else {
    float s = 0.0f;
    for (int c = tid; c < nch; c += kThreads) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s = s + sy[8 * c + e] * sy[8 * c + e];
    }
    s = wave_sum(s);
    if (l == 0) red[wv] = s;
  }
  __syncthreads();
  const float tot = torch_order ? red[0] : (red[0] + red[1]) + (red[2] + red[3]);
  // the mean as torch forms it (the sum times fl(1 / H)); 1 / sqrt evaluated in
  // fp64 and rounded to fp32, which matched torch.rsqrt on every input measured
  const float inv = static_cast<float>(
      1.0 / __builtin_sqrt(static_cast<double>(tot * (1.0f / static_cast<float>(a.H)) + a.eps)));
  for (int c = tid; c < nch; c += kThreads) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float g = a.w_f32 ? static_cast<const float*>(a.norm_w)[8 * c + e]
                        : fd_bf16_to_f32(static_cast<const uint16_t*>(a.norm_w)[8 * c + e]);
      if (a.gain_offset) g = 1.0f + g;
      sy[8 * c + e] = bf16r((sy[8 * c + e] * inv) * g);
    }
  }
  __syncthreads();

  // letter logits: wavefront wv takes letters wv, wv + 4, ...
  for (int k = wv; k < a.K; k += kThreads / 64) {
    const uint16_t* wr = a.letters + static_cast<int64_t>(k) * a.H;
    float acc = 0.0f;
    for (int c = l; c < nch; c += 64) {
      const uint4 raw = *reinterpret_cast<const uint4*>(wr + 8 * c);
      const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
      const float* yv = sy + 8 * c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = fmaf(yv[2 * i], fd_lo(wd[i]), acc);
        acc = fmaf(yv[2 * i + 1], fd_hi(wd[i]), acc);
      }
    }
    acc = wave_sum(acc);
    if (l == 0) {
      const float lg = bf16r(acc);
      sl[k] = lg;
      a.logits[static_cast<int64_t>(n) * a.K + k] = lg;
    }
  }
  if (a.probs == nullptr) return;
  __syncthreads();

  // masked softmax at temperature: one wavefront
  if (wv == 0) {
    const int nopt = a.nopts ? min(max(a.nopts[n], 0), a.K) : a.K;
    float m = -__builtin_inff();
    for (int k = l; k < nopt; k += 64) m = fmaxf(m, sl[k] / a.temp);
    m = fd_xor_max<32>(m);
    m = fd_xor_max<16>(m);
    m = fd_xor_max<8>(m);
    m = fd_xor_max<4>(m);
    m = fd_xor_max<2>(m);
    m = fd_xor_max<1>(m);
    float sum = 0.0f;
    for (int k = l; k < nopt; k += 64) sum += expf(sl[k] / a.temp - m);
    sum = wave_sum(sum);
    for (int k = l; k < a.K; k += 64)
      a.probs[static_cast<int64_t>(n) * a.K + k] = k < nopt ? expf(sl[k] / a.temp - m) / sum : 0.0f;
  }
}

}  // namespace

extern "C" FD_API int fd_slot_readout_fwd(const void* hidden, int batch, int seq_len, int width,
                                          const void* norm_weight, int weight_dtype, int gain_offset, float eps,
                                          const void* letters, int n_letters, const int32_t* slot_rows,
                                          const int32_t* slot_positions, const int32_t* nopts, int n_slots,
                                          float temperature, float* logits, float* probs, void* stream) {
  FD_REQUIRE(hidden && norm_weight && letters && slot_rows && slot_positions && logits, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: hidden, weights, slot indices and logits must be non-null");
  FD_REQUIRE(batch >= 1 && seq_len >= 1 && n_slots >= 0, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: batch and seq_len must be >= 1 and n_slots >= 0");
  FD_REQUIRE(width >= 8 && width <= kMaxWidth && width % 8 == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: width must be a multiple of 8 in [8, %d] (got %d)", kMaxWidth, width);
  FD_REQUIRE(n_letters >= 1 && n_letters <= kMaxLetters, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: n_letters must be in [1, %d]", kMaxLetters);
  FD_REQUIRE(weight_dtype == FD_DTYPE_BF16 || weight_dtype == FD_DTYPE_F32, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: weight_dtype must be FD_DTYPE_BF16 or FD_DTYPE_F32");
  FD_REQUIRE(eps >= 0.0f && temperature > 0.0f, FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: eps must be >= 0 and temperature > 0");
  FD_REQUIRE(fd_aligned16(hidden) && fd_aligned16(letters), FD_ERR_ALIGNMENT,
             "fd_slot_readout_fwd: hidden and letters must be 16-byte aligned");
  FD_REQUIRE(static_cast<int64_t>(batch) * seq_len * width < (1LL << 40), FD_ERR_INVALID_ARGUMENT,
             "fd_slot_readout_fwd: hidden too large");
  if (n_slots == 0) return FD_OK;
  SlotArgs a;
  a.hidden = static_cast<const uint16_t*>(hidden);
  a.norm_w = norm_weight;
  a.letters = static_cast<const uint16_t*>(letters);
  a.rows = slot_rows;
  a.pos = slot_positions;
  a.nopts = nopts;
  a.logits = logits;
  a.probs = probs;
  a.B = batch;
  a.T = seq_len;
  a.H = width;
  a.K = n_letters;
  a.w_f32 = weight_dtype == FD_DTYPE_F32;
  a.gain_offset = gain_offset != 0;
  a.eps = eps;
  a.temp = temperature;
  hipLaunchKernelGGL(slot_readout_kernel, dim3(n_slots), dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  return fd_check_launch("fd_slot_readout_fwd");
}

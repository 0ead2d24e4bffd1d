/*
 * TEST INFRASTRUCTURE — CPU oracle for the decider hot path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this; the
 * product never does.
 *
 * Plain-C restatement, in fp32 with every operation rounded where written
 * (build with -ffp-contract=off), of:
 *   - the packed causal depthwise conv1d + SiLU with head-split store
 *     (ref: src/decider/packed_conv_kernel.py:128-191: taps :139-177,
 *      zero taps before the sequence start :128-176, SiLU :178-182,
 *      q/k/v split :184-191), with the tap sum rounded once to fp32 as
 *      PyTorch's fp32 GPU conv1d rounds it (BASELINE config 2's definition);
 *   - the attention prologue (per-head RMSNorm of q / k, partial rotary
 *     embedding; ref: experiments/native_gqa/bench_native_gqa_model.py:47-53);
 *   - the fused residual add + RMSNorm (ref: src/decider/residual_rms_baseline.py:48-85
 *     for eps placement, ref: src/decider/persistent_residual_rms_kernel.py:59-72 for
 *     the (w + 1) gain; the residual is rounded to bf16 before it is normalised as in
 *     transformers' Qwen3_5DecoderLayer + Qwen3_5RMSNorm).
 * The summation order of the RMSNorm matches the GPU kernel's documented order
 * (widths a multiple of 1024: PyTorch's GPU row-mean order, 4-feature groups per
 * lane strided by 256, four accumulators, a pairwise tree over 64 lanes; other
 * widths: per-lane chunk order, then a 6-step xor butterfly), so GPU output is
 * compared bit for bit; the mathematics pins this restatement independently
 * (tests/test_oracle.py: fp64 closed forms, torch's F.conv1d and eager RMSNorm,
 * special cases), and on the GPU eager RMSNorm at width 2048 equals it bit for bit.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16, NaN -> 0x7fc0 (torch's rule). */
uint16_t fd_oracle_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* SiLU as PyTorch's fp32 kernel writes it and the reference restates it,
 * y / (1 + expf(-y)) (ref: src/decider/packed_conv_kernel.py:178-182), with the
 * C library's expf.  The device expf the GPU kernel calls is a different
 * approximation (within 1 fp32 ulp), so on rare inputs the two SiLUs land on
 * neighbouring bf16 values; the GPU tests bound that, and compare the kernel
 * bit for bit with torch's own GPU silu instead. */
float fd_oracle_silu(float y) { return y / (1.0f + expf(-y)); }

/* One conv output before the activation: the exact sum of the taps
 * w[j] * x[j] (x[0] is the oldest row; zeros stand for rows before the
 * sequence start), rounded once to fp32, then + bias in fp32.  Each product of
 * two bf16 values is exact in double, and so is their running sum (unless the
 * products span more than 2^37).  Accumulated from +0 in tap order, so an
 * exact zero is +0. */
static float conv_taps_f32(const double* xv, const uint16_t* w, int width, const uint16_t* bias) {
  double acc = 0.0;
  for (int j = 0; j < width; ++j) acc = fma((double)bf16_to_f32(w[j]), xv[j], acc);
  float t = (float)acc;
  if (bias) t = t + bf16_to_f32(*bias);
  return t;
}

/* conv_taps_f32 over n independent windows: xwin [n, width] and w [n, width]
 * bf16 bits, bias [n] or NULL; out [n] fp32. */
void fd_oracle_conv_taps(const uint16_t* xwin, const uint16_t* w, const uint16_t* bias, float* out, int64_t n,
                         int width) {
  for (int64_t i = 0; i < n; ++i) {
    double xv[4];
    for (int j = 0; j < width && j < 4; ++j) xv[j] = (double)bf16_to_f32(xwin[(size_t)i * width + j]);
    out[i] = conv_taps_f32(xv, w + (size_t)i * width, width, bias ? bias + i : NULL);
  }
}

/* Packed causal depthwise conv1d + activation, token-major [B, T, C] input,
 * C = 2*key_dim + value_dim, weight [C, width], optional bias [C].
 * Returns 0, or -1 on invalid arguments. */
int fd_oracle_packed_conv(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* q, uint16_t* k,
                          uint16_t* v, int batch, int seq_len, int key_dim, int value_dim, int width,
                          const int32_t* cu_seqlens, int n_seqs, int activation) {
  if (batch < 0 || seq_len < 0 || key_dim <= 0 || value_dim <= 0 || width < 1 || width > 4) return -1;
  const int C = 2 * key_dim + value_dim;
  const int64_t total = (int64_t)batch * seq_len;
  for (int64_t r = 0; r < total; ++r) {
    /* start of the sequence that holds row r */
    int64_t start;
    if (cu_seqlens) {
      int s = 0;
      while (s + 1 < n_seqs && cu_seqlens[s + 1] <= r) ++s;
      start = cu_seqlens[s];
    } else {
      start = (r / seq_len) * seq_len;
    }
    for (int c = 0; c < C; ++c) {
      double xv[4];
      for (int j = 0; j < width; ++j) {
        const int64_t src = r - (width - 1) + j;
        xv[j] = src >= start ? (double)bf16_to_f32(x[(size_t)src * C + c]) : 0.0;
      }
      const float t = conv_taps_f32(xv, w + (size_t)c * width, width, bias ? bias + c : NULL);
      const float y = activation == 1 ? fd_oracle_silu(t) : t;
      const uint16_t h = fd_oracle_f32_to_bf16(y);
      if (c < key_dim)
        q[(size_t)r * key_dim + c] = h;
      else if (c < 2 * key_dim)
        k[(size_t)r * key_dim + (c - key_dim)] = h;
      else
        v[(size_t)r * value_dim + (c - 2 * key_dim)] = h;
    }
  }
  return 0;
}

/* Fused residual add + RMSNorm over rows of `width` (a multiple of 8, <= 8192).
 * weight_dtype 0: bf16 weight, 1: fp32 weight.  residual / residual_out may be NULL. */
int fd_oracle_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const void* weight, uint16_t* out,
                          uint16_t* residual_out, int64_t rows, int width, float eps, int weight_dtype,
                          int gain_offset) {
  if (width < 8 || width > 8192 || width % 8 || rows < 0) return -1;
  const int nchunks = width / 8;
  float h[8192];
  for (int64_t row = 0; row < rows; ++row) {
    const size_t base = (size_t)row * width;
    for (int i = 0; i < width; ++i) {
      if (residual) {
        const float sum = bf16_to_f32(x[base + i]) + bf16_to_f32(residual[base + i]);
        const uint16_t hb = fd_oracle_f32_to_bf16(sum);
        h[i] = bf16_to_f32(hb);
        if (residual_out) residual_out[base + i] = hb;
      } else {
        h[i] = bf16_to_f32(x[base + i]);
      }
    }
    float row_sum;
    float lane_sum[64];
    if (width % 1024 == 0) {
      /* width a multiple of 1024 (PyTorch's GPU row-mean order at this width):
       * lane l owns the 4-feature groups at 256 k + 4 l, k = 0 .. width/256 - 1;
       * one accumulator per group position, summed over k in order, then
       * ((a0 + a1) + a2) + a3, then a pairwise tree over the lanes with
       * partner offsets 1, 2, .., 32 */
      for (int l = 0; l < 64; ++l) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < width / 256; ++k)
          for (int i = 0; i < 4; ++i) {
            const float hv = h[256 * k + 4 * l + i];
            const float sq = hv * hv;
            acc[i] = acc[i] + sq;
          }
        lane_sum[l] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
      }
      for (int off = 1; off <= 32; off <<= 1) {
        float next[64];
        for (int l = 0; l < 64; ++l) next[l] = lane_sum[l] + lane_sum[l ^ off];
        memcpy(lane_sum, next, sizeof(next));
      }
    } else {
      /* other widths: lane l owns the 8-feature chunks l, l+64, l+128, ..., its sum in
       * chunk order, then an xor butterfly with offsets 32, 16, .., 1 */
      for (int l = 0; l < 64; ++l) {
        float s = 0.0f;
        for (int c = l; c < nchunks; c += 64)
          for (int e = 0; e < 8; ++e) {
            const float hv = h[c * 8 + e];
            const float sq = hv * hv;
            s = s + sq;
          }
        lane_sum[l] = s;
      }
      for (int off = 32; off >= 1; off >>= 1) {
        float next[64];
        for (int l = 0; l < 64; ++l) next[l] = lane_sum[l] + lane_sum[l ^ off];
        memcpy(lane_sum, next, sizeof(next));
      }
    }
    row_sum = lane_sum[0];
    /* the mean as PyTorch forms it (the sum times fl(1 / width)); the inverse root
     * evaluated in fp64 (root and quotient) and rounded to fp32 */
    const float mean = row_sum * (1.0f / (float)width);
    const float inv = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int i = 0; i < width; ++i) {
      float g = weight_dtype == 1 ? ((const float*)weight)[i] : bf16_to_f32(((const uint16_t*)weight)[i]);
      if (gain_offset) g = 1.0f + g;
      const float y = (h[i] * inv) * g;
      out[base + i] = fd_oracle_f32_to_bf16(y);
    }
  }
  return 0;
}

/* Attention prologue on rows of 128 bf16 features (row r belongs to token r / heads):
 * RMSNorm with PyTorch's GPU summation order at width 128 (32 slots of 4 features,
 * then a pairwise tree) and the inverse root evaluated in fp64, gain (1 + w) or w,
 * one bf16 rounding; then the rotary embedding of the first `rot` features with
 * every bf16 product and sum rounded (transformers apply_rotary_pos_emb on bf16;
 * ref: experiments/native_gqa/bench_native_gqa_model.py:47-53).
 * weight_dtype 0: bf16, 1: fp32.  cos / sin: [rows / heads][rot] bf16.  Returns 0 or -1. */
static float r16(float x) { return bf16_to_f32(fd_oracle_f32_to_bf16(x)); }

int fd_oracle_attn_prologue(const uint16_t* x, int64_t rows, int heads, const void* weight, int weight_dtype,
                            int gain_offset, float eps, const uint16_t* cos, const uint16_t* sin, int rot,
                            uint16_t* out) {
  if (rows < 0 || heads < 1 || rot < 0 || rot > 128 || (rot % 16)) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + (size_t)r * 128;
    float v[128], y[128];
    for (int i = 0; i < 128; ++i) v[i] = bf16_to_f32(xr[i]);
    /* PyTorch's GPU row-mean order at width 128: 32 slots of 4 features, each
     * ((x0^2 + x1^2) + x2^2) + x3^2, then a pairwise tree over the slots */
    float slot[32];
    for (int l = 0; l < 32; ++l) {
      float s = v[4 * l] * v[4 * l];
      for (int e = 1; e < 4; ++e) {
        const float sq = v[4 * l + e] * v[4 * l + e];
        s = s + sq;
      }
      slot[l] = s;
    }
    for (int off = 1; off <= 16; off <<= 1) {
      float next[32];
      for (int l = 0; l < 32; ++l) next[l] = slot[l] + slot[l ^ off];
      memcpy(slot, next, sizeof(next));
    }
    const float mean = slot[0] * (1.0f / 128.0f);
    const float inv = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int i = 0; i < 128; ++i) {
      float g = weight_dtype == 1 ? ((const float*)weight)[i] : bf16_to_f32(((const uint16_t*)weight)[i]);
      if (gain_offset) g = 1.0f + g;
      const float t = v[i] * inv;
      y[i] = r16(t * g);
    }
    const int64_t tok = r / heads;
    uint16_t* o = out + (size_t)r * 128;
    for (int i = 0; i < 128; ++i) {
      float res = y[i];
      if (i < rot) {
        const int h = rot / 2;
        const float rh = i < h ? -y[i + h] : y[i - h];
        const float c = bf16_to_f32(cos[(size_t)tok * rot + i]);
        const float s = bf16_to_f32(sin[(size_t)tok * rot + i]);
        res = r16(r16(y[i] * c) + r16(rh * s));
      }
      o[i] = fd_oracle_f32_to_bf16(res);
    }
  }
  return 0;
}

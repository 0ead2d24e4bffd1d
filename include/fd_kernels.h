/*
 * fd_kernels.h — C ABI of the FastDecisions MI355X (gfx950) hot-path kernels.
 *
 * Forward kernels of the decider model, each a drop-in for one Python
 * launcher or call of the reference:
 *
 *   fd_gqa_fwd          native GQA causal attention
 *                       replaces native_gqa_attention(q, k, v)
 *                       (ref: src/decider/native_gqa_kernel.py:116-173, kernel :6-113)
 *   fd_packed_conv_fwd  packed causal depthwise conv1d + SiLU, head-split q/k/v store
 *                       replaces prep_qkv(input_qkv, weight)
 *                       (ref: src/decider/packed_conv_kernel.py:194-232, kernel :115-191)
 *   fd_add_rmsnorm_fwd  fused residual add + RMSNorm returning both outputs
 *                       replaces residual_rms(a, b, weight)
 *                       (ref: src/decider/persistent_residual_rms_kernel.py:75-104, kernel :49-72;
 *                        eps placement as ref: src/decider/residual_rms_baseline.py:75-78)
 *   fd_gated_delta_fwd  chunked gated delta rule of the Gated-DeltaNet layers
 *                       replaces the torch_chunk_gated_delta_rule call
 *                       (ref: src/decider/packed_conv.py:55-59)
 *   fd_gated_delta_norm_fwd  fd_gated_delta_fwd followed by the layer's gated RMSNorm
 *   fd_gqa_gated_fwd    fd_gqa_fwd with the attention layer's sigmoid output gate applied in the store
 *   fd_attn_prologue_fwd   q/k RMSNorm over head_dim + partial rotary embedding of the attention layers
 *                       replaces the eager prologue of the patched attention forward
 *                       (ref: experiments/native_gqa/bench_native_gqa_model.py:47-53)
 *   fd_slot_readout_fwd final RMSNorm + option-letter projection + masked softmax at the slots only
 *                       replaces SlotProjectionForward and read_slots
 *                       (ref: src/decider/slot_projection.py:6-21, src/decider/engine.py:48-56)
 *   fd_gated_rmsnorm_fwd   gated RMSNorm of the delta rule's output (transformers Qwen3_5RMSNormGated)
 *   fd_silu_mul_fwd     the MLP's silu(gate) * up on a combined gate|up projection
 *   fd_silu_mul_split_fwd  the same on two gate|up projections (the MLP's GEMM split in two)
 *   fd_gate_transform_fwd  gate transform (decay g and beta) of the Gated-DeltaNet layers
 *                       replaces unpack_gate(combined, a_log, dt_bias)
 *                       (ref: src/decider/unpack_gate_transform_kernel.py:94-133, kernel :51-91)
 *   fd_gate_proj_fwd    the combined a|b gate projection fused with the gate transform
 *                       replaces F.linear(x, cat(W_a, W_b)) + unpack_gate
 *                       (ref: src/decider/combined_gates.py:19-43, packed_conv.py:45-53)
 *   fd_packed_conv_gate_fwd  fd_packed_conv_strided_fwd and fd_gate_proj_fwd of one layer in one launch
 *   fd_silu_check       numerics self-check of the conv's SiLU (no reference counterpart)
 *   fd_gated_silu_check numerics self-check of the gated RMSNorm's last product (no reference counterpart)
 *   fd_hbm_copy         streaming device copy, the measured HBM ceiling (no reference counterpart)
 *
 * Conventions shared by every entry point:
 *   - every tensor pointer is a device pointer; bf16 tensors are passed as raw
 *     16-bit storage (torch.bfloat16 bit layout);
 *   - no entry point allocates, frees or synchronises: work is enqueued on
 *     `stream` (a hipStream_t; NULL is the legacy default stream), so calls
 *     can be captured into a HIP graph;
 *   - the return value is FD_OK (0) or a negative FD_ERR_* code; the message
 *     of the last failure on the calling thread is fd_last_error().
 */
#ifndef FD_KERNELS_H
#define FD_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define FD_API __attribute__((visibility("default")))
#else
#define FD_API
#endif

#define FD_ABI_VERSION 12

#define FD_OK 0
#define FD_ERR_INVALID_ARGUMENT (-1) /* shape, size, stride or flag out of range */
#define FD_ERR_UNSUPPORTED (-2)      /* valid request this build does not implement */
#define FD_ERR_ALIGNMENT (-3)        /* pointer or stride breaks the 16-byte vector contract */
#define FD_ERR_LAUNCH (-4)           /* the HIP runtime rejected the launch */

#define FD_DTYPE_BF16 0
#define FD_DTYPE_F32 1

#define FD_ACT_NONE 0
#define FD_ACT_SILU 1

/* Version of this ABI (FD_ABI_VERSION of the library that was built). */
FD_API int fd_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
FD_API const char* fd_last_error(void);

/*
 * Causal grouped-query attention forward, bf16 in/out, fp32 softmax.
 *
 * Logical layouts (strides in elements, innermost stride must be 1):
 *   q   [batch, q_heads,  seq_len, head_dim]   q_strides   = {b, h, t, d}
 *   k,v [batch, kv_heads, seq_len, head_dim]   k/v_strides = {b, h, t, d}
 *   out [batch, q_heads,  seq_len, head_dim]   out_strides = {b, h, t, d}
 * Query head h reads key/value head h / (q_heads / kv_heads), as the
 * reference kernel does (ref: src/decider/native_gqa_kernel.py:39-41).
 * Key j is visible to query i iff j <= i (same sequence).  P is rounded to
 * bf16 before the P·V product (ref: src/decider/native_gqa_kernel.py:98-102).
 *
 * Varlen: with cu_seqlens != NULL (device int32[n_seqs + 1], non-decreasing,
 * cu_seqlens[0] == 0, cu_seqlens[n_seqs] == seq_len), batch must be 1 and the
 * T axis holds n_seqs packed requests; masking is causal within each request
 * and no request sees another.  max_seqlen (host) must be at least the longest
 * request: it sets the number of query tiles per request, so the rows of a
 * longer request past max_seqlen are not written.  Offsets are clamped to
 * [0, seq_len] on the device.
 *
 * workspace / workspace_bytes: optional device memory (16-byte aligned) for
 * the key split of long query tiles at head_dim 256, see
 * fd_gqa_workspace_bytes; NULL / 0 runs unsplit.  With a split the call
 * enqueues two launches on `stream`.
 *
 * Batch invariance: for head_dim 64 and 128 every call runs the same loop
 * (two wavefronts per (head, 32 queries), one on each 32-key half of every
 * 64-key tile, merged at the end), whatever the batch, the packing or the
 * workspace, so a request's output rows are bit-identical alone, packed with
 * others through cu_seqlens, or in a padded batch.  For head_dim 256 that
 * holds when no key split runs (workspace NULL or 0 bytes, or more work items
 * than fd_gqa_workspace_bytes splits); a split rounds the split tiles
 * differently, by at most about one bf16 step.
 *
 * Limits: head_dim in {64, 128, 256}; q_heads % kv_heads == 0; every base
 * pointer and every non-unit stride keeps 16-byte alignment.
 */
FD_API int fd_gqa_fwd(const void* q, const void* k, const void* v, void* out,
               const int64_t q_strides[4], const int64_t k_strides[4],
               const int64_t v_strides[4], const int64_t out_strides[4],
               int batch, int q_heads, int kv_heads, int seq_len, int head_dim,
               float scale, const int32_t* cu_seqlens, int n_seqs, int max_seqlen,
               void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace with which fd_gqa_fwd / fd_gqa_gated_fwd split the
 * key range of the long query tiles of these sizes (n_seqs = 0 for a padded
 * batch), 0 when they run unsplit, or a negative FD_ERR_* code.
 *
 * Causal attention gives the query tiles near the end of a sequence up to
 * twice the average work; when a padded batch has fewer work items than the
 * GPU has CUs (B=1, T=2048, 8/2 heads of 256: 128), those tiles set the
 * kernel's length.  With a workspace of at least this size the longest half
 * of the tiles of every (sequence, head group) run as two work items over the
 * two halves of their key tiles, and a second launch on the same stream
 * merges the halves (their running maxima and denominators) and stores the
 * rows.  A null or smaller workspace runs every tile whole: same results
 * within rounding, no split.  Only head_dim 256 splits (0 for 64 and 128);
 * packed requests (n_seqs > 0) never do.
 */
FD_API int64_t fd_gqa_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int head_dim,
                                      int n_seqs, int max_seqlen);

/*
 * fd_gqa_fwd followed by the attention layer's output gate, applied before the
 * store (ref: experiments/native_gqa/bench_native_gqa_model.py:54-55,
 * `output * torch.sigmoid(gate)`):
 *   out = bf16(bf16(attn) * bf16(1 / (1 + exp(-gate))))
 * gate has the logical layout of out, [batch, q_heads, seq_len, head_dim]
 * (gate_strides = {b, h, t, d}, innermost 1, 16-byte rows).  Other arguments
 * and limits as fd_gqa_fwd.
 */
FD_API int fd_gqa_gated_fwd(const void* q, const void* k, const void* v, const void* gate, void* out,
                            const int64_t q_strides[4], const int64_t k_strides[4],
                            const int64_t v_strides[4], const int64_t gate_strides[4],
                            const int64_t out_strides[4], int batch, int q_heads, int kv_heads,
                            int seq_len, int head_dim, float scale, const int32_t* cu_seqlens,
                            int n_seqs, int max_seqlen, void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * Attention prologue: per-head RMSNorm of q and k over head_dim, then the
 * rotary embedding of the first rotary_dim features, replacing the eager
 * q_norm / k_norm / apply_rotary_pos_emb of the patched attention forward
 * (ref: experiments/native_gqa/bench_native_gqa_model.py:47-53; transformers
 * Qwen3_5RMSNorm and apply_rotary_pos_emb):
 *   y   = bf16((x * (1 / sqrt(mean(x^2) + eps))) * g),  g = 1 + w (gain_offset) or w
 *   out = bf16(bf16(y_i * cos_i) + bf16(rot_i * sin_i)) for i < rotary_dim,
 *         rot = (-y[R/2:R], y[0:R/2]);  out_i = y_i for i >= rotary_dim
 * fp32 arithmetic; the sum of squares in the order PyTorch's GPU row mean uses
 * at width 128 and the inverse root evaluated in fp64 and rounded to fp32, so the
 * rows equal the eager ops on the GPU bit for bit.
 *
 *   q_in  token t, head h at q_in + t*q_token_stride + h*q_head_stride (bf16, 128 contiguous)
 *         (e.g. the query half of the q_proj output [tokens, q_heads, 2*head_dim])
 *   k_in  likewise with k_token_stride, k_head_stride
 *   q_weight, k_weight  [head_dim] of weight_dtype (FD_DTYPE_BF16 or FD_DTYPE_F32)
 *   cos, sin  [tokens, rotary_dim] bf16 contiguous (NULL when rotary_dim == 0)
 *   q_out [tokens, q_heads, head_dim], k_out [tokens, kv_heads, head_dim] bf16 contiguous
 *
 * Limits: head_dim == 128; rotary_dim in {0, 16, 32, 64, 128}; 16-byte aligned
 * pointers and strides that are multiples of 8 elements.
 */
FD_API int fd_attn_prologue_fwd(const void* q_in, int64_t q_token_stride, int64_t q_head_stride,
                                const void* k_in, int64_t k_token_stride, int64_t k_head_stride,
                                const void* q_weight, const void* k_weight, int weight_dtype,
                                int gain_offset, float eps, const void* cos, const void* sin,
                                int rotary_dim, void* q_out, void* k_out, int64_t tokens, int q_heads,
                                int kv_heads, int head_dim, void* stream);

/*
 * Packed causal depthwise conv1d + activation with a head-split store.
 *
 *   x      [batch, seq_len, C] bf16 contiguous, C = 2*key_dim + value_dim
 *   weight [C, width] bf16 contiguous (tap `width-1` multiplies the current token)
 *   bias   [C] bf16 or NULL
 *   q, k   [batch, seq_len, key_dim] bf16 contiguous (any head split of key_dim)
 *   v      [batch, seq_len, value_dim] bf16 contiguous
 *
 * y[t, c] = act(w[c, W-1]*x[t, c] + w[c, 0]*x[t-W+1, c] + ... + w[c, W-2]*x[t-1, c] + bias[c])
 * with the taps of the reference (ref: src/decider/packed_conv_kernel.py:139-177):
 * the W products are summed exactly (in fp64; products of two bf16 values are
 * exact) and rounded once to fp32, the bias is added in fp32, SiLU is
 * y / (1 + expf(-y)) in fp32 (ref: :178-182), then one bf16 rounding.  This is
 * PyTorch's fp32 GPU conv1d + SiLU, then a cast, bit for bit (BASELINE config 2's
 * definition; any fp32 tap order, the reference kernel's included, differs from
 * it on about 0.3 % of outputs).  Taps before the start of the sequence read
 * zero (ref: :128-176); channels [0, key_dim) go to q, the next key_dim to k,
 * the rest to v (ref: :184-191).
 *
 * Varlen: cu_seqlens (device int32[n_seqs + 1]) with batch == 1 restarts the
 * causal window at every request start.
 *
 * Limits: width in [1, 4]; key_dim, value_dim multiples of 8; all pointers
 * 16-byte aligned (as ref: src/decider/packed_conv_kernel.py:211-212).
 */
FD_API int fd_packed_conv_fwd(const void* x, const void* weight, const void* bias, void* q,
                       void* k, void* v, int batch, int seq_len, int key_dim,
                       int value_dim, int width, const int32_t* cu_seqlens, int n_seqs,
                       int activation, void* stream);

/*
 * fd_packed_conv_fwd on x rows x_row_stride elements apart (a multiple of 8, >= C):
 * the q|k|v channels may be the first C columns of a wider combined projection
 * output.  Other arguments and limits as fd_packed_conv_fwd.
 */
FD_API int fd_packed_conv_strided_fwd(const void* x, int64_t x_row_stride, const void* weight,
                                      const void* bias, void* q, void* k, void* v, int batch,
                                      int seq_len, int key_dim, int value_dim, int width,
                                      const int32_t* cu_seqlens, int n_seqs, int activation,
                                      void* stream);

/*
 * fd_packed_conv_strided_fwd (SiLU, no bias) and fd_gate_proj_fwd of the same
 * Gated-DeltaNet layer in one launch.  The two are independent; the gate
 * projection alone is a small latency-bound launch, so here its workgroups run
 * beside the conv's instead of after them.  No counterpart in the reference:
 * it stands for its prep_qkv (ref: src/decider/packed_conv_kernel.py:194-232)
 * followed by the combined gate projection and unpack_gate
 * (ref: src/decider/combined_gates.py:19-43,
 *  ref: src/decider/unpack_gate_transform_kernel.py:94-133).
 *
 *   x .. n_seqs          as fd_packed_conv_strided_fwd (activation SiLU, bias NULL);
 *   hidden_states        token r at hidden_states + r*hidden_row_stride, [hidden] bf16
 *                        (batch*seq_len tokens: the layer input the a|b projection reads)
 *   gate_weight .. heads as fd_gate_proj_fwd (ab not written)
 *
 * q, k, v, g and beta are bit-identical to fd_packed_conv_strided_fwd followed
 * by fd_gate_proj_fwd.  Limits: the union of both.
 */
FD_API int fd_packed_conv_gate_fwd(const void* x, int64_t x_row_stride, const void* weight, void* q,
                                   void* k, void* v, int batch, int seq_len, int key_dim,
                                   int value_dim, int width, const int32_t* cu_seqlens, int n_seqs,
                                   const void* hidden_states, int64_t hidden_row_stride,
                                   const void* gate_weight, int hidden, const void* a_log,
                                   int a_log_dtype, const void* dt_bias, int dt_bias_dtype, float* g,
                                   void* beta, int heads, void* stream);

/*
 * Numerics self-check of the conv's SiLU; no counterpart in the reference.
 * The conv kernels evaluate SiLU with the hardware exp2 and reciprocal and
 * fall back to y / (1 + expf(-y)) (the expression PyTorch's fp32 SiLU
 * evaluates) where the two could round to different bf16 values.  This entry
 * point adds to *mismatches (a device uint64 the caller zeroes) the number of
 * fp32 bit patterns in [begin, begin + count) whose two bf16 roundings differ
 * (both NaN counts as equal).  The GPU tests run it over all 2^32 patterns
 * and require 0.
 */
FD_API int fd_silu_check(uint32_t begin, uint32_t count, unsigned long long* mismatches, void* stream);

/*
 * Numerics self-check of fd_gated_rmsnorm_fwd with a bf16 weight (no
 * counterpart in the reference): its last product out = bf16(y2 * silu(z))
 * takes y2 and z as bf16 values and runs on the hardware exp2 and reciprocal,
 * with the exact y2 * (z / (1 + expf(-z))) where the bf16 roundings could
 * differ.  Adds to *mismatches (device unsigned long long) the number of pairs
 * (y2, z) = (bf16 bits i >> 16, bf16 bits i & 0xffff), i in [begin, begin + count),
 * where the two bf16 roundings differ (both NaN counts as equal).
 * begin + count <= 2^32.  The GPU test runs all 2^32 pairs and requires 0.
 */
FD_API int fd_gated_silu_check(uint32_t begin, uint32_t count, unsigned long long* mismatches, void* stream);

/*
 * Streaming device copy of `bytes` (a multiple of 16; src and dst 16-byte
 * aligned, not overlapping) with nontemporal 16-byte loads and stores, each
 * thread moving `chunks_per_thread` (1, 2 or 4) chunks in workgroups of
 * `block` (256 or 512) threads; no counterpart in the reference.  It is the
 * copy of known traffic that bench.py measures at each bandwidth-bound
 * kernel's byte count (the best of its shapes), so that those kernels are set
 * against a ceiling measured on the same box and not only against the
 * 8 TB/s published peak.
 */
FD_API int fd_hbm_copy(const void* src, void* dst, int64_t bytes, int chunks_per_thread, int block, void* stream);

/*
 * Fused residual add + RMSNorm over rows of `width` features.
 *
 *   h            = bf16(x + residual)            (residual == NULL: h = x)
 *   residual_out = h                             (skipped when NULL; may alias x or residual)
 *   out          = bf16((f32(h) * rsqrt(mean(f32(h)^2) + eps)) * g),
 *                  g = 1 + weight (gain_offset = 1, Qwen3.5 form) or weight (0)
 *
 * x, residual, out, residual_out: [rows, width] bf16 contiguous; weight:
 * [width] of weight_dtype (FD_DTYPE_BF16 or FD_DTYPE_F32).  fp32 accumulation
 * in a fixed order; mean = sum * fl(1 / width); the inverse root evaluated in
 * fp64 and rounded to fp32.  For widths that are a multiple of 1024 the order is the one
 * PyTorch's GPU row mean uses at width 2048, so at that width `out` equals
 * eager Qwen3_5RMSNorm on the GPU bit for bit.  out may alias x.
 *
 * Limits: width a multiple of 8 in [8, 8192]; pointers 16-byte aligned.
 */
FD_API int fd_add_rmsnorm_fwd(const void* x, const void* residual, const void* weight, void* out,
                       void* residual_out, int64_t rows, int width, float eps,
                       int weight_dtype, int gain_offset, void* stream);

/*
 * Bytes of device workspace fd_gated_delta_fwd needs for these sizes
 * (n_seqs = number of packed requests with cu_seqlens, 0 for a padded batch),
 * or a negative FD_ERR_* code.
 */
FD_API int64_t fd_gated_delta_workspace_bytes(int batch, int seq_len, int v_heads, int head_k_dim,
                                              int head_v_dim, int n_seqs);

/*
 * Chunked gated delta rule forward (the linear attention of the decider's
 * Gated-DeltaNet layers), fp32 arithmetic, bf16 in/out.  Replaces the
 * reference call of transformers' torch_chunk_gated_delta_rule
 * (ref: src/decider/packed_conv.py:55-59; transformers modeling_qwen3_5.py:249-328).
 *
 *   q, k  [batch, seq_len, k_heads, head_k_dim] bf16 contiguous
 *   v     [batch, seq_len, v_heads, head_v_dim] bf16 contiguous
 *   g     [batch, seq_len, v_heads] fp32 (log decay, <= 0)
 *   beta  [batch, seq_len, v_heads] of beta_dtype (FD_DTYPE_BF16 or FD_DTYPE_F32)
 *   out   [batch, seq_len, v_heads, head_v_dim] bf16
 *   initial_state, final_state  [n, v_heads, head_k_dim, head_v_dim] fp32 or NULL
 *                               (n = batch, or n_seqs with cu_seqlens)
 *
 * Value head h uses key head h / (v_heads / k_heads).  With l2norm_qk, q and k
 * rows are first normalised as transformers' l2norm does on bf16 tensors
 * (eps 1e-6, every step rounded to bf16); q is then scaled by `scale`.  Per
 * value head, with state S [head_k_dim, head_v_dim] (zero or initial_state):
 *   S <- e^{g_t} S;  S <- S + k_t (beta_t (v_t - S^T k_t))^T;  out_t = S^T q_t
 * evaluated in 64-token chunks as the reference does.  Varlen: cu_seqlens
 * (device int32[n_seqs + 1], non-decreasing, from 0 to seq_len) with batch == 1;
 * each request starts from its own state and no state crosses a request.
 * Work runs in `workspace` (fd_gated_delta_workspace_bytes, 16-byte aligned).
 *
 * Limits: head_k_dim == head_v_dim == 128; v_heads % k_heads == 0;
 * batch * seq_len < 2^31.
 */
FD_API int fd_gated_delta_fwd(const void* q, const void* k, const void* v, const float* g,
                              const void* beta, void* out, const float* initial_state,
                              float* final_state, void* workspace, int64_t workspace_bytes,
                              int batch, int seq_len, int k_heads, int v_heads, int head_k_dim,
                              int head_v_dim, float scale, int beta_dtype, int l2norm_qk,
                              const int32_t* cu_seqlens, int n_seqs, void* stream);

/* Bytes of the static device scratch fd_gated_delta_fwd_noalloc works in (80 MiB: the
 * decider's B=1, T=2048 call with 16 value heads, 72.4 MiB, and a few chunks of margin). */
#define FD_GD_SCRATCH_BYTES 83886080LL

/*
 * fd_gated_delta_fwd without a workspace argument: the work runs in a static
 * device array of FD_GD_SCRATCH_BYTES that the library holds on every GPU it
 * runs on until the process ends, and the call allocates no memory.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The caller still passes inputs and outputs.
 *
 * Limit: fd_gated_delta_workspace_bytes of the same sizes must not exceed
 * FD_GD_SCRATCH_BYTES (the decider's B=1, T=2048, 16-value-head call needs
 * about 73 MiB), else FD_ERR_UNSUPPORTED.  Every call on one GPU shares that
 * GPU's scratch: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller.  The scratch needs no clearing:
 * each call writes every byte it reads.  The first call on a device looks the
 * scratch's address up with that device current (the stream's device).
 * Other arguments, results and limits as fd_gated_delta_fwd.
 */
FD_API int fd_gated_delta_fwd_noalloc(const void* q, const void* k, const void* v, const float* g,
                                      const void* beta, void* out, const float* initial_state,
                                      float* final_state, int batch, int seq_len, int k_heads, int v_heads,
                                      int head_k_dim, int head_v_dim, float scale, int beta_dtype,
                                      int l2norm_qk, const int32_t* cu_seqlens, int n_seqs, void* stream);

/*
 * fd_gated_delta_fwd followed by the layer's gated RMSNorm (transformers
 * Qwen3_5RMSNormGated, the call after the delta rule at ref: src/decider/packed_conv.py:60-61),
 * applied to each (token, head) row of 128 (the delta rule's rows go to the workspace,
 * and fd_gated_rmsnorm_fwd's kernel normalises them into `out`):
 *   x = bf16(delta-rule output);  y = bf16(x / sqrt(mean(x^2) + eps));
 *   y2 = bf16(w * y) (fp32 for an fp32 weight);  out = bf16(y2 * z / (1 + exp(-z)))
 * the same values fd_gated_delta_fwd then fd_gated_rmsnorm_fwd produce.
 *   z  gate of token row r (the batch's flattened token index), value head h at
 *      z + r * z_token_stride + h * z_head_stride (bf16, 128 contiguous; e.g. part of a
 *      combined projection output)
 *   norm_weight [128] of norm_weight_dtype (FD_DTYPE_BF16 or FD_DTYPE_F32)
 * Other arguments and limits as fd_gated_delta_fwd; z strides multiples of 8 elements.
 */
FD_API int fd_gated_delta_norm_fwd(const void* q, const void* k, const void* v, const float* g,
                                   const void* beta, const void* z, int64_t z_token_stride,
                                   int64_t z_head_stride, const void* norm_weight, int norm_weight_dtype,
                                   float norm_eps, void* out, const float* initial_state,
                                   float* final_state, void* workspace, int64_t workspace_bytes,
                                   int batch, int seq_len, int k_heads, int v_heads, int head_k_dim,
                                   int head_v_dim, float scale, int beta_dtype, int l2norm_qk,
                                   const int32_t* cu_seqlens, int n_seqs, void* stream);

/*
 * Gate transform of the Gated-DeltaNet layers (ref: src/decider/unpack_gate_transform_kernel.py:51-91,
 * the eager form at ref: src/decider/packed_conv.py:49-53):
 *   g[r, h]    = -exp(a_log[h]) * softplus(a[r, h] + dt_bias[h])   fp32
 *                softplus(x) = x > 20 ? x : log1p(exp(x))
 *   beta[r, h] = bf16(1 / (1 + exp(-b[r, h])))
 * fp32 arithmetic with the same library exp / log1p as PyTorch's elementwise kernels.
 *
 *   a, b          [rows, heads] bf16 with row strides a_row_stride, b_row_stride
 *                 (elements; a and b may be the two halves of one combined
 *                 projection output, ref: src/decider/combined_gates.py:19-43)
 *   a_log, dt_bias [heads] of a_log_dtype / dt_bias_dtype (FD_DTYPE_BF16 or FD_DTYPE_F32)
 *   g             [rows, heads] fp32 contiguous
 *   beta          [rows, heads] bf16 contiguous
 */
FD_API int fd_gate_transform_fwd(const void* a, const void* b, int64_t a_row_stride,
                                 int64_t b_row_stride, const void* a_log, int a_log_dtype,
                                 const void* dt_bias, int dt_bias_dtype, float* g, void* beta,
                                 int64_t rows, int heads, void* stream);

/*
 * The combined a|b gate projection of a Gated-DeltaNet layer fused with the
 * gate transform: the reference's F.linear(x, cat(in_proj_a.weight,
 * in_proj_b.weight)) followed by unpack_gate (ref: src/decider/combined_gates.py:19-43,
 * src/decider/packed_conv.py:45-53), in one launch:
 *   a = bf16(x . W[h]),  b = bf16(x . W[heads + h])   (bf16 products, fp32 sums)
 *   g, beta as fd_gate_transform_fwd on those a, b
 *
 *   x        token r at x + r*x_row_stride, [hidden] bf16 contiguous
 *   weight   [2*heads, hidden] bf16 contiguous (a rows, then b rows)
 *   g        [rows, heads] fp32, beta [rows, heads] bf16 (contiguous)
 *   ab       NULL or [rows, 2*heads] bf16: the a|b values the transform used
 *
 * Limits: heads in {8, 16, 24, 32}; hidden a multiple of 128; x rows and
 * weight 16-byte aligned.  The fp32 sums run in one fixed order whatever the
 * number of tokens: 4 parts, part p taking the 32-wide slice 128 j + 32 p of
 * every 128-deep block j on one MFMA accumulator, then ((p0 + p1) + p2) + p3,
 * the order hipBLASLt's bf16 GEMM uses for a 16-output projection on the
 * MI355X.  With 16 heads a and b therefore equal the eager in_proj_a /
 * in_proj_b outputs bit for bit; other GEMMs can differ by one bf16 ulp where
 * a sum lies near a rounding boundary.
 */
FD_API int fd_gate_proj_fwd(const void* x, int64_t x_row_stride, const void* weight, int hidden,
                            const void* a_log, int a_log_dtype, const void* dt_bias, int dt_bias_dtype,
                            float* g, void* beta, void* ab, int64_t rows, int heads, void* stream);

/*
 * Slot-only readout: for each slot n (hidden row slot_rows[n], position
 * slot_positions[n]) the model's final RMSNorm, the option-letter projection
 * and the masked softmax at temperature (ref: src/decider/slot_projection.py:6-21,
 * src/decider/engine.py:48-56, src/decider/temperature.py:136-144):
 *   y         = bf16((x * (1 / sqrt(mean(x^2) + eps))) * g),  g = 1 + w (gain_offset) or w
 *   logits[n] = bf16(y . letters[k]) for every letter k           (F.linear on bf16)
 *   probs[n]  = softmax(logits[n, :nopts[n]] / temperature), 0 for k >= nopts[n]
 * fp32 arithmetic; for widths that are a multiple of 256 the sum of squares runs
 * in the order PyTorch's GPU row mean uses (y then equals eager's normed row bit
 * for bit), the inverse root evaluated in fp64 and rounded to fp32; slots outside
 * [0, batch) x [0, seq_len) read row 0, position 0.
 *
 *   hidden   [batch, seq_len, width] bf16 contiguous (the residual stream before the final norm)
 *   norm_weight [width] of weight_dtype;  letters [n_letters, width] bf16 contiguous
 *   slot_rows, slot_positions [n_slots] int32 (device);  nopts [n_slots] int32 or NULL (all letters)
 *   logits   [n_slots, n_letters] fp32;  probs [n_slots, n_letters] fp32 or NULL
 *
 * Limits: width a multiple of 8 in [8, 8192]; n_letters in [1, 1024].
 */
FD_API int fd_slot_readout_fwd(const void* hidden, int batch, int seq_len, int width,
                               const void* norm_weight, int weight_dtype, int gain_offset, float eps,
                               const void* letters, int n_letters, const int32_t* slot_rows,
                               const int32_t* slot_positions, const int32_t* nopts, int n_slots,
                               float temperature, float* logits, float* probs, void* stream);

/*
 * Gated RMSNorm of the Gated-DeltaNet output (transformers Qwen3_5RMSNormGated,
 * called after the delta rule, ref: src/decider/packed_conv.py:60-61), eager rounding:
 *   y = bf16(x / sqrt(mean(x^2) + eps));  y2 = bf16(w * y) (fp32 for an fp32 weight);
 *   out = bf16(y2 * z / (1 + exp(-z)))
 * x, out [rows, width] bf16 contiguous, rows = tokens * heads (row r = token r / heads,
 * head r % heads); gate z of row r at gate + token*gate_token_stride + head*gate_head_stride
 * (elements: a [tokens, heads, width] view, e.g. part of a combined projection output);
 * weight [width] of weight_dtype.  The sum of squares runs in the order PyTorch's GPU
 * row mean uses at these widths and the inverse root is evaluated in fp64 and rounded
 * to fp32, so `out` equals eager Qwen3_5RMSNormGated on the GPU bit for bit.
 * Limits: width in {64, 128, 256}; 16-byte aligned pointers, strides multiples of 8.
 */
FD_API int fd_gated_rmsnorm_fwd(const void* x, const void* gate, int64_t gate_token_stride,
                                int64_t gate_head_stride, int heads, const void* weight, int weight_dtype,
                                void* out, int64_t rows, int width, float eps, void* stream);

/*
 * The MLP's activation (transformers Qwen3_5MLP: act_fn(gate_proj(x)) * up_proj(x)) on a
 * combined projection gate_up [rows, row_stride] holding gate in columns [0, width)
 * and up in [width, 2*width):  out = bf16(bf16(silu(gate)) * up), out [rows, width].
 * Limits: width a multiple of 8; 16-byte aligned pointers and row_stride a multiple of 8.
 */
FD_API int fd_silu_mul_fwd(const void* gate_up, int64_t row_stride, void* out, int64_t rows, int width,
                           void* stream);

/*
 * fd_silu_mul_fwd over two gate|up projections: output features [0, width1) come
 * from gate_up1 (gate in its columns [0, width1), up in [width1, 2*width1)), the
 * next width2 from gate_up2 likewise; out [rows, width1 + width2] contiguous.
 * Each feature is computed exactly as fd_silu_mul_fwd computes it.  No
 * counterpart in the reference: the MLP's combined gate|up GEMM runs as two
 * GEMMs whose widths hipBLASLt tiles better (transformers Qwen3_5MLP).
 * width2 == 0 (gate_up2 unused) is fd_silu_mul_fwd.
 * Limits: widths multiples of 8; 16-byte aligned pointers, row strides multiples of 8.
 */
FD_API int fd_silu_mul_split_fwd(const void* gate_up1, int64_t row_stride1, int width1,
                                 const void* gate_up2, int64_t row_stride2, int width2, void* out,
                                 int64_t rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FD_KERNELS_H */

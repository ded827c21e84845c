/*
 * kai_gdn_hip.h -- device-pointer entry points of libkai_gdn_hip.so (gfx950).
 *
 * The four kai_run_gdn_* symbols of include/kai/ukernels/gdn/ are the
 * drop-in boundary (host or device pointers, synchronous).  The functions
 * below are the stream-ordered forms a GPU caller uses: every pointer is
 * device memory, work is enqueued on `stream` (a hipStream_t; NULL = the
 * null stream) and the call returns without waiting.  They return 0 on
 * success or a hipError_t code; kai_gdn_hip_error_string() names it.
 * Argument checks happen before anything is enqueued: on an error nothing
 * is written.
 *
 * Names keep the kai pattern kai_run_<op>_<types>_<isa>
 * (kleidiai_submission/README.md:122-142) with isa = hip.
 */
#ifndef KAI_GDN_HIP_H
#define KAI_GDN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kai ukernels, device pointers -------------------------------------- */

/* Replaces kai_run_gdn_cumdecay_f32_sve
 * (kleidiai_submission/kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.h:33-34).
 * The cumulative decay and gated scan entry points below run a single-pass
 * look-back scan whose waits are bounded: a wait that gives up marks that
 * launch's output invalid and sets a device error word, which the caller
 * reads with kai_gdn_hip_check_device_error() (the synchronous kai symbols
 * check it themselves and exit(1)). */
int kai_run_gdn_cumdecay_f32_hip(const float *a, float *decay, size_t seq,
                                 size_t channels, void *stream);

/* No counterpart in the reference.  kai_run_gdn_cumdecay_f32_hip without any
 * allocation, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops): the look-back scan's scratch is a
 * fixed array in the library's device code (about 6 MiB per GPU, held until
 * the process ends) instead of memory allocated on first use.  It covers
 * ceil(seq / 128) * channels <= KAI_GDN_NOALLOC_SCAN_MAX_WORDS (for example
 * seq = 4096, channels = 8192); larger shapes return hipErrorInvalidValue
 * without writing anything.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU race, so order them (one stream, or
 * synchronise between streams).  A timed-out look-back wait is reported by
 * kai_gdn_hip_check_device_error().  The first call on a device (or
 * kai_gdn_hip_init on it) sets the scratch up and synchronises the device. */
#define KAI_GDN_NOALLOC_SCAN_MAX_WORDS 262144
int kai_run_gdn_cumdecay_f32_noalloc_hip(const float *a, float *decay, size_t seq,
                                         size_t channels, void *stream);

/* Replaces kai_run_gdn_gated_scan_f32_sve (kai_gdn_gated_scan_f32_sve.h:35-36). */
int kai_run_gdn_gated_scan_f32_hip(const float *g, const float *x, float *s,
                                   float *state, size_t seq, size_t channels,
                                   void *stream);

/* Replaces kai_run_gdn_causal_dwconv1d_f32_k4_sve
 * (kai_gdn_causal_dwconv1d_f32_k4_sve.h:39-41). */
int kai_run_gdn_causal_dwconv1d_f32_k4_hip(const float *in, const float *w,
                                           float *out, float *hist, size_t seq,
                                           size_t channels, void *stream);

/* The same conv with the SiLU epilogue out = y / (1 + exp(-y)) fused, as HF
 * Qwen3.5 applies after the depthwise conv (transformers
 * modeling_qwen3_5.py:222-239, activation="silu").  No reference kai symbol. */
int kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(const float *in, const float *w,
                                                float *out, float *hist, size_t seq,
                                                size_t channels, void *stream);

/* Replaces kai_run_gdn_gemv_f32_f32_f32_1x4_neon
 * (kai_gdn_gemv_f32_f32_f32_1x4_neon.h:40-42). */
int kai_run_gdn_gemv_f32_f32_f32_hip(const float *a, const float *b, float *c,
                                     size_t k, size_t n, void *stream);

/* Replaces gdn_delta_rule_matmul
 * (src/orionsbelt/engines/cpu/kernels/gdn_delta_matmul.h:15-16) on the
 * caller's stream: C[M][N] = A[M][K] . B[K][N], row-major fp32, each element
 * the k-ordered sum of rounded products.  K == 0 writes zeros. */
int kai_run_gdn_delta_rule_matmul_f32_hip(const float *A, const float *B, float *C, size_t M,
                                          size_t K, size_t N, void *stream);

/* ---- mixed-precision diagonal kernels (gdn_sve.h:56-72) ------------------
 * fp16 values are IEEE binary16 bit patterns, bf16 values the upper half of a
 * binary32 (round to nearest even), both passed as uint16_t.  fp32
 * accumulation; only the narrow array is narrowed (gdn_sve.c:433-441). */
int kai_run_gdn_cumdecay_f16_hip(const float *a, uint16_t *decay, size_t seq,
                                 size_t channels, void *stream);
int kai_run_gdn_cumdecay_bf16_hip(const float *a, uint16_t *decay, size_t seq,
                                  size_t channels, void *stream);
int kai_run_gdn_gated_scan_f16_hip(const float *g, const float *x, float *s,
                                   uint16_t *state, size_t seq, size_t channels,
                                   void *stream);
int kai_run_gdn_gated_scan_bf16_hip(const float *g, const float *x, float *s,
                                    uint16_t *state, size_t seq, size_t channels,
                                    void *stream);

/* GDN-2 decoupled-gating scan (gdn2_gated_scan_f32, gdn_sve.h:83-86):
 *   s[t][c] = w[t][c] * x[t][c] + s[t-1][c] * (g[t][c] * b[t][c]),
 * both products rounded before the sum (gdn_sve.c:861-874); state[]
 * carried across calls.  The products are formed into library-owned device
 * buffers (2 * seq * channels floats, kept for later calls), then the
 * gated scan runs over them. */
int kai_run_gdn2_gated_scan_f32_hip(const float *g, const float *b_gate, const float *w_gate,
                                    const float *x, float *s, float *state, size_t seq,
                                    size_t channels, void *stream);

/* ---- matrix-state gated delta rule, single-token decode ------------------
 * Replaces the OpenCL gdn_delta_rule_decode (gpu/gdn_gpu_kernels.cl:158-206)
 * and its host oracle ref_delta_rule (gpu/gdn_gpu_validate.c:100-118), with
 * per-(sequence, value-head) gates as HF torch_recurrent_gated_delta_rule
 * uses them (modeling_qwen3_5.py:331-380).  For every sequence b and value
 * head h (key head kh = h / (num_v_heads / num_k_heads)):
 *     S *= exp(g[b][h]);  kv = S^T k;  delta = (v - kv) * beta[b][h];
 *     S += k (x) delta;   o = S^T (q * q_scale)
 * Layouts: S [batch][num_v_heads][head_k_dim][head_v_dim] (in/out),
 * q,k [batch][num_k_heads][head_k_dim], v,o [batch][num_v_heads][head_v_dim],
 * g,beta [batch][num_v_heads].  q and k are used as given (L2-normalise
 * them beforehand, as HF does with use_qk_l2norm_in_kernel).
 * head_k_dim, head_v_dim in {32, 64, 128}; num_v_heads % num_k_heads == 0. */
int kai_run_gdn_delta_rule_decode_f32_hip(float *S, const float *q, const float *k,
                                          const float *v, const float *g,
                                          const float *beta, float *o, int batch,
                                          int num_v_heads, int num_k_heads,
                                          int head_k_dim, int head_v_dim,
                                          float q_scale, void *stream);

/* Same step with S stored as IEEE fp16 (bit patterns): widened to fp32 on
 * load, narrowed (round to nearest even) on store.  Halves the state
 * footprint and the bytes the step moves. */
int kai_run_gdn_delta_rule_decode_f16state_hip(uint16_t *S, const float *q,
                                               const float *k, const float *v,
                                               const float *g, const float *beta,
                                               float *o, int batch, int num_v_heads,
                                               int num_k_heads, int head_k_dim,
                                               int head_v_dim, float q_scale,
                                               void *stream);

/* ---- chunkwise (WY) gated delta rule, prefill ----------------------------
 * The algorithm of HF torch_chunk_gated_delta_rule (modeling_qwen3_5.py:
 * 248-328) with chunk size 64: per chunk, the UT transform
 * T = (I + tril(beta K K^T * Gamma, -1))^-1, W = T (beta K e^G),
 * U = T (beta V) and the masked Q K^T, then the state recurrence.  The
 * recurrence is affine in the state, so long sequences are cut into segments
 * that run in parallel (each segment's transition is composed with its
 * predecessors'), then rerun from their true start states.  q,k,v bf16 (bit
 * patterns), products on bf16 MFMA with fp32 accumulation, fp32 state.
 * Layouts (token-major, HF's [B, T, H, D]):
 *   q,k [batch][seq_len][num_k_heads][128]   v [batch][seq_len][num_v_heads][128]
 *   g,beta [batch][seq_len][num_v_heads] fp32 (g = log-gate, beta = write gate)
 *   o [batch][seq_len][num_v_heads][128] bf16
 *   S [batch][num_v_heads][128][128] fp32: initial state in, final state out.
 * seq_len need not be a multiple of 64.  head_k_dim = head_v_dim = 128.
 * Results depend on where a sequence is cut into segments only within the
 * bf16 rounding bound; calls on one device must not overlap (they share a
 * carry buffer; calls on one stream never do). */
int kai_run_gdn_chunk_delta_rule_bf16_f32_hip(const uint16_t *q, const uint16_t *k,
                                              const uint16_t *v, const float *g,
                                              const float *beta, uint16_t *o,
                                              float *S, int batch, int seq_len,
                                              int num_v_heads, int num_k_heads,
                                              float q_scale, void *stream);

/* Same prefill with S stored as IEEE fp16 bit patterns (widened on entry,
 * fp32 across all chunks, narrowed once on exit). */
int kai_run_gdn_chunk_delta_rule_bf16_f16state_hip(const uint16_t *q,
                                                   const uint16_t *k,
                                                   const uint16_t *v, const float *g,
                                                   const float *beta, uint16_t *o,
                                                   uint16_t *S, int batch,
                                                   int seq_len, int num_v_heads,
                                                   int num_k_heads, float q_scale,
                                                   void *stream);

/* ---- layer glue on either side of the recurrence ------------------------
 * No reference kai symbol: the reference's layer runs these steps in its CPU
 * model code; the definitions are HF transformers modeling_qwen3_5.py
 * (Qwen3_5GatedDeltaNet.forward:481-502, l2norm:242-245,
 * Qwen3_5RMSNormGated:168-184), which the reference documents at
 * docs/GDN_LAYER_AUDIT.md:138-163.  Head dims are 128.
 *
 * Gating prologue.  x [rows][(2 Hk + Hv) * 128] fp32 is the conv+SiLU output
 * of rows = batch * seq_len tokens, channels ordered q heads, k heads, v heads
 * (HF's torch.split of the conv output); a, b [rows][Hv] fp32 are the in_proj_a
 * and in_proj_b outputs; A_log, dt_bias [Hv].  Writes
 *   q, k [rows][Hk][128] = x_head / sqrt(sum x_head^2 + 1e-6)
 *   v [rows][Hv][128]    = x_head
 *   g [rows][Hv]    = -exp(A_log) * softplus(a + dt_bias)  (threshold 20)
 *   beta [rows][Hv] = sigmoid(b)
 * in the layouts the recurrence entry points read (bf16 bit patterns for the
 * prefill, fp32 for the decode step).  The 1/sqrt(128) query scale is the
 * recurrence's q_scale argument (HF applies it after the norm), and the GQA
 * repeat_interleave is not materialised: value head h reads key head
 * h / (Hv / Hk).  x, q, k, v 16-byte aligned; Hv % Hk == 0. */
int kai_run_gdn_gating_prologue_bf16_hip(const float *x, const float *a, const float *b,
                                         const float *A_log, const float *dt_bias,
                                         uint16_t *q, uint16_t *k, uint16_t *v, float *g,
                                         float *beta, size_t rows, int num_k_heads,
                                         int num_v_heads, void *stream);
int kai_run_gdn_gating_prologue_f32_hip(const float *x, const float *a, const float *b,
                                        const float *A_log, const float *dt_bias, float *q,
                                        float *k, float *v, float *g, float *beta,
                                        size_t rows, int num_k_heads, int num_v_heads,
                                        void *stream);
/* Gated RMSNorm epilogue: for each of `rows` rows of 128 values (rows =
 * batch * seq_len * num_v_heads, the recurrence output o and the in_proj_z
 * gate z in the same layout), y = w * (o / sqrt(mean(o^2) + eps)) * silu(z).
 * The bf16 form rounds as HF's module does in a bf16 model: the normalised
 * row to bf16, its product with w to bf16, the final product to bf16.
 * y is the input of out_proj.  Pointers 16-byte aligned; eps >= 0
 * (Qwen3.5: 1e-6). */
int kai_run_gdn_gated_rmsnorm_bf16_hip(const uint16_t *o, const uint16_t *z,
                                       const uint16_t *w, uint16_t *y, size_t rows,
                                       float eps, void *stream);
int kai_run_gdn_gated_rmsnorm_f32_hip(const float *o, const float *z, const float *w,
                                      float *y, size_t rows, float eps, void *stream);
/* ---- state formats of the prefill -> decode hand-off ----------------------
 * No reference kai symbol.  HF keeps a GDN layer's cache as conv_state
 * [batch][channels][4] (the last four conv inputs of each sequence, newest
 * last, zero-padded after a prefill shorter than four tokens;
 * transformers cache_utils.py LinearAttentionLayer.update_conv_state:
 * 1032-1070) and the recurrent state [batch][Hv][128][128] in the model
 * dtype.  The kai conv carries hist [3][channels] per sequence, oldest
 * first (kai_gdn_causal_dwconv1d_f32_k4_sve.h:28-36).  Pointers to
 * conv_state and w are 16-byte aligned; batch <= 65535. */

/* HF causal_conv1d_update (modeling_qwen3_5.py:199-217) for a batch of
 * sequences: x, out [batch][seq_len][channels] (token-major, as in_proj
 * writes it), conv_state [batch][channels][4] updated in place, w
 * [channels][4] (HF's conv1d.weight.squeeze(1)).  For each token:
 *   out = ((s1*w0 + s2*w1) + s3*w2) + x*w3,  then SiLU if silu != 0,
 *   state <- (s1, s2, s3, x)
 * in the kai reference's order without contraction, so decode steps that
 * continue a sequence are bit-identical to the kai conv over the whole
 * sequence.  out may equal x. */
int kai_run_gdn_causal_conv1d_update_f32_hip(const float *x, float *conv_state,
                                             const float *w, float *out, int batch,
                                             int seq_len, size_t channels, int silu,
                                             void *stream);
/* conv_state [batch][channels][4] after a prefill of seq_len tokens whose
 * conv inputs are x [batch][seq_len][channels]: the last four rows, zero
 * where seq_len < 4 (HF's prefill path of update_conv_state). */
int kai_run_gdn_conv_state_from_inputs_f32_hip(const float *x, float *conv_state,
                                               int batch, size_t seq_len,
                                               size_t channels, void *stream);
/* conv_state [batch][channels][4] -> hist [batch][3][channels] (entries
 * 1..3, oldest first) and back.  Entry 0 of the HF state, the input four
 * steps back, feeds no later output; hist -> state writes it as 0. */
int kai_run_gdn_conv_state_to_hist_f32_hip(const float *conv_state, float *hist,
                                           int batch, size_t channels, void *stream);
int kai_run_gdn_conv_hist_to_state_f32_hip(const float *hist, float *conv_state,
                                           int batch, size_t channels, void *stream);
/* Element format conversion of `count` values (a recurrent state, e.g. fp32
 * from the prefill to the fp16-state decode step): formats below, narrowing
 * to nearest even (bf16 by the reference's rule, gdn_sve.c:81-87).  src and
 * dst must not overlap unless they are the same array in the same format. */
#define KAI_GDN_FMT_F32 0
#define KAI_GDN_FMT_F16 1
#define KAI_GDN_FMT_BF16 2
int kai_run_gdn_state_convert_hip(const void *src, int src_format, void *dst,
                                  int dst_format, size_t count, void *stream);
/* ---- matmuls of the hybrid decode loop ------------------------------------
 * int8 weight-only matmul, fp16 activations, per-output-channel symmetric
 * weight scales: the reference's INT8_WEIGHTS matmul (gdn_e2e_decode.c:
 * quantize_weight:175-199, gemv_int8_neon:296-359), with the weights stored
 * output-major (Wq[N][K], row n = output channel n) so that MFMA operands
 * are contiguous bytes.
 *   y[m][n] = scale[n] * sum_k x[m][k] * Wq[n][k]      (fp32 accumulation)
 * x [M][K] fp16 bit patterns, y [M][N] fp32, 1 <= M <= 16 (the batch),
 * N % 16 == 0, K % 256 == 0, pointers 16-byte aligned.  Narrow layers split
 * k across blocks into `workspace` (at least
 * kai_gdn_w8a16_gemm_workspace_bytes(M, N, K) bytes, 0 = none needed) and
 * reduce it in a fixed order: results are deterministic. */
size_t kai_gdn_w8a16_gemm_workspace_bytes(int M, int N, int K);
int kai_run_gdn_w8a16_gemm_hip(const uint16_t *x, const int8_t *Wq, const float *scale,
                               float *y, int M, int N, int K, void *workspace,
                               size_t workspace_bytes, void *stream);
/* The same GEMM on pre-tiled weights, the form the hybrid loop uses: every
 * wave load is one contiguous 1 KB (lm_head 389 MB at about 6.5 TB/s).
 * kai_run_gdn_w8_tile_hip rearranges row-major Wq [N][K] into Wt (the same
 * N * K bytes); N % 64 == 0, K % 256 == 0.  For 1 <= M <= 16 (decode),
 * narrow matrices split k across blocks and the last block of each
 * 64-channel group sums the splits in a fixed order (deterministic); the
 * workspace holds the partials and one counter per group, must be zeroed
 * once before its first use (each call leaves the counters at zero), and
 * calls that share it must not overlap.  0 workspace bytes: none needed.
 * For M <= 3, N <= 32768 and K of 2560, 4096 or 9216 (the Qwen3.5-4B
 * matrices but the LM head) one 16-channel tile per block runs instead,
 * with no k-split; the workspace is then unused.  M > 16 (a prompt's rows: the counterpart of the reference
 * e2e loop's M > 1 gemm_int8_neon, gdn_e2e_decode.c:606-612) takes the
 * prefill GEMM on fp16 MFMA (128 x 128 output tiles below 512 rows, 256 x
 * 256 from 512), and no workspace. */
int kai_run_gdn_w8_tile_hip(const int8_t *Wq, int8_t *Wt, int N, int K, void *stream);
size_t kai_gdn_w8a16_gemm_tiled_workspace_bytes(int M, int N, int K);
int kai_run_gdn_w8a16_gemm_tiled_hip(const uint16_t *x, const int8_t *Wt, const float *scale,
                                     float *y, int M, int N, int K, void *workspace,
                                     size_t workspace_bytes, void *stream);
/* Quantise W[N][K] fp32 per output channel (row): scale[n] = max|W[n]|/127
 * (1 for an all-zero row), Wq = clamp(round_half_away(W * (1/scale)),
 * -128, 127), as the reference's quantize_weight does per column. */
int kai_run_gdn_w8_quantize_hip(const float *W, int8_t *Wq, float *scale, int N, int K,
                                void *stream);
/* Attention decode of the hybrid loop's full-attention layers (HF
 * Qwen3_5Attention with a KV cache, modeling_qwen3_5.py:629-701, and
 * eager_attention_forward:606-627; the reference's GQA attention,
 * gdn_e2e_decode.c:1532-1634): one new token per sequence,
 *   out[b][h] = softmax_t(scaling * q[b][h] . K[b][kv][t]) . V[b][kv][t],
 *   t < length, kv = h / (num_q_heads / num_kv_heads)
 * q [batch][num_q_heads][256] fp16 (after q_norm and RoPE), k_cache, v_cache
 * [batch][num_kv_heads][max_len][256] fp16, out fp32; softmax and sums in
 * fp32.  num_q_heads / num_kv_heads <= 4.  `workspace` holds at least
 * kai_gdn_attn_decode_workspace_bytes(batch, num_q_heads, length) bytes. */
size_t kai_gdn_attn_decode_workspace_bytes(int batch, int num_q_heads, int length);
int kai_run_gdn_attn_decode_f16kv_hip(const uint16_t *q, const uint16_t *k_cache,
                                      const uint16_t *v_cache, float *out, int batch,
                                      int num_q_heads, int num_kv_heads, int max_len,
                                      int length, float scaling, void *workspace,
                                      size_t workspace_bytes, void *stream);
/* ---- library ------------------------------------------------------------ */

/* Initialise the HIP runtime state of the current device (optional; every
 * entry point does it lazily).  Returns 0 or a hipError_t code. */
int kai_gdn_hip_init(void);

/* Text for a code returned by the functions above. */
const char *kai_gdn_hip_error_string(int code);

/* Non-zero when a scan kernel's bounded wait for a predecessor tile timed
 * out on the current device since the last call (the result of that launch
 * is invalid).  Synchronises the device, then clears the flag. */
int kai_gdn_hip_check_device_error(void);

/* ---- device memory queries -----------------------------------------------
 * No reference counterpart (the reference's kernels allocate nothing on a
 * device).  Bytes of library-owned device workspace that one chunked-prefill
 * call of this shape uses (the segment carry buffer; 0 when the call runs as
 * one segment).  Calls on one device share that buffer, so a model's layers
 * need it once, not once per layer.  Needs no device. */
size_t kai_gdn_hip_prefill_workspace_bytes(int batch, int seq_len, int num_v_heads);
/* Device bytes the library holds on the current device right now (prefill
 * carry buffer, scan status arrays, host-pointer staging buffers); they grow
 * with the largest call seen and are kept until the process ends. */
size_t kai_gdn_hip_device_bytes_held(void);
/* No reference counterpart.  How many (sequence, value head) pairs of the
 * last chunked-prefill call ran as windowed segments (each
 * segment restarted from a zero state a few chunks before its first output,
 * taken where the state map over that window has norm at most 2^-24) rather
 * than by the exact two-pass segment algorithm; 0 when that call ran as one
 * segment.  Counts the last call on the current device.  Synchronises the
 * device.  Returns -1 on a device error. */
int kai_gdn_hip_prefill_windowed_heads(void);

/* ---- measurement probes --------------------------------------------------
 * No reference counterpart: what the current device delivers for a
 * streaming copy or read and for dense bf16 MFMA, so that roofline fractions
 * can be stated against measured ceilings as well as datasheet peaks.  They
 * compute nothing of the GDN path.  `sink` is device memory of
 * kai_gdn_hip_probe_sink_bytes() bytes (written, contents meaningless). */
size_t kai_gdn_hip_probe_sink_bytes(void);
/* mode 0: dst = src over `bytes` (a multiple of 16, 16-byte aligned);
 * mode 1: read src only (dst unused).  Time it with events on `stream`. */
int kai_gdn_hip_probe_stream(const void *src, void *dst, size_t bytes, int mode, void *sink,
                             void *stream);
/* Independent bf16 MFMA chains of `iters` steps on every wave of 16 blocks
 * per CU: shape 0 is 32x32x16 (four chains per wave), 1 is 16x16x32 (eight);
 * *flops receives the launch's multiply-add count x 2. */
int kai_gdn_hip_probe_mfma_bf16(int iters, int shape, void *sink, unsigned long long *flops,
                                void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KAI_GDN_HIP_H */

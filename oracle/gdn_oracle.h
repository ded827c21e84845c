/*
 * gdn_oracle.h -- CPU restatement of the OrionsBelt GDN hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in orionsbelt_amd/.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it.  The product library
 * (libkai_gdn_hip.so) never links, loads or calls anything in oracle/.
 *
 * Every function restates one reference routine in plain scalar C, in the
 * reference's own evaluation order, and cites the file:line it follows
 * (paths relative to the OrionsBelt tree).  Compiled with -ffp-contract=off
 * so that a*b+c is two roundings, as the reference's portable scalar branch
 * is on a target without FMA contraction.
 *
 * Pinning (what checks each function; see tests/):
 *   orc_cumdecay_f32, orc_gated_scan_f32, orc_causal_dwconv1d_f32_k4,
 *   orc_gemv_f32            -- bit-identical to the reference kai sources
 *                              compiled in oracle/_ref, plus closed forms.
 *   orc_delta_rule_matmul_f32 -- bit-identical to the reference's
 *                              gdn_delta_matmul.c (portable branch) compiled
 *                              in oracle/_ref and to its golden vectors;
 *                              within the fp32 error bound of a float64
 *                              product; K = 0 gives zeros.
 *   orc_*_f16 / orc_*_bf16  -- bit-identical to the reference gdn_sve.c
 *                              compiled in oracle/_ref (clang), plus numpy
 *                              float16 / RNE-bfloat16 conversion checks.
 *   orc_causal_dwconv1d_silu_f32_k4 -- conv part as above; SiLU checked
 *                              against torch.nn.functional.silu.
 *   orc_delta_rule_head     -- known answers (k=e_i, beta=0, decay=0) and
 *                              a double-precision brute force.
 *   orc_delta_rule_decode_f32 -- the per-head routine above looped; matched
 *                              against HF torch_recurrent_gated_delta_rule
 *                              golden vectors (tests/golden).
 *   orc_chunk_gdr_f32/_f64  -- HF torch_chunk_gated_delta_rule golden
 *                              vectors, and equality with T stepped decodes.
 *   orc_gating_prologue_f32 -- torch golden vectors of the HF forward's
 *                              gate expressions and HF l2norm; closed forms
 *                              (unit norms, softplus(0) = ln 2, sigmoid(0)
 *                              = 1/2, the softplus threshold).
 *   orc_causal_conv1d_update_f32 -- HF causal_conv1d_update golden vectors
 *                              (tolerance: HF's conv sums in another order)
 *                              and bit-identity with orc_causal_dwconv1d over
 *                              the whole sequence (continuation).
 *   orc_w8_quantize, orc_w8_gemm -- closed forms (the largest weight maps
 *                              to +-127, halves round away from zero, zero
 *                              rows); a float64 numpy restatement.
 *   orc_attn_decode         -- closed forms (one position returns its v; equal
 *                              scores average the values; a dominant score
 *                              selects one value) and a float64 numpy
 *                              restatement of softmax(q K^T) V.
 *   orc_gated_rmsnorm_*     -- golden vectors of HF Qwen3_5RMSNormGated in
 *                              fp32 and bf16; closed forms (constant rows,
 *                              z = 0 gives 0, w scales linearly).
 */
#ifndef ORC_GDN_ORACLE_H
#define ORC_GDN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kai ukernels, portable scalar branch ------------------------------ */

/* decay[t][c] = prod_{i<=t} a[i][c]; running product starts at 1.0f.
 * kleidiai_submission/kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.c:82-90 */
void orc_cumdecay_f32(const float *a, float *decay, size_t seq, size_t channels);

/* acc = x + acc*g per channel, state in/out.
 * kleidiai_submission/kai/ukernels/gdn/kai_gdn_gated_scan_f32_sve.c:86-95 */
void orc_gated_scan_f32(const float *g, const float *x, float *s, float *state,
                        size_t seq, size_t channels);

/* out = h0*w0 + h1*w1 + h2*w2 + cur*w3, hist[3][C] in/out.
 * kleidiai_submission/kai/ukernels/gdn/kai_gdn_causal_dwconv1d_f32_k4_sve.c:149-166 */
void orc_causal_dwconv1d_f32_k4(const float *in, const float *w, float *out,
                                float *hist, size_t seq, size_t channels);

/* Same conv followed by SiLU y = x / (1 + exp(-x)).  The kai kernel has no
 * activation; the SiLU epilogue is HF Qwen3.5 causal_conv1d_fn with
 * activation="silu" (transformers modeling_qwen3_5.py:222-239). */
void orc_causal_dwconv1d_silu_f32_k4(const float *in, const float *w, float *out,
                                     float *hist, size_t seq, size_t channels);

/* c[j] = sum_k a[k]*b[k][j], k-loop inner, acc from 0.0f.
 * kleidiai_submission/kai/ukernels/gdn/kai_gdn_gemv_f32_f32_f32_1x4_neon.c:78-86 */
void orc_gemv_f32(const float *a, const float *b, float *c, size_t k, size_t n);

/* C[i][j] = sum_k A[i][k]*B[k][j], k-loop inner, acc from 0.0f.
 * src/orionsbelt/engines/cpu/kernels/gdn_delta_matmul.c:111-118 */
void orc_delta_rule_matmul_f32(const float *A, const float *B, float *C, size_t m, size_t k, size_t n);

/* ---- mixed precision (gdn_sve.c scalar branches) ------------------------ */
/* fp16 values are passed as IEEE binary16 bit patterns (uint16_t), bf16 as the
 * upper half of a binary32 (uint16_t).  Conversions are round-to-nearest-even. */

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
/* src/orionsbelt/engines/cpu/kernels/gdn_sve.c:81-87 */
uint16_t orc_f32_to_bf16(float f);
/* src/orionsbelt/engines/cpu/kernels/gdn_sve.c:89-94 */
float orc_bf16_to_f32(uint16_t b);

/* gdn_sve.c:589-600 */
void orc_cumdecay_f16(const float *a, uint16_t *decay, size_t seq, size_t channels);
/* gdn_sve.c:511-523 */
void orc_gated_scan_f16(const float *g, const float *x, float *s, uint16_t *state,
                        size_t seq, size_t channels);
/* gdn_sve.c:754-765 */
void orc_cumdecay_bf16(const float *a, uint16_t *decay, size_t seq, size_t channels);
/* gdn_sve.c:682-694 */
void orc_gated_scan_bf16(const float *g, const float *x, float *s, uint16_t *state,
                         size_t seq, size_t channels);
/* GDN-2 decoupled-gating scan, the portable branch gdn_sve.c:861-874:
 *   acc = w[t][c] * x[t][c] + acc * (g[t][c] * b[t][c])  (no contraction)
 * Pinned bit-exact against the reference build (oracle/_ref) and by its
 * reduction to gated_scan_f32 when b = w = 1. */
void orc_gdn2_gated_scan_f32(const float *g, const float *b, const float *w, const float *x, float *s,
                             float *state, size_t seq, size_t channels);

/* ---- matrix-state delta rule ------------------------------------------- */

/* One head, one token, in the reference order:
 *   S *= decay; for each column i: kv = sum_j S[j][i]*k[j];
 *   delta = (v[i]-kv)*beta; S[:,i] += k*delta; out[i] = sum_j S[j][i]*q[j].
 * S is [hkd][hvd] row-major.  gpu/gdn_gpu_validate.c:100-118 */
void orc_delta_rule_head(float *S, const float *k, const float *v, const float *q,
                         float beta, float decay, float *out, size_t hkd, size_t hvd);

/* Batched single-token decode with per-(sequence, value-head) gates:
 *   S  [B][Hv][dk][dv] fp32, in/out
 *   q,k [B][Hk][dk], v [B][Hv][dv], g,beta [B][Hv], o [B][Hv][dv]
 * Value head h reads key head h / (Hv/Hk) (HF repeat_interleave,
 * modeling_qwen3_5.py:500-502).  decay = expf(g) (HF :366), q is scaled by
 * q_scale before the read-out (HF :356-357; 1 reproduces the reference's
 * unscaled ref_delta_rule).  Per head this is orc_delta_rule_head. */
void orc_delta_rule_decode_f32(float *S, const float *q, const float *k,
                               const float *v, const float *g, const float *beta,
                               float *o, int B, int Hv, int Hk, int dk, int dv,
                               float q_scale);

/* Same step with the state stored as fp16 bit patterns: widen on load, fp32
 * arithmetic, narrow (RNE) on store -- the narrow-storage / wide-compute rule
 * of gdn_sve.c:433-441 applied to the matrix state. */
void orc_delta_rule_decode_f16state(uint16_t *S, const float *q, const float *k,
                                    const float *v, const float *g,
                                    const float *beta, float *o, int B, int Hv,
                                    int Hk, int dk, int dv, float q_scale);

/* ---- chunkwise (WY) gated delta rule, HF torch_chunk_gated_delta_rule ----
 * transformers/models/qwen3_5/modeling_qwen3_5.py:248-328 restated per
 * (batch, value head).  Layouts (token-major, as HF's [B, T, H, D]):
 *   q,k [B][T][Hk][dk]  v [B][T][Hv][dv]  g,beta [B][T][Hv]
 *   o [B][T][Hv][dv]    S [B][Hv][dk][dv] (initial state in, final out)
 * q/k are used as given (no L2 norm inside; HF applies it in the caller with
 * use_qk_l2norm_in_kernel); q is multiplied by q_scale (HF :278-279).
 * T need not be a multiple of `chunk`; the tail chunk is zero-padded (HF
 * :270-276).  _f32 computes in float, _f64 in double (inputs and outputs
 * are float in both). */
void orc_chunk_gdr_f32(const float *q, const float *k, const float *v,
                       const float *g, const float *beta, float *o, float *S,
                       int B, int T, int Hv, int Hk, int dk, int dv, int chunk,
                       float q_scale);
void orc_chunk_gdr_f64(const float *q, const float *k, const float *v,
                       const float *g, const float *beta, float *o, float *S,
                       int B, int T, int Hv, int Hk, int dk, int dv, int chunk,
                       float q_scale);

/* Gating prologue of one GDN layer: HF transformers
 * modeling_qwen3_5.py Qwen3_5GatedDeltaNet.forward:497-499 (gates) and
 * l2norm:242-245 (q, k norm with eps 1e-6, use_qk_l2norm_in_kernel,
 * :262-264).  x [rows][(2 Hk + Hv) * 128] holds the conv output of each
 * token, q heads then k heads then v heads (the torch.split / reshape of
 * :481-492); a, b [rows][Hv]; A_log, dt_bias [Hv].  Outputs:
 *   q, k [rows][Hk][128] = x_head / sqrt(sum x_head^2 + 1e-6)
 *   v [rows][Hv][128]    = x_head
 *   g [rows][Hv]    = -exp(A_log) * softplus(a + dt_bias),
 *                     softplus(y) = y > 20 ? y : log1p(exp(y)) (torch's)
 *   beta [rows][Hv] = 1 / (1 + exp(-b))
 * The sum of squares is accumulated in double and rounded once. */
void orc_gating_prologue_f32(const float *x, const float *a, const float *b,
                             const float *A_log, const float *dt_bias, float *q,
                             float *k, float *v, float *g, float *beta, size_t rows,
                             int Hk, int Hv);

/* Gated RMSNorm with the SiLU gate (HF Qwen3_5RMSNormGated.forward,
 * modeling_qwen3_5.py:175-184) over rows of n values:
 *   fp32 model: y = (w * (o / sqrt(mean(o^2) + eps))) * silu(z)
 *   bf16 model: h = bf16(o / sqrt(mean(o^2) + eps)), h = bf16(w * h),
 *               y = bf16(h * silu(z))   (o, z, w, y bf16 bit patterns)
 * with silu(z) = z / (1 + exp(-z)) in fp32 and mean(o^2) in fp32 from a
 * double sum. */
void orc_gated_rmsnorm_f32(const float *o, const float *z, const float *w, float *y,
                           size_t rows, int n, float eps);
void orc_gated_rmsnorm_bf16(const uint16_t *o, const uint16_t *z, const uint16_t *w,
                            uint16_t *y, size_t rows, int n, float eps);

/* HF causal_conv1d_update (modeling_qwen3_5.py:199-217) for B sequences
 * of T new tokens: x, out [B][T][C], conv_state [B][C][4] (in/out; the last
 * four inputs, newest last), w [C][4].  Per token, with the window
 * (s1, s2, s3, x) of the state and the new input:
 *   out = ((s1*w0 + s2*w1) + s3*w2) + x*w3   (the kai reference's order,
 *         kai_gdn_causal_dwconv1d_f32_k4_sve.c:149-166), SiLU if silu,
 *   state <- (s1, s2, s3, x). */
void orc_causal_conv1d_update_f32(const float *x, float *conv_state, const float *w,
                                  float *out, int B, int T, size_t C, int silu);

/* int8 weight-only matmul of the hybrid decode loop (the reference's
 * INT8_WEIGHTS path, gdn_e2e_decode.c).  orc_w8_quantize restates
 * quantize_weight (:175-199) on the rows of W[N][K] (the reference quantises
 * the columns of its [K][N] layout): scale = max|w| / 127 (1 for a zero
 * row), q = clamp(lroundf(w * (1 / scale)), -128, 127).  orc_w8_gemm:
 * y[m][n] = scale[n] * sum_k x[m][k] q[n][k] with x fp16 bit patterns, the
 * sum in double, rounded to fp32 once, then scaled (gemv_int8_neon
 * (:296-359) sums in fp32 and scales per column). */
void orc_w8_quantize(const float *W, int8_t *Wq, float *scale, int N, int K);
void orc_w8_gemm(const uint16_t *x, const int8_t *Wq, const float *scale, float *y, int M,
                 int N, int K);

/* Attention decode over an fp16 KV cache (HF eager_attention_forward with
 * repeat_kv, modeling_qwen3_5.py:606-627): q [B][Hq][D], k, v
 * [B][Hkv][Tmax][D] fp16 bits, out [B][Hq][D] fp32; softmax and sums in
 * double. */
void orc_attn_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *out, int B,
                     int Hq, int Hkv, int Tmax, int L, int D, float scaling);

/* ---- hybrid decode loop (gdn_hybrid_oracle.c) ---------------------------
 * The CPU model of include/kai_gdn_hybrid.h: same configuration fields in
 * the same order, same drawn weights and states, same step (see the file
 * header for the layer definitions and how it is pinned). */
typedef struct {
    int layers, attn_every, hidden, inter, vocab, gdn_k_heads, gdn_v_heads, attn_q_heads,
        attn_kv_heads, max_batch, max_context;
    float rope_theta, rms_eps;
} orc_hybrid_config;
typedef struct orc_hybrid orc_hybrid;
orc_hybrid *orc_hybrid_create(const orc_hybrid_config *cfg, uint64_t seed);
void orc_hybrid_reset(orc_hybrid *m, int batch, int context, uint64_t seed);
void orc_hybrid_step(orc_hybrid *m, const int32_t *tokens, int32_t *next, float *logits);
int orc_hybrid_position(const orc_hybrid *m);
/* With on != 0, each GDN layer rounds the recurrence's q, k, v (after the
 * gating prologue) and its output o (before the gated RMSNorm) to bf16 by
 * round-to-nearest-even: the formats the device prefill hands between its
 * kernels (bf16 gating prologue, bf16 chunked delta rule), so that a device
 * prefill compares with this model up to the kernels' own arithmetic. */
void orc_hybrid_set_gdn_bf16_io(orc_hybrid *m, int on);
long orc_hybrid_tensor(const orc_hybrid *m, int layer, int id, float *dst);
void orc_hybrid_destroy(orc_hybrid *m);

/* Number of OpenMP threads the oracle uses (1 when built without OpenMP),
 * and a way to set it (the CPU baseline's single-thread run). */
int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif /* ORC_GDN_ORACLE_H */

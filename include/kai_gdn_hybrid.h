/*
 * kai_gdn_hybrid.h -- the end-to-end hybrid decode loop of libkai_gdn_hip.so
 * (gfx950): a random-init, Qwen3.5-shaped model of Gated DeltaNet and full
 * attention layers with int8 per-output-channel weights and fp16
 * activations, decoded one token per sequence per step.
 *
 * No reference kai symbol: the reference's loop is the C program
 * src/orionsbelt/engines/cpu/kernels/gdn_e2e_decode.c (:1921-2865), which
 * uses a simplified GDN and produces no logits.  The layer definitions
 * followed here are HF transformers modeling_qwen3_5.py
 * (Qwen3_5DecoderLayer:740-794: pre-norm, mixer, residual, post-norm,
 * SwiGLU MLP, residual; Qwen3_5GatedDeltaNet:387-543; Qwen3_5Attention:
 * 629-701 with q/k norm, partial rotary embedding and the sigmoid output
 * gate; Qwen3_5RMSNorm:720-737, whose weight enters as 1 + w), with the
 * residual stream kept in fp32 and every matmul input rounded to fp16.
 *
 * Weights, norms and gate parameters are drawn from a counter-based hash of
 * (seed, tensor, index), so a CPU restatement draws the same model; matmul
 * weights are quantised per output channel as the reference's
 * quantize_weight does.  A context of `context` tokens is represented by
 * states drawn the same way (KV caches, recurrent and conv states), which
 * is what a prefill of that length leaves behind for the decode steps to
 * read; a context of 0 starts empty, and tokens fed through
 * kai_gdn_hybrid_step build the context for real.
 *
 * All functions return 0 or a hipError_t code (kai_gdn_hip_error_string).
 */
#ifndef KAI_GDN_HYBRID_H
#define KAI_GDN_HYBRID_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef struct kai_gdn_hybrid kai_gdn_hybrid;

typedef struct {
    int layers;      /* 32 */
    int attn_every;  /* 4: layer i is full attention iff (i + 1) % attn_every == 0 */
    int hidden;      /* 2560 (% 256 == 0, <= 8192) */
    int inter;       /* 9216 (% 256 == 0) */
    int vocab;       /* 151936 (% 16 == 0) */
    int gdn_k_heads; /* 16; key and value head dims are 128 */
    int gdn_v_heads; /* 32 (% 16 == 0, a multiple of gdn_k_heads) */
    int attn_q_heads;  /* 16; head dim 256 */
    int attn_kv_heads; /* 4 (q_heads / kv_heads <= 4) */
    int max_batch;   /* <= 16 */
    int max_context; /* KV cache length (<= 2^24) */
    float rope_theta; /* 1e7 */
    float rms_eps;    /* 1e-6 */
} kai_gdn_hybrid_config;

/* The Qwen3.5-4B shape of the benchmark, with the given
 * batch and context limits. */
kai_gdn_hybrid_config kai_gdn_hybrid_qwen35_4b(int max_batch, int max_context);

/* Allocate the model on the current device and draw its weights. */
int kai_gdn_hybrid_create(const kai_gdn_hybrid_config *cfg, unsigned long long seed,
                          kai_gdn_hybrid **out);
/* Start `batch` sequences at position `context`, with drawn states for the
 * context (0: empty states).  batch <= max_batch, context < max_context. */
int kai_gdn_hybrid_reset(kai_gdn_hybrid *m, int batch, int context, unsigned long long seed);
/* One decode step on `stream`: tokens [batch] int32 (device) in, the next
 * tokens by greedy argmax (device, may be NULL) and the logits [batch][vocab]
 * fp32 (device, may be NULL) out.  The position advances by one.  A pointer
 * that is not device (or managed) memory is refused (hipErrorInvalidValue)
 * before anything is launched; so is a step when the KV cache is full. */
int kai_gdn_hybrid_step(kai_gdn_hybrid *m, const int32_t *tokens, int32_t *next, float *logits,
                        void *stream);
/* Prefill: start `batch` sequences from empty states and run the `length`
 * prompt tokens of each (tokens [batch][length] int32, device) through
 * every layer at once -- all positions of a sequence per launch: int8 GEMMs
 * on MFMA for the projections, the conv and gating glue, the chunked delta
 * rule (kai_run_gdn_chunk_delta_rule_bf16_f32_hip) and causal attention that
 * writes the KV cache -- leaving the recurrent states, conv caches and KV
 * caches where kai_gdn_hybrid_step reads them, at position `length`.  The
 * next tokens (greedy) and logits of each sequence's last position are
 * written as by kai_gdn_hybrid_step.  batch <= max_batch, 1 <= length <
 * max_context.  The first call allocates the prefill's activation buffers
 * for max_context positions (freed by kai_gdn_hybrid_destroy).  The
 * reference e2e program's --prefill mode runs its prompt the same way
 * (gdn_e2e_decode.c:2644-2700, with the M > 1 GEMM of :606-612). */
int kai_gdn_hybrid_prefill(kai_gdn_hybrid *m, const int32_t *tokens, int batch, int length,
                           int32_t *next, float *logits, void *stream);
/* Per-layer-type timing, the GPU counterpart of the e2e program's phase
 * timers (gdn_e2e_decode.c:1365-1371, reported at :2708-2710,2820-2857).
 * With timing on, kai_gdn_hybrid_step and kai_gdn_hybrid_prefill record a
 * HIP event on their stream at every phase boundary (about 130 per step,
 * which adds their own cost to the call); kai_gdn_hybrid_phase_times waits
 * for the last one, adds each interval to its phase and writes the sums in
 * microseconds since the previous read (or since timing was switched on)
 * to us[0 .. n-1] in KAI_GDN_PHASE_* order, then starts new sums.  Phases:
 * the GDN layers' input projection (in_proj_qkvz|b|a), their conv update,
 * gating, delta rule and gated RMSNorm (one fused kernel in a decode step;
 * conv, gating prologue, chunked delta rule and norm in a prefill), their
 * out_proj with the residual add; the attention layers whole; the MLPs
 * (with the norm that feeds them in a prefill); and the rest (embedding,
 * first norm, LM head, argmax).  Returns 0, or hipErrorInvalidValue. */
enum {
    KAI_GDN_PHASE_GDN_PROJ = 0,
    KAI_GDN_PHASE_GDN_CORE = 1,
    KAI_GDN_PHASE_GDN_OPROJ = 2,
    KAI_GDN_PHASE_ATTN = 3,
    KAI_GDN_PHASE_FFN = 4,
    KAI_GDN_PHASE_OTHER = 5,
    KAI_GDN_PHASE_COUNT = 6
};
int kai_gdn_hybrid_set_timing(kai_gdn_hybrid *m, int on);
int kai_gdn_hybrid_phase_times(kai_gdn_hybrid *m, double *us, int n);
/* Current position (context + steps taken) and device bytes held. */
int kai_gdn_hybrid_position(const kai_gdn_hybrid *m);
size_t kai_gdn_hybrid_device_bytes(const kai_gdn_hybrid *m);
/* Weight bytes a step reads (int8 matrices + scales), for bandwidth figures. */
size_t kai_gdn_hybrid_weight_bytes(const kai_gdn_hybrid *m);
void kai_gdn_hybrid_destroy(kai_gdn_hybrid *m);

#ifdef __cplusplus
}
#endif
#endif /* KAI_GDN_HYBRID_H */

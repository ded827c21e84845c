/*
 * gdn_hybrid_oracle.c -- CPU restatement of the hybrid decode loop of
 * libkai_gdn_hip.so (include/kai_gdn_hybrid.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP model, never linked into
 * the product.  It draws the same model from the same counter-based hash and
 * steps it with the scalar restatements of gdn_oracle.c (w8 quantise and
 * matmul, conv update, gating prologue, delta-rule decode, gated RMSNorm,
 * attention decode), in plain loops, with double accumulation where the
 * device sums.
 *
 * The layer definitions follow HF transformers modeling_qwen3_5.py
 * (Qwen3_5DecoderLayer:740-794, Qwen3_5GatedDeltaNet:387-543,
 * Qwen3_5Attention:629-701, Qwen3_5MLP:704-717, Qwen3_5RMSNorm:720-737,
 * Qwen3_5TextRotaryEmbedding:84-160 with apply_rotary_pos_emb) with every
 * matmul input rounded to fp16, the fp16 KV cache, and int8 per-output-
 * channel weights (the reference quantize_weight, gdn_e2e_decode.c:175-199).
 * Pinning: tests/test_oracle.py compares the logits of teacher-forced steps
 * with those of HF Qwen3_5ForCausalLM run in fp32 on the dequantised weights
 * (tests/golden/hf_hybrid.npz), over the whole token sequence at once.
 */
#include "gdn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- drawn values (the device's hash, bit for bit) ------------------------ */

static uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static float hash_value(uint64_t seed, uint64_t stream, uint64_t i, float amp, float center) {
    const uint64_t h = mix64(mix64(seed ^ (stream * 0x100000001B3ull)) + i);
    const float u = (float)(h >> 40) * (1.0f / 16777216.0f);
    return (u * 2.0f - 1.0f) * amp + center;
}
/* Element i is a function of (seed, stream, i) alone, so the loops below may
 * run in any order or in parallel and draw the same values. */
static void draw(float *dst, size_t n, uint64_t seed, uint64_t stream, float amp, float center) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) dst[i] = hash_value(seed, stream, i, amp, center);
}

enum {
    T_LN_IN = 0, T_LN_POST, T_QKV, T_Z, T_BP, T_AP, T_OUT, T_CONVW, T_DTBIAS, T_ALOG, T_NORMW,
    T_QP, T_KP, T_VP, T_OP, T_QN, T_KN, T_GATE, T_UP, T_DOWN
};
enum { G_EMBED = 1, G_FINAL_NORM = 2, G_LM_HEAD = 3 };
enum { S_CONV = 0, S_S = 1, S_K = 2, S_V = 3 };
#define W_AMP 0.034641016f

typedef struct {
    int8_t *q;
    float *s;
    int N, K;
} mat;

typedef struct {
    int attn;
    float *ln_in, *ln_post;
    mat qkv, z, bp, ap, out, qp, kp, vp, op, gate, up, down;
    float *conv_w, *dt_bias, *A_log, *norm_w, *q_norm, *k_norm;
    float *S, *conv_state;
    uint16_t *Kc, *Vc;
} layer;

struct orc_hybrid {
    orc_hybrid_config c;
    int conv_dim, value_dim;
    layer *L;
    uint16_t *embed;
    float *final_norm;
    mat lm;
    int batch, pos;
    int gdn_bf16_io;  /* orc_hybrid_set_gdn_bf16_io */
};

static void make_mat(mat *w, int N, int K, uint64_t seed, uint64_t stream) {
    float *tmp = malloc(sizeof(float) * (size_t)N * K);
    draw(tmp, (size_t)N * K, seed, stream, W_AMP, 0.f);
    w->N = N;
    w->K = K;
    w->q = malloc((size_t)N * K);
    w->s = malloc(sizeof(float) * N);
    orc_w8_quantize(tmp, w->q, w->s, N, K);
    free(tmp);
}
static float *make_vec(size_t n, uint64_t seed, uint64_t stream, float amp, float center) {
    float *v = malloc(sizeof(float) * n);
    draw(v, n, seed, stream, amp, center);
    return v;
}
static void free_mat(mat *w) {
    free(w->q);
    free(w->s);
}

orc_hybrid *orc_hybrid_create(const orc_hybrid_config *cfg, uint64_t seed) {
    orc_hybrid *m = calloc(1, sizeof(*m));
    m->c = *cfg;
    const orc_hybrid_config *c = &m->c;
    const int H = c->hidden, I = c->inter, Hv = c->gdn_v_heads, Hk = c->gdn_k_heads, Hq = c->attn_q_heads,
              Hkv = c->attn_kv_heads, Bm = c->max_batch;
    m->conv_dim = 2 * Hk * 128 + Hv * 128;
    m->value_dim = Hv * 128;
    m->L = calloc(c->layers, sizeof(layer));
    for (int l = 0; l < c->layers; ++l) {
        layer *L = &m->L[l];
        const uint64_t base = 64ull * (l + 1);
        L->attn = (l + 1) % c->attn_every == 0;
        L->ln_in = make_vec(H, seed, base + T_LN_IN, 0.1f, 0.f);
        L->ln_post = make_vec(H, seed, base + T_LN_POST, 0.1f, 0.f);
        if (!L->attn) {
            make_mat(&L->qkv, m->conv_dim, H, seed, base + T_QKV);
            make_mat(&L->z, m->value_dim, H, seed, base + T_Z);
            make_mat(&L->bp, Hv, H, seed, base + T_BP);
            make_mat(&L->ap, Hv, H, seed, base + T_AP);
            make_mat(&L->out, H, m->value_dim, seed, base + T_OUT);
            L->conv_w = make_vec((size_t)m->conv_dim * 4, seed, base + T_CONVW, 0.5f, 0.f);
            L->dt_bias = make_vec(Hv, seed, base + T_DTBIAS, 0.5f, 1.0f);
            L->A_log = make_vec(Hv, seed, base + T_ALOG, 1.3862944f, 1.3862944f);
            L->norm_w = make_vec(128, seed, base + T_NORMW, 0.1f, 1.0f);
            L->S = calloc((size_t)Bm * Hv * 128 * 128, sizeof(float));
            L->conv_state = calloc((size_t)Bm * m->conv_dim * 4, sizeof(float));
        } else {
            make_mat(&L->qp, Hq * 512, H, seed, base + T_QP);
            make_mat(&L->kp, Hkv * 256, H, seed, base + T_KP);
            make_mat(&L->vp, Hkv * 256, H, seed, base + T_VP);
            make_mat(&L->op, H, Hq * 256, seed, base + T_OP);
            L->q_norm = make_vec(256, seed, base + T_QN, 0.1f, 0.f);
            L->k_norm = make_vec(256, seed, base + T_KN, 0.1f, 0.f);
            L->Kc = calloc((size_t)Bm * Hkv * c->max_context * 256, 2);
            L->Vc = calloc((size_t)Bm * Hkv * c->max_context * 256, 2);
        }
        make_mat(&L->gate, I, H, seed, base + T_GATE);
        make_mat(&L->up, I, H, seed, base + T_UP);
        make_mat(&L->down, H, I, seed, base + T_DOWN);
    }
    const size_t ne = (size_t)c->vocab * H;
    m->embed = malloc(2 * ne);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < ne; ++i) m->embed[i] = orc_f32_to_f16(hash_value(seed, G_EMBED, i, 1.0f, 0.f));
    m->final_norm = make_vec(H, seed, G_FINAL_NORM, 0.1f, 0.f);
    make_mat(&m->lm, c->vocab, H, seed, G_LM_HEAD);
    m->batch = Bm;
    return m;
}

void orc_hybrid_destroy(orc_hybrid *m) {
    if (!m) return;
    for (int l = 0; l < m->c.layers; ++l) {
        layer *L = &m->L[l];
        free(L->ln_in);
        free(L->ln_post);
        if (!L->attn) {
            free_mat(&L->qkv); free_mat(&L->z); free_mat(&L->bp); free_mat(&L->ap); free_mat(&L->out);
            free(L->conv_w); free(L->dt_bias); free(L->A_log); free(L->norm_w);
            free(L->S); free(L->conv_state);
        } else {
            free_mat(&L->qp); free_mat(&L->kp); free_mat(&L->vp); free_mat(&L->op);
            free(L->q_norm); free(L->k_norm); free(L->Kc); free(L->Vc);
        }
        free_mat(&L->gate); free_mat(&L->up); free_mat(&L->down);
    }
    free(m->L);
    free(m->embed);
    free(m->final_norm);
    free_mat(&m->lm);
    free(m);
}

void orc_hybrid_reset(orc_hybrid *m, int batch, int context, uint64_t seed) {
    const orc_hybrid_config *c = &m->c;
    m->batch = batch;
    m->pos = context;
    for (int l = 0; l < c->layers; ++l) {
        layer *L = &m->L[l];
        const uint64_t base = (1ull << 20) + 16ull * l;
        if (!L->attn) {
            const size_t ns = (size_t)batch * c->gdn_v_heads * 128 * 128, nc = (size_t)batch * m->conv_dim * 4;
            if (context > 0) {
                draw(L->S, ns, seed, base + S_S, 0.034641016f, 0.f);
                draw(L->conv_state, nc, seed, base + S_CONV, 1.0f, 0.f);
            } else {
                memset(L->S, 0, ns * 4);
                memset(L->conv_state, 0, nc * 4);
            }
        } else {
            const size_t n = (size_t)batch * c->attn_kv_heads * c->max_context * 256;
#pragma omp parallel for schedule(static)
            for (size_t i = 0; i < n; ++i) {
                const int t = (int)((i / 256) % c->max_context);
                L->Kc[i] = t < context ? orc_f32_to_f16(hash_value(seed, base + S_K, i, 1.0f, 0.f)) : 0;
                L->Vc[i] = t < context ? orc_f32_to_f16(hash_value(seed, base + S_V, i, 1.0f, 0.f)) : 0;
            }
        }
    }
}

/* Qwen3_5RMSNorm with the residual add: h += d, x16 = fp16(h * rsqrt(mean(h^2) + eps) * (1 + w)). */
static void addnorm(float *h, const float *d, const float *w, uint16_t *x16, int B, int H, float eps) {
    for (int b = 0; b < B; ++b) {
        float *hr = h + (size_t)b * H;
        double ss = 0.0;
        for (int i = 0; i < H; ++i) {
            if (d) hr[i] += d[(size_t)b * H + i];
            ss += (double)hr[i] * hr[i];
        }
        const float inv = 1.0f / sqrtf((float)(ss / H) + eps);
        for (int i = 0; i < H; ++i) x16[(size_t)b * H + i] = orc_f32_to_f16(hr[i] * inv * (1.0f + w[i]));
    }
}

static void gemm(const uint16_t *x, const mat *w, float *y, int B) { orc_w8_gemm(x, w->q, w->s, y, B, w->N, w->K); }

static void gdn_mixer(orc_hybrid *m, layer *L, const uint16_t *x16, float *out) {
    const orc_hybrid_config *c = &m->c;
    const int B = m->batch, Hk = c->gdn_k_heads, Hv = c->gdn_v_heads, C = m->conv_dim, V = m->value_dim;
    float *qkv = malloc(sizeof(float) * B * C), *cv = malloc(sizeof(float) * B * C);
    float *z = malloc(sizeof(float) * B * V), *a = malloc(sizeof(float) * B * Hv), *bb = malloc(sizeof(float) * B * Hv);
    float *q = malloc(sizeof(float) * B * Hk * 128), *k = malloc(sizeof(float) * B * Hk * 128);
    float *v = malloc(sizeof(float) * B * V), *g = malloc(sizeof(float) * B * Hv), *beta = malloc(sizeof(float) * B * Hv);
    float *o = malloc(sizeof(float) * B * V), *y = malloc(sizeof(float) * B * V);
    uint16_t *y16 = malloc(2 * (size_t)B * V);
    gemm(x16, &L->qkv, qkv, B);
    gemm(x16, &L->z, z, B);
    gemm(x16, &L->bp, bb, B);
    gemm(x16, &L->ap, a, B);
    orc_causal_conv1d_update_f32(qkv, L->conv_state, L->conv_w, cv, B, 1, (size_t)C, 1);
    orc_gating_prologue_f32(cv, a, bb, L->A_log, L->dt_bias, q, k, v, g, beta, (size_t)B, Hk, Hv);
    if (m->gdn_bf16_io) {  /* the recurrence's operands in the device prefill's format */
        for (size_t i = 0; i < (size_t)B * Hk * 128; ++i) {
            q[i] = orc_bf16_to_f32(orc_f32_to_bf16(q[i]));
            k[i] = orc_bf16_to_f32(orc_f32_to_bf16(k[i]));
        }
        for (size_t i = 0; i < (size_t)B * V; ++i) v[i] = orc_bf16_to_f32(orc_f32_to_bf16(v[i]));
    }
    orc_delta_rule_decode_f32(L->S, q, k, v, g, beta, o, B, Hv, Hk, 128, 128, 1.0f / sqrtf(128.0f));
    if (m->gdn_bf16_io)
        for (size_t i = 0; i < (size_t)B * V; ++i) o[i] = orc_bf16_to_f32(orc_f32_to_bf16(o[i]));
    orc_gated_rmsnorm_f32(o, z, L->norm_w, y, (size_t)B * Hv, 128, c->rms_eps);
    for (size_t i = 0; i < (size_t)B * V; ++i) y16[i] = orc_f32_to_f16(y[i]);
    gemm(y16, &L->out, out, B);
    free(qkv); free(cv); free(z); free(a); free(bb); free(q); free(k); free(v); free(g); free(beta);
    free(o); free(y); free(y16);
}

/* q/k RMSNorm over one 256-dim head, rounded to fp16, then the rotary
 * embedding on dims 0..63 (rotate_half), rounded to fp16. */
static void norm_rope(const float *x, const float *w, float theta, float eps, int pos, uint16_t *dst) {
    double ss = 0.0;
    for (int d = 0; d < 256; ++d) ss += (double)x[d] * x[d];
    const float inv = 1.0f / sqrtf((float)(ss / 256) + eps);
    float xn[256];
    for (int d = 0; d < 256; ++d) xn[d] = orc_f16_to_f32(orc_f32_to_f16(x[d] * inv * (1.0f + w[d])));
    for (int d = 0; d < 256; ++d) {
        float y = xn[d];
        if (d < 64) {
            const int i = d & 31;
            const float inv_freq = 1.0f / powf(theta, (float)(2 * i) / 64.0f);
            const float f = inv_freq * (float)pos;
            const float cs = cosf(f), sn = sinf(f);
            y = d < 32 ? xn[d] * cs - xn[d + 32] * sn : xn[d] * cs + xn[d - 32] * sn;
        }
        dst[d] = orc_f32_to_f16(y);
    }
}

static void attn_mixer(orc_hybrid *m, layer *L, const uint16_t *x16, float *out) {
    const orc_hybrid_config *c = &m->c;
    const int B = m->batch, Hq = c->attn_q_heads, Hkv = c->attn_kv_heads, T = c->max_context, pos = m->pos;
    float *qg = malloc(sizeof(float) * B * Hq * 512), *kx = malloc(sizeof(float) * B * Hkv * 256);
    float *vx = malloc(sizeof(float) * B * Hkv * 256), *ao = malloc(sizeof(float) * B * Hq * 256);
    uint16_t *q16 = malloc(2 * (size_t)B * Hq * 256), *o16 = malloc(2 * (size_t)B * Hq * 256);
    gemm(x16, &L->qp, qg, B);
    gemm(x16, &L->kp, kx, B);
    gemm(x16, &L->vp, vx, B);
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hq; ++h)
            norm_rope(qg + ((size_t)b * Hq + h) * 512, L->q_norm, c->rope_theta, c->rms_eps, pos,
                      q16 + ((size_t)b * Hq + h) * 256);
        for (int h = 0; h < Hkv; ++h) {
            const size_t row = (((size_t)b * Hkv + h) * T + pos) * 256;
            norm_rope(kx + ((size_t)b * Hkv + h) * 256, L->k_norm, c->rope_theta, c->rms_eps, pos, L->Kc + row);
            for (int d = 0; d < 256; ++d) L->Vc[row + d] = orc_f32_to_f16(vx[((size_t)b * Hkv + h) * 256 + d]);
        }
    }
    orc_attn_decode(q16, L->Kc, L->Vc, ao, B, Hq, Hkv, T, pos + 1, 256, 1.0f / 16.0f);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h)
            for (int d = 0; d < 256; ++d) {
                const size_t bh = (size_t)b * Hq + h;
                const float gt = qg[bh * 512 + 256 + d];
                o16[bh * 256 + d] = orc_f32_to_f16(ao[bh * 256 + d] * (1.0f / (1.0f + expf(-gt))));
            }
    gemm(o16, &L->op, out, B);
    free(qg); free(kx); free(vx); free(ao); free(q16); free(o16);
}

void orc_hybrid_step(orc_hybrid *m, const int32_t *tokens, int32_t *next, float *logits) {
    const orc_hybrid_config *c = &m->c;
    const int B = m->batch, H = c->hidden, I = c->inter;
    const int wide = m->conv_dim > I ? (m->conv_dim > m->value_dim ? m->conv_dim : m->value_dim) : I;
    float *h = malloc(sizeof(float) * B * H), *mix = malloc(sizeof(float) * B * H);
    float *mlp = malloc(sizeof(float) * B * H), *gt = malloc(sizeof(float) * B * I), *up = malloc(sizeof(float) * B * I);
    uint16_t *x16 = malloc(2 * (size_t)B * (wide > H ? wide : H));
    for (int b = 0; b < B; ++b) {
        int t = tokens[b];
        t = t < 0 ? 0 : t >= c->vocab ? c->vocab - 1 : t;
        for (int i = 0; i < H; ++i) h[(size_t)b * H + i] = orc_f16_to_f32(m->embed[(size_t)t * H + i]);
    }
    const float *pending = NULL;
    for (int l = 0; l < c->layers; ++l) {
        layer *L = &m->L[l];
        addnorm(h, pending, L->ln_in, x16, B, H, c->rms_eps);
        if (L->attn) attn_mixer(m, L, x16, mix);
        else gdn_mixer(m, L, x16, mix);
        addnorm(h, mix, L->ln_post, x16, B, H, c->rms_eps);
        gemm(x16, &L->gate, gt, B);
        gemm(x16, &L->up, up, B);
        for (size_t i = 0; i < (size_t)B * I; ++i) {
            const float g = gt[i];
            x16[i] = orc_f32_to_f16(g / (1.0f + expf(-g)) * up[i]);
        }
        gemm(x16, &L->down, mlp, B);
        pending = mlp;
    }
    addnorm(h, pending, m->final_norm, x16, B, H, c->rms_eps);
    gemm(x16, &m->lm, logits, B);
    for (int b = 0; b < B; ++b) {
        const float *row = logits + (size_t)b * c->vocab;
        int best = 0;
        for (int i = 1; i < c->vocab; ++i)
            if (row[i] > row[best]) best = i;
        if (next) next[b] = best;
    }
    ++m->pos;
    free(h); free(mix); free(mlp); free(gt); free(up); free(x16);
}

int orc_hybrid_position(const orc_hybrid *m) { return m->pos; }

void orc_hybrid_set_gdn_bf16_io(orc_hybrid *m, int on) { m->gdn_bf16_io = on != 0; }

/* Export one drawn tensor as fp32 (matrices dequantised: q * scale, [N][K]).
 * layer < 0 selects the model-level tensors (G_*).  Returns the element
 * count (dst may be NULL to ask), or -1 for a tensor the layer lacks. */
long orc_hybrid_tensor(const orc_hybrid *m, int layer_idx, int id, float *dst) {
    const mat *w = NULL;
    const float *v = NULL;
    size_t n = 0;
    if (layer_idx < 0) {
        if (id == G_EMBED) {
            n = (size_t)m->c.vocab * m->c.hidden;
            if (dst)
                for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(m->embed[i]);
            return (long)n;
        }
        if (id == G_FINAL_NORM) v = m->final_norm, n = m->c.hidden;
        else if (id == G_LM_HEAD) w = &m->lm;
        else return -1;
    } else {
        if (layer_idx >= m->c.layers) return -1;
        const layer *L = &m->L[layer_idx];
        const int H = m->c.hidden;
        switch (id) {
            case T_LN_IN: v = L->ln_in, n = H; break;
            case T_LN_POST: v = L->ln_post, n = H; break;
            case T_QKV: w = L->attn ? NULL : &L->qkv; break;
            case T_Z: w = L->attn ? NULL : &L->z; break;
            case T_BP: w = L->attn ? NULL : &L->bp; break;
            case T_AP: w = L->attn ? NULL : &L->ap; break;
            case T_OUT: w = L->attn ? NULL : &L->out; break;
            case T_CONVW: v = L->conv_w, n = (size_t)m->conv_dim * 4; break;
            case T_DTBIAS: v = L->dt_bias, n = m->c.gdn_v_heads; break;
            case T_ALOG: v = L->A_log, n = m->c.gdn_v_heads; break;
            case T_NORMW: v = L->norm_w, n = 128; break;
            case T_QP: w = L->attn ? &L->qp : NULL; break;
            case T_KP: w = L->attn ? &L->kp : NULL; break;
            case T_VP: w = L->attn ? &L->vp : NULL; break;
            case T_OP: w = L->attn ? &L->op : NULL; break;
            case T_QN: v = L->q_norm, n = 256; break;
            case T_KN: v = L->k_norm, n = 256; break;
            case T_GATE: w = &L->gate; break;
            case T_UP: w = &L->up; break;
            case T_DOWN: w = &L->down; break;
            default: return -1;
        }
        if (!w && !v) return -1;
    }
    if (w) {
        n = (size_t)w->N * w->K;
        if (dst)
            for (size_t i = 0; i < n; ++i) dst[i] = (float)w->q[i] * w->s[i / w->K];
        return (long)n;
    }
    if (dst) memcpy(dst, v, n * sizeof(float));
    return (long)n;
}

/*
 * gdn_oracle.c -- CPU restatement of the OrionsBelt GDN hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the thing
 * measured or shipped.  See gdn_oracle.h for the function list, the reference
 * file:line each one follows and what pins it.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp).
 */
#include "gdn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

/* ======================================================================== */
/* kai ukernels (portable scalar branches)                                   */
/* ======================================================================== */

/* The channel loops below walk ORC_CB adjacent channels through the
 * sequence together (t outer, the channel group inner: one cache line of
 * each row per step) instead of one channel at a time.  Every channel's
 * operations and their order are unchanged, so the results are those of
 * the reference's channel-by-channel loops, whatever the thread count. */
#define ORC_CB 16
#define ORC_GROUPS(channels) ((long)(((channels) + ORC_CB - 1) / ORC_CB))
#define ORC_GROUP_WIDTH(gg, channels) \
    ((channels) - (size_t)(gg) * ORC_CB < ORC_CB ? (channels) - (size_t)(gg) * ORC_CB : ORC_CB)

void orc_cumdecay_f32(const float *a, float *decay, size_t seq, size_t channels) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (seq * channels > 65536)
#endif
    for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {
        const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);
        float run[ORC_CB];
        for (size_t j = 0; j < n; ++j) run[j] = 1.0f;
        for (size_t t = 0; t < seq; ++t) {
            const float *ar = a + t * channels + c0;
            float *dr = decay + t * channels + c0;
            for (size_t j = 0; j < n; ++j) {
                run[j] = run[j] * ar[j];
                dr[j] = run[j];
            }
        }
    }
}

void orc_gated_scan_f32(const float *g, const float *x, float *s, float *state,
                        size_t seq, size_t channels) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (seq * channels > 65536)
#endif
    for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {
        const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);
        float acc[ORC_CB];
        for (size_t j = 0; j < n; ++j) acc[j] = state[c0 + j];
        for (size_t t = 0; t < seq; ++t) {
            const size_t r = t * channels + c0;
            for (size_t j = 0; j < n; ++j) {
                acc[j] = x[r + j] + acc[j] * g[r + j];
                s[r + j] = acc[j];
            }
        }
        for (size_t j = 0; j < n; ++j) state[c0 + j] = acc[j];
    }
}

void orc_gdn2_gated_scan_f32(const float *g, const float *b, const float *w, const float *x, float *s,
                             float *state, size_t seq, size_t channels) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (seq * channels > 65536)
#endif
    for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {
        const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);
        float acc[ORC_CB];
        for (size_t j = 0; j < n; ++j) acc[j] = state[c0 + j];
        for (size_t t = 0; t < seq; ++t) {
            const size_t r = t * channels + c0;
            for (size_t j = 0; j < n; ++j) {
                acc[j] = w[r + j] * x[r + j] + acc[j] * (g[r + j] * b[r + j]);
                s[r + j] = acc[j];
            }
        }
        for (size_t j = 0; j < n; ++j) state[c0 + j] = acc[j];
    }
}

static void conv_k4(const float *in, const float *w, float *out, float *hist,
                    size_t seq, size_t channels, int silu) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (seq * channels > 65536)
#endif
    for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {
        const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);
        float h0[ORC_CB], h1[ORC_CB], h2[ORC_CB], w0[ORC_CB], w1[ORC_CB], w2[ORC_CB], w3[ORC_CB];
        for (size_t j = 0; j < n; ++j) {
            const size_t c = c0 + j;
            h0[j] = hist[0 * channels + c];
            h1[j] = hist[1 * channels + c];
            h2[j] = hist[2 * channels + c];
            w0[j] = w[0 * channels + c];
            w1[j] = w[1 * channels + c];
            w2[j] = w[2 * channels + c];
            w3[j] = w[3 * channels + c];
        }
        for (size_t t = 0; t < seq; ++t) {
            const size_t r = t * channels + c0;
            for (size_t j = 0; j < n; ++j) {
                const float cur = in[r + j];
                /* left-to-right: ((h0*w0 + h1*w1) + h2*w2) + cur*w3 */
                float acc = h0[j] * w0[j] + h1[j] * w1[j] + h2[j] * w2[j] + cur * w3[j];
                if (silu) acc = acc / (1.0f + expf(-acc));
                out[r + j] = acc;
                h0[j] = h1[j];
                h1[j] = h2[j];
                h2[j] = cur;
            }
        }
        for (size_t j = 0; j < n; ++j) {
            const size_t c = c0 + j;
            hist[0 * channels + c] = h0[j];
            hist[1 * channels + c] = h1[j];
            hist[2 * channels + c] = h2[j];
        }
    }
}

void orc_causal_dwconv1d_f32_k4(const float *in, const float *w, float *out,
                                float *hist, size_t seq, size_t channels) {
    conv_k4(in, w, out, hist, seq, channels, 0);
}

void orc_causal_dwconv1d_silu_f32_k4(const float *in, const float *w, float *out,
                                     float *hist, size_t seq, size_t channels) {
    conv_k4(in, w, out, hist, seq, channels, 1);
}

void orc_gemv_f32(const float *a, const float *b, float *c, size_t k, size_t n) {
    for (size_t j = 0; j < n; ++j) {
        float acc = 0.0f;
        for (size_t kk = 0; kk < k; ++kk) acc = acc + a[kk] * b[kk * n + j];
        c[j] = acc;
    }
}

/* C = A.B, A [m][k], B [k][n], C [m][n] row-major: the portable branch of
 * the reference's delta-rule matmul (gdn_delta_matmul.c:111-118, the same
 * loop as its test's naive_matmul, test_gdn_delta_matmul.c:32-41). */
void orc_delta_rule_matmul_f32(const float *A, const float *B, float *C, size_t m, size_t k, size_t n) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; ++kk) acc = acc + A[i * k + kk] * B[kk * n + j];
            C[i * n + j] = acc;
        }
}

/* ======================================================================== */
/* Narrow formats                                                            */
/* ======================================================================== */

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* binary32 -> binary16, round to nearest even, with subnormals, infinities
 * and NaN (quiet, sign kept).  Written from the IEEE 754 encodings. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;

    if (exp == 0xFFu) /* inf or NaN */
        return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));

    int e = (int)exp - 127 + 15; /* rebiased exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u); /* overflow -> inf */

    if (e <= 0) {
        /* subnormal (or zero) result: value = man24 * 2^(exp-150) expressed in
         * units of 2^-24 (the fp16 subnormal quantum). */
        if (e < -10) return sign; /* below half of the smallest subnormal */
        uint32_t m = man | 0x800000u; /* implicit bit */
        int shift = 14 - e;           /* 24-bit mantissa -> subnormal field */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q); /* q may carry into the exponent field */
    }

    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may carry to inf */
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1Fu) return bits_f32(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        float v = (float)man * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp - 15u + 127u) << 23) | (man << 13));
}

/* Round-to-nearest-even by bias-and-truncate, as gdn_sve.c:81-87 does (no
 * NaN special case there either). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

#define ORC_NARROW_DECAY(name, cvt)                                                      \
    void name(const float *a, uint16_t *decay, size_t seq, size_t channels) {            \
        _Pragma("omp parallel for schedule(static) if (seq * channels > 65536)")          \
        for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {                              \
            const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);     \
            float run[ORC_CB];                                                            \
            for (size_t j = 0; j < n; ++j) run[j] = 1.0f;                                 \
            for (size_t t = 0; t < seq; ++t) {                                            \
                const size_t r = t * channels + c0;                                       \
                for (size_t j = 0; j < n; ++j) {                                          \
                    run[j] = run[j] * a[r + j];                                           \
                    decay[r + j] = cvt(run[j]);                                           \
                }                                                                         \
            }                                                                             \
        }                                                                                 \
    }

#define ORC_NARROW_SCAN(name, to_f32, from_f32)                                          \
    void name(const float *g, const float *x, float *s, uint16_t *state, size_t seq,     \
              size_t channels) {                                                          \
        _Pragma("omp parallel for schedule(static) if (seq * channels > 65536)")          \
        for (long gg = 0; gg < ORC_GROUPS(channels); ++gg) {                              \
            const size_t c0 = (size_t)gg * ORC_CB, n = ORC_GROUP_WIDTH(gg, channels);     \
            float acc[ORC_CB];                                                            \
            for (size_t j = 0; j < n; ++j) acc[j] = to_f32(state[c0 + j]);                \
            for (size_t t = 0; t < seq; ++t) {                                            \
                const size_t r = t * channels + c0;                                       \
                for (size_t j = 0; j < n; ++j) {                                          \
                    acc[j] = x[r + j] + acc[j] * g[r + j];                                \
                    s[r + j] = acc[j];                                                    \
                }                                                                         \
            }                                                                             \
            for (size_t j = 0; j < n; ++j) state[c0 + j] = from_f32(acc[j]);              \
        }                                                                                 \
    }

/* fp32 running product / state, narrowed on store (gdn_sve.c's mixed-
 * precision branches); the same channel grouping as the fp32 loops. */
ORC_NARROW_DECAY(orc_cumdecay_f16, orc_f32_to_f16)
ORC_NARROW_SCAN(orc_gated_scan_f16, orc_f16_to_f32, orc_f32_to_f16)
ORC_NARROW_DECAY(orc_cumdecay_bf16, orc_f32_to_bf16)
ORC_NARROW_SCAN(orc_gated_scan_bf16, orc_bf16_to_f32, orc_f32_to_bf16)

/* ======================================================================== */
/* Matrix-state delta rule                                                   */
/* ======================================================================== */

void orc_delta_rule_head(float *S, const float *k, const float *v, const float *q,
                         float beta, float decay, float *out, size_t hkd, size_t hvd) {
    for (size_t j = 0; j < hkd; ++j)
        for (size_t i = 0; i < hvd; ++i) S[j * hvd + i] = S[j * hvd + i] * decay;
    for (size_t i = 0; i < hvd; ++i) {
        float kv = 0.0f;
        for (size_t j = 0; j < hkd; ++j) kv = kv + S[j * hvd + i] * k[j];
        float delta = (v[i] - kv) * beta;
        for (size_t j = 0; j < hkd; ++j) S[j * hvd + i] = S[j * hvd + i] + k[j] * delta;
        float o = 0.0f;
        for (size_t j = 0; j < hkd; ++j) o = o + S[j * hvd + i] * q[j];
        out[i] = o;
    }
}

static void decode_one(float *Sh, const float *qh, const float *kh, const float *vh,
                       float g, float beta, float *oh, int dk, int dv, float q_scale) {
    float *qbuf = (float *)malloc((size_t)dk * sizeof(float));
    for (int j = 0; j < dk; ++j) qbuf[j] = qh[j] * q_scale;
    orc_delta_rule_head(Sh, kh, vh, qbuf, beta, expf(g), oh, (size_t)dk, (size_t)dv);
    free(qbuf);
}

void orc_delta_rule_decode_f32(float *S, const float *q, const float *k,
                               const float *v, const float *g, const float *beta,
                               float *o, int B, int Hv, int Hk, int dk, int dv,
                               float q_scale) {
    const int rep = Hv / Hk;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) collapse(2)
#endif
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int kh = h / rep;
            float *Sh = S + ((size_t)b * Hv + h) * (size_t)dk * dv;
            decode_one(Sh, q + ((size_t)b * Hk + kh) * dk, k + ((size_t)b * Hk + kh) * dk,
                       v + ((size_t)b * Hv + h) * dv, g[(size_t)b * Hv + h],
                       beta[(size_t)b * Hv + h], o + ((size_t)b * Hv + h) * dv, dk, dv,
                       q_scale);
        }
    }
}

void orc_delta_rule_decode_f16state(uint16_t *S, const float *q, const float *k,
                                    const float *v, const float *g,
                                    const float *beta, float *o, int B, int Hv,
                                    int Hk, int dk, int dv, float q_scale) {
    const int rep = Hv / Hk;
    const size_t hs = (size_t)dk * dv;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) collapse(2)
#endif
    for (int b = 0; b < B; ++b) {
        for (int h = 0; h < Hv; ++h) {
            const int kh = h / rep;
            uint16_t *Sn = S + ((size_t)b * Hv + h) * hs;
            float *Sw = (float *)malloc(hs * sizeof(float));
            for (size_t e = 0; e < hs; ++e) Sw[e] = orc_f16_to_f32(Sn[e]);
            decode_one(Sw, q + ((size_t)b * Hk + kh) * dk, k + ((size_t)b * Hk + kh) * dk,
                       v + ((size_t)b * Hv + h) * dv, g[(size_t)b * Hv + h],
                       beta[(size_t)b * Hv + h], o + ((size_t)b * Hv + h) * dv, dk, dv,
                       q_scale);
            for (size_t e = 0; e < hs; ++e) Sn[e] = orc_f32_to_f16(Sw[e]);
            free(Sw);
        }
    }
}

/* ======================================================================== */
/* Chunkwise gated delta rule (HF torch_chunk_gated_delta_rule)              */
/* ======================================================================== */
/* The body is written once over a scalar type REAL and instantiated for float
 * and double.  Step numbers refer to modeling_qwen3_5.py. */

#define ORC_CHUNK_BODY(REAL, EXPF)                                                        \
    const int rep = Hv / Hk;                                                              \
    const int nchunks = (T + chunk - 1) / chunk;                                          \
    const int C = chunk;                                                                  \
    _Pragma("omp parallel for schedule(dynamic) collapse(2)")                             \
    for (int b = 0; b < B; ++b) {                                                         \
        for (int h = 0; h < Hv; ++h) {                                                    \
            const int kh = h / rep;                                                       \
            REAL *St = (REAL *)malloc((size_t)dk * dv * sizeof(REAL));                    \
            REAL *Q = (REAL *)malloc((size_t)C * dk * sizeof(REAL));                      \
            REAL *K = (REAL *)malloc((size_t)C * dk * sizeof(REAL));                      \
            REAL *V = (REAL *)malloc((size_t)C * dv * sizeof(REAL));                      \
            REAL *KB = (REAL *)malloc((size_t)C * dk * sizeof(REAL));                     \
            REAL *VB = (REAL *)malloc((size_t)C * dv * sizeof(REAL));                     \
            REAL *G = (REAL *)malloc((size_t)C * sizeof(REAL));                           \
            REAL *Bt = (REAL *)malloc((size_t)C * sizeof(REAL));                          \
            REAL *DM = (REAL *)malloc((size_t)C * C * sizeof(REAL));                      \
            REAL *A = (REAL *)malloc((size_t)C * C * sizeof(REAL));                       \
            REAL *row = (REAL *)malloc((size_t)C * sizeof(REAL));                         \
            REAL *U = (REAL *)malloc((size_t)C * dv * sizeof(REAL));                      \
            REAL *W = (REAL *)malloc((size_t)C * dk * sizeof(REAL));                      \
            REAL *AT = (REAL *)malloc((size_t)C * C * sizeof(REAL));                      \
            REAL *VN = (REAL *)malloc((size_t)C * dv * sizeof(REAL));                     \
            REAL *O = (REAL *)malloc((size_t)C * dv * sizeof(REAL));                      \
            REAL *EG = (REAL *)malloc((size_t)C * sizeof(REAL));                          \
            REAL *EL = (REAL *)malloc((size_t)C * sizeof(REAL));                          \
            REAL *KG = (REAL *)malloc((size_t)C * dk * sizeof(REAL));                     \
            float *Sg = S + ((size_t)b * Hv + h) * (size_t)dk * dv;                       \
            for (size_t e = 0; e < (size_t)dk * dv; ++e) St[e] = (REAL)Sg[e];             \
            for (int c = 0; c < nchunks; ++c) {                                           \
                /* load chunk, zero-padding rows past T (:270-276) */                     \
                for (int i = 0; i < C; ++i) {                                             \
                    const int t = c * C + i;                                              \
                    const int live = t < T;                                               \
                    const size_t qk_off = (((size_t)b * T + t) * Hk + kh) * dk;           \
                    const size_t v_off = (((size_t)b * T + t) * Hv + h) * dv;             \
                    const size_t gb_off = ((size_t)b * T + t) * Hv + h;                   \
                    for (int j = 0; j < dk; ++j) {                                        \
                        /* q * scale (:278-279) */                                        \
                        Q[i * dk + j] = live ? (REAL)q[qk_off + j] * (REAL)q_scale : 0;   \
                        K[i * dk + j] = live ? (REAL)k[qk_off + j] : 0;                   \
                    }                                                                     \
                    for (int j = 0; j < dv; ++j) V[i * dv + j] = live ? (REAL)v[v_off + j] : 0; \
                    Bt[i] = live ? (REAL)beta[gb_off] : 0;                                \
                    G[i] = live ? (REAL)g[gb_off] : 0;                                    \
                }                                                                         \
                /* k_beta, v_beta (:281-282) */                                           \
                for (int i = 0; i < C; ++i) {                                             \
                    for (int j = 0; j < dk; ++j) KB[i * dk + j] = K[i * dk + j] * Bt[i];  \
                    for (int j = 0; j < dv; ++j) VB[i * dv + j] = V[i * dv + j] * Bt[i];  \
                }                                                                         \
                /* g = g.cumsum(-1) within the chunk (:291) */                            \
                for (int i = 1; i < C; ++i) G[i] = G[i - 1] + G[i];                       \
                for (int i = 0; i < C; ++i) {                                             \
                    EG[i] = EXPF(G[i]);                                                   \
                    EL[i] = EXPF(G[C - 1] - G[i]);                                        \
                    for (int j = 0; j < dk; ++j) KG[i * dk + j] = KB[i * dk + j] * EG[i]; \
                }                                                                         \
                /* decay_mask = exp(tril(G_i - G_j)) masked to the lower triangle (:292) */ \
                for (int i = 0; i < C; ++i)                                               \
                    for (int j = 0; j < C; ++j)                                           \
                        DM[i * C + j] = j <= i ? EXPF(G[i] - G[j]) : (REAL)0;             \
                /* attn = -((k_beta @ k^T) * decay_mask), upper incl. diagonal = 0 (:293) */ \
                for (int i = 0; i < C; ++i)                                               \
                    for (int j = 0; j < C; ++j) {                                         \
                        if (j >= i) { A[i * C + j] = 0; continue; }                       \
                        REAL s = 0;                                                       \
                        for (int d = 0; d < dk; ++d) s += KB[i * dk + d] * K[j * dk + d]; \
                        A[i * C + j] = -(s * DM[i * C + j]);                              \
                    }                                                                     \
                /* row recursion (:294-297): row_i += row_i @ A[:i,:i] */                 \
                for (int i = 1; i < C; ++i) {                                             \
                    for (int j = 0; j < i; ++j) row[j] = A[i * C + j];                    \
                    for (int j = 0; j < i; ++j) {                                         \
                        REAL s = 0;                                                       \
                        for (int m = 0; m < i; ++m) s += row[m] * A[m * C + j];           \
                        A[i * C + j] = row[j] + s;                                        \
                    }                                                                     \
                }                                                                         \
                for (int i = 0; i < C; ++i) A[i * C + i] += 1; /* + I (:298) */           \
                /* U = A @ v_beta ; W = A @ (k_beta * exp(g)) (:299-300) */               \
                for (int i = 0; i < C; ++i) {                                             \
                    for (int j = 0; j < dv; ++j) {                                        \
                        REAL s = 0;                                                       \
                        for (int m = 0; m < C; ++m) s += A[i * C + m] * VB[m * dv + j];   \
                        U[i * dv + j] = s;                                                \
                    }                                                                     \
                    for (int j = 0; j < dk; ++j) {                                        \
                        REAL s = 0;                                                       \
                        for (int m = 0; m < C; ++m) s += A[i * C + m] * KG[m * dk + j];   \
                        W[i * dk + j] = s;                                                \
                    }                                                                     \
                }                                                                         \
                /* attn = (q @ k^T) * decay_mask (:312) */                                \
                for (int i = 0; i < C; ++i)                                               \
                    for (int j = 0; j < C; ++j) {                                         \
                        REAL s = 0;                                                       \
                        for (int d = 0; d < dk; ++d) s += Q[i * dk + d] * K[j * dk + d];  \
                        AT[i * C + j] = s * DM[i * C + j];                                \
                    }                                                                     \
                /* v_new = U - W @ S (:313-314) */                                        \
                for (int i = 0; i < C; ++i)                                               \
                    for (int j = 0; j < dv; ++j) {                                        \
                        REAL s = 0;                                                       \
                        for (int d = 0; d < dk; ++d) s += W[i * dk + d] * St[d * dv + j]; \
                        VN[i * dv + j] = U[i * dv + j] - s;                               \
                    }                                                                     \
                /* o = (q * exp(g)) @ S + attn @ v_new (:315-316) */                      \
                for (int i = 0; i < C; ++i) {                                             \
                    const REAL eg = EG[i];                                                \
                    for (int j = 0; j < dv; ++j) {                                        \
                        REAL s = 0;                                                       \
                        for (int d = 0; d < dk; ++d) s += (Q[i * dk + d] * eg) * St[d * dv + j]; \
                        REAL s2 = 0;                                                      \
                        for (int m = 0; m < C; ++m) s2 += AT[i * C + m] * VN[m * dv + j]; \
                        O[i * dv + j] = s + s2;                                           \
                    }                                                                     \
                }                                                                         \
                /* S = S * exp(g_last) + (k * exp(g_last - g))^T @ v_new (:317-320) */    \
                {                                                                         \
                    const REAL el = EG[C - 1];                                            \
                    for (int d = 0; d < dk; ++d)                                          \
                        for (int j = 0; j < dv; ++j) {                                    \
                            REAL s = 0;                                                   \
                            for (int m = 0; m < C; ++m)                                   \
                                s += (K[m * dk + d] * EL[m]) * VN[m * dv + j];            \
                            St[d * dv + j] = St[d * dv + j] * el + s;                     \
                        }                                                                 \
                }                                                                         \
                /* write the live rows of this chunk (:324-326) */                        \
                for (int i = 0; i < C; ++i) {                                             \
                    const int t = c * C + i;                                              \
                    if (t >= T) break;                                                    \
                    float *orow = o + (((size_t)b * T + t) * Hv + h) * dv;                \
                    for (int j = 0; j < dv; ++j) orow[j] = (float)O[i * dv + j];          \
                }                                                                         \
            }                                                                             \
            for (size_t e = 0; e < (size_t)dk * dv; ++e) Sg[e] = (float)St[e];            \
            free(St); free(Q); free(K); free(V); free(KB); free(VB); free(G); free(Bt);   \
            free(DM); free(A); free(row); free(U); free(W); free(AT); free(VN); free(O);  \
            free(EG); free(EL); free(KG);                                                 \
        }                                                                                 \
    }

void orc_chunk_gdr_f32(const float *q, const float *k, const float *v,
                       const float *g, const float *beta, float *o, float *S,
                       int B, int T, int Hv, int Hk, int dk, int dv, int chunk,
                       float q_scale) {
    ORC_CHUNK_BODY(float, expf)
}

void orc_chunk_gdr_f64(const float *q, const float *k, const float *v,
                       const float *g, const float *beta, float *o, float *S,
                       int B, int T, int Hv, int Hk, int dk, int dv, int chunk,
                       float q_scale) {
    ORC_CHUNK_BODY(double, exp)
}

/* ---- layer glue: gating prologue and gated RMSNorm ------------------------ */

/* Qwen3_5GatedDeltaNet.forward:497-499 and l2norm:242-245 (see header). */
static float softplus_torch(float y) { return y > 20.f ? y : log1pf(expf(y)); }

void orc_gating_prologue_f32(const float *x, const float *a, const float *b,
                             const float *A_log, const float *dt_bias, float *q,
                             float *k, float *v, float *g, float *beta, size_t rows,
                             int Hk, int Hv) {
    const int D = 128, H = 2 * Hk + Hv;
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * (size_t)H * D;
        for (int h = 0; h < H; ++h) {
            const float *xh = xr + (size_t)h * D;
            float *dst = h < Hk ? q + (r * Hk + h) * D
                       : h < 2 * Hk ? k + (r * Hk + (h - Hk)) * D
                                    : v + (r * Hv + (h - 2 * Hk)) * D;
            if (h < 2 * Hk) {
                double ss = 0.0;
                for (int i = 0; i < D; ++i) ss += (double)xh[i] * xh[i];
                const float inv = 1.0f / sqrtf((float)ss + 1e-6f);
                for (int i = 0; i < D; ++i) dst[i] = xh[i] * inv;
            } else {
                for (int i = 0; i < D; ++i) dst[i] = xh[i];
            }
        }
        for (int h = 0; h < Hv; ++h) {
            const size_t i = r * Hv + h;
            g[i] = -expf(A_log[h]) * softplus_torch(a[i] + dt_bias[h]);
            beta[i] = 1.0f / (1.0f + expf(-b[i]));
        }
    }
}

/* Qwen3_5RMSNormGated.forward:175-184 (see header). */
static float silu_f32(float z) { return z / (1.0f + expf(-z)); }

static float row_inv_rms(const float *x, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    const float var = (float)ss / (float)n;
    return 1.0f / sqrtf(var + eps);
}

void orc_gated_rmsnorm_f32(const float *o, const float *z, const float *w, float *y,
                           size_t rows, int n, float eps) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        const float *orow = o + r * n, *zrow = z + r * n;
        const float inv = row_inv_rms(orow, n, eps);
        for (int i = 0; i < n; ++i) {
            const float h = orow[i] * inv;
            y[r * n + i] = (w[i] * h) * silu_f32(zrow[i]);
        }
    }
}

void orc_gated_rmsnorm_bf16(const uint16_t *o, const uint16_t *z, const uint16_t *w,
                            uint16_t *y, size_t rows, int n, float eps) {
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        float row[n];
        for (int i = 0; i < n; ++i) row[i] = orc_bf16_to_f32(o[r * n + i]);
        const float inv = row_inv_rms(row, n, eps);
        for (int i = 0; i < n; ++i) {
            const float h = orc_bf16_to_f32(orc_f32_to_bf16(row[i] * inv));
            const float hw = orc_bf16_to_f32(orc_f32_to_bf16(orc_bf16_to_f32(w[i]) * h));
            y[r * n + i] = orc_f32_to_bf16(hw * silu_f32(orc_bf16_to_f32(z[r * n + i])));
        }
    }
}

/* ---- decode-step conv on HF's state layout (see header) ------------------- */

void orc_causal_conv1d_update_f32(const float *x, float *conv_state, const float *w,
                                  float *out, int B, int T, size_t C, int silu) {
    for (int b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c) {
            float *s = conv_state + ((size_t)b * C + c) * 4;
            const float *wc = w + c * 4;
            for (int t = 0; t < T; ++t) {
                const size_t i = ((size_t)b * T + t) * C + c;
                const float cur = x[i];
                float acc = s[1] * wc[0] + s[2] * wc[1] + s[3] * wc[2] + cur * wc[3];
                if (silu) acc = acc / (1.0f + expf(-acc));
                out[i] = acc;
                s[0] = s[1];
                s[1] = s[2];
                s[2] = s[3];
                s[3] = cur;
            }
        }
}

/* ---- int8 weight-only matmul (see header) --------------------------------- */

void orc_w8_quantize(const float *W, int8_t *Wq, float *scale, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        const float *row = W + (size_t)n * K;
        float max_abs = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float v = fabsf(row[k]);
            if (v > max_abs) max_abs = v;
        }
        const float s = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        scale[n] = s;
        for (int k = 0; k < K; ++k) {
            long vi = lroundf(row[k] * inv);
            if (vi > 127) vi = 127;
            if (vi < -128) vi = -128;
            Wq[(size_t)n * K + k] = (int8_t)vi;
        }
    }
}

static float f16_bits_to_float(uint16_t h) { return orc_f16_to_f32(h); }

void orc_w8_gemm(const uint16_t *x, const int8_t *Wq, const float *scale, float *y, int M,
                 int N, int K) {
    /* the activations widened once (the same values the sum would widen) */
    float *xf = malloc(sizeof(float) * (size_t)M * K);
    for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = f16_bits_to_float(x[i]);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k)
                acc += (double)xf[(size_t)m * K + k] * Wq[(size_t)n * K + k];
            y[(size_t)m * N + n] = (float)acc * scale[n];
        }
    free(xf);
}

/* ---- attention decode (see header) ---------------------------------------- */

void orc_attn_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *out, int B,
                     int Hq, int Hkv, int Tmax, int L, int D, float scaling) {
    const int rep = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h) {
            const int kv = h / rep;
            const uint16_t *qh = q + ((size_t)b * Hq + h) * D;
            const size_t base = ((size_t)b * Hkv + kv) * Tmax;
            double *s = malloc(sizeof(double) * L), mx = -1e300, sum = 0.0;
            for (int t = 0; t < L; ++t) {
                double dot = 0.0;
                for (int d = 0; d < D; ++d)
                    dot += (double)orc_f16_to_f32(qh[d]) * orc_f16_to_f32(k[(base + t) * D + d]);
                s[t] = dot * scaling;
                if (s[t] > mx) mx = s[t];
            }
            for (int t = 0; t < L; ++t) {
                s[t] = exp(s[t] - mx);
                sum += s[t];
            }
            for (int d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int t = 0; t < L; ++t) acc += s[t] * orc_f16_to_f32(v[(base + t) * D + d]);
                out[((size_t)b * Hq + h) * D + d] = (float)(acc / sum);
            }
            free(s);
        }
}

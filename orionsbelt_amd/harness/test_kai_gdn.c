/*
 * test_kai_gdn.c -- test harness for the GDN kai entry points on MI355X.
 *
 * Keeps the reference harness's interface (kleidiai_submission/
 * test_kai_gdn.c:643-676): `int main(void)`, one "[ RUN      ] name" line
 * per suite followed by "[       OK ] name" or "[  FAILED  ] name", a
 * "Tests run:" / "Tests failed:" summary, "ALL TESTS PASSED" and exit 0 on
 * success, "SOME TESTS FAILED" and exit 1 otherwise.  The 14 suites cover
 * the same cases as the reference (sizes test_kai_gdn.c:167-168, LCG inputs
 * with the same value ranges and tolerances, continuity, tails, degenerate
 * sizes) against naive scalar references written here; further suites
 * exercise the device-pointer entry points of include/kai_gdn_hip.h.
 *
 * Build: python -m orionsbelt_amd.build  (links libkai_gdn_hip.so)
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kai/ukernels/gdn/kai_gdn_causal_dwconv1d_f32_k4_sve.h"
#include "kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.h"
#include "kai/ukernels/gdn/kai_gdn_gated_scan_f32_sve.h"
#include "kai/ukernels/gdn/kai_gdn_gemv_f32_f32_f32_1x4_neon.h"
#include "kai_gdn_hip.h"

static int n_run, n_failed;

static void *alloc(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(1);
    }
    return p;
}

/* 32-bit LCG, the generator the reference test seeds with 0x5EED1234 */
static uint32_t rng = 0x5EED1234u;
static float urand(float lo, float hi) {
    rng = rng * 1103515245u + 12345u;
    return lo + ((float)((rng >> 8) & 0xFFFFFFu) / (float)0xFFFFFFu) * (hi - lo);
}
static void fill(float *p, size_t n, float lo, float hi) {
    for (size_t i = 0; i < n; ++i) p[i] = urand(lo, hi);
}

static int close_enough(float a, float b, float atol, float rtol) {
    float d = fabsf(a - b);
    return d <= atol || d <= rtol * fmaxf(fabsf(a), fabsf(b));
}

static int compare(const float *got, const float *want, size_t n, const char *what, float atol,
                   float rtol) {
    size_t bad = 0;
    for (size_t i = 0; i < n; ++i) {
        if (!close_enough(got[i], want[i], atol, rtol)) {
            if (bad < 8)
                printf("  %s[%zu]: got %.7e want %.7e (diff %.3e)\n", what, i, got[i], want[i],
                       fabsf(got[i] - want[i]));
            ++bad;
        }
    }
    if (bad) printf("  %s: %zu of %zu outside tolerance\n", what, bad, n);
    return bad == 0;
}

#define SUITE(name, body)                                     \
    do {                                                      \
        ++n_run;                                              \
        printf("[ RUN      ] %s\n", name);                    \
        int ok_ = (body);                                     \
        if (ok_) printf("[       OK ] %s\n\n", name);         \
        else {                                                \
            ++n_failed;                                       \
            printf("[  FAILED  ] %s\n\n", name);              \
        }                                                     \
    } while (0)

/* ---- naive references ---------------------------------------------------- */

static void naive_cumdecay(const float *a, float *d, size_t T, size_t C) {
    for (size_t c = 0; c < C; ++c) {
        float p = 1.0f;
        for (size_t t = 0; t < T; ++t) d[t * C + c] = (p = p * a[t * C + c]);
    }
}

static void naive_scan(const float *g, const float *x, float *s, float *st, size_t T, size_t C) {
    for (size_t c = 0; c < C; ++c) {
        float v = st[c];
        for (size_t t = 0; t < T; ++t) s[t * C + c] = (v = x[t * C + c] + v * g[t * C + c]);
        st[c] = v;
    }
}

static void naive_conv(const float *in, const float *w, float *out, float *h, size_t T, size_t C,
                       int silu) {
    for (size_t c = 0; c < C; ++c) {
        float x0 = h[c], x1 = h[C + c], x2 = h[2 * C + c];
        for (size_t t = 0; t < T; ++t) {
            float x3 = in[t * C + c];
            float y = x0 * w[c] + x1 * w[C + c] + x2 * w[2 * C + c] + x3 * w[3 * C + c];
            out[t * C + c] = silu ? y / (1.0f + expf(-y)) : y;
            x0 = x1;
            x1 = x2;
            x2 = x3;
        }
        h[c] = x0;
        h[C + c] = x1;
        h[2 * C + c] = x2;
    }
}

static void naive_gemv(const float *a, const float *b, float *c, size_t K, size_t N) {
    for (size_t j = 0; j < N; ++j) {
        float s = 0.0f;
        for (size_t k = 0; k < K; ++k) s = s + a[k] * b[k * N + j];
        c[j] = s;
    }
}

/* ---- the reference suites -------------------------------------------------- */

static const size_t SEQS[] = {1, 4, 16, 64};
static const size_t CHANS[] = {1, 3, 7, 8, 12, 16, 17, 32, 33, 128};
#define NELEM(a) (sizeof(a) / sizeof((a)[0]))

static int cumdecay_case(size_t T, size_t C, float lo, float hi, float atol, float rtol) {
    size_t n = T * C;
    float *a = alloc(n * 4), *got = alloc(n * 4), *want = alloc(n * 4);
    fill(a, n, lo, hi);
    naive_cumdecay(a, want, T, C);
    kai_run_gdn_cumdecay_f32_sve(a, got, T, C);
    int ok = compare(got, want, n, "cumdecay", atol, rtol);
    free(a), free(got), free(want);
    return ok;
}

static int scan_case(size_t T, size_t C) {
    size_t n = T * C;
    float *g = alloc(n * 4), *x = alloc(n * 4), *s = alloc(n * 4), *sw = alloc(n * 4);
    float *st = alloc(C * 4), *stw = alloc(C * 4);
    fill(g, n, -0.99f, 0.99f);
    fill(x, n, -2.0f, 2.0f);
    fill(st, C, -1.0f, 1.0f);
    memcpy(stw, st, C * 4);
    naive_scan(g, x, sw, stw, T, C);
    kai_run_gdn_gated_scan_f32_sve(g, x, s, st, T, C);
    int ok = compare(s, sw, n, "gated_scan output", 1e-4f, 5e-4f) &
             compare(st, stw, C, "gated_scan state", 1e-4f, 5e-4f);
    free(g), free(x), free(s), free(sw), free(st), free(stw);
    return ok;
}

static int conv_case(size_t T, size_t C) {
    size_t n = T * C;
    float *in = alloc(n * 4), *w = alloc(16 * C), *o = alloc(n * 4), *ow = alloc(n * 4);
    float *h = alloc(12 * C), *hw = alloc(12 * C);
    fill(in, n, -1.0f, 1.0f);
    fill(w, 4 * C, -1.0f, 1.0f);
    fill(h, 3 * C, -1.0f, 1.0f);
    memcpy(hw, h, 12 * C);
    naive_conv(in, w, ow, hw, T, C, 0);
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in, w, o, h, T, C);
    int ok = compare(o, ow, n, "dwconv1d output", 1e-4f, 5e-4f) &
             compare(h, hw, 3 * C, "dwconv1d history", 1e-4f, 5e-4f);
    free(in), free(w), free(o), free(ow), free(h), free(hw);
    return ok;
}

static int gemv_case(size_t K, size_t N) {
    float *a = alloc(K * 4), *b = alloc(K * N * 4), *c = alloc(N * 4), *cw = alloc(N * 4);
    fill(a, K, -1.0f, 1.0f);
    fill(b, K * N, -1.0f, 1.0f);
    naive_gemv(a, b, cw, K, N);
    kai_run_gdn_gemv_f32_f32_f32_1x4_neon(a, b, c, K, N);
    int ok = compare(c, cw, N, "gemv", 1e-3f, 5e-3f);
    free(a), free(b), free(c), free(cw);
    return ok;
}

static int t_cumdecay(void) {
    int ok = 1;
    for (size_t i = 0; i < NELEM(SEQS); ++i)
        for (size_t j = 0; j < NELEM(CHANS); ++j)
            ok &= cumdecay_case(SEQS[i], CHANS[j], 0.5f, 1.5f, 1e-5f, 1e-4f);
    return ok;
}

static int t_gated_scan(void) {
    int ok = 1;
    for (size_t i = 0; i < NELEM(SEQS); ++i)
        for (size_t j = 0; j < NELEM(CHANS); ++j) ok &= scan_case(SEQS[i], CHANS[j]);
    return ok;
}

static int t_conv(void) {
    int ok = 1;
    for (size_t i = 0; i < NELEM(SEQS); ++i)
        for (size_t j = 0; j < NELEM(CHANS); ++j) ok &= conv_case(SEQS[i], CHANS[j]);
    return ok;
}

static int t_gemv(void) {
    static const size_t K[] = {1, 4, 16, 64, 128};
    static const size_t N[] = {1, 3, 4, 7, 8, 16, 17, 32, 33, 128, 256};
    int ok = 1;
    for (size_t i = 0; i < NELEM(K); ++i)
        for (size_t j = 0; j < NELEM(N); ++j) ok &= gemv_case(K[i], N[j]);
    return ok;
}

static int t_scan_continuity(void) {
    const size_t C = 16, T1 = 8, T2 = 8, T = T1 + T2;
    float *g = alloc(T * C * 4), *x = alloc(T * C * 4), *s = alloc(T * C * 4),
          *sw = alloc(T * C * 4), *st = alloc(C * 4), *stw = alloc(C * 4);
    fill(g, T * C, -0.99f, 0.99f);
    fill(x, T * C, -2.0f, 2.0f);
    fill(stw, C, -1.0f, 1.0f);
    memcpy(st, stw, C * 4);
    naive_scan(g, x, sw, stw, T, C);
    kai_run_gdn_gated_scan_f32_sve(g, x, s, st, T1, C);
    kai_run_gdn_gated_scan_f32_sve(g + T1 * C, x + T1 * C, s + T1 * C, st, T2, C);
    int ok = compare(s, sw, T * C, "scan continuity", 1e-4f, 5e-4f) &
             compare(st, stw, C, "scan continuity state", 1e-4f, 5e-4f);
    free(g), free(x), free(s), free(sw), free(st), free(stw);
    return ok;
}

static int t_conv_continuity(void) {
    const size_t C = 17, T1 = 8, T2 = 8, T = T1 + T2;
    float *in = alloc(T * C * 4), *w = alloc(16 * C), *o = alloc(T * C * 4),
          *ow = alloc(T * C * 4), *h = alloc(12 * C), *hw = alloc(12 * C);
    fill(in, T * C, -1.0f, 1.0f);
    fill(w, 4 * C, -1.0f, 1.0f);
    fill(hw, 3 * C, -1.0f, 1.0f);
    memcpy(h, hw, 12 * C);
    naive_conv(in, w, ow, hw, T, C, 0);
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in, w, o, h, T1, C);
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in + T1 * C, w, o + T1 * C, h, T2, C);
    int ok = compare(o, ow, T * C, "conv continuity", 1e-4f, 5e-4f) &
             compare(h, hw, 3 * C, "conv continuity hist", 1e-4f, 5e-4f);
    free(in), free(w), free(o), free(ow), free(h), free(hw);
    return ok;
}

static int t_gemv_tail(void) {
    static const size_t K[] = {1, 128, 1024};
    static const size_t N[] = {1, 3, 5, 7, 130, 257};
    int ok = 1;
    for (size_t i = 0; i < NELEM(K); ++i)
        for (size_t j = 0; j < NELEM(N); ++j) ok &= gemv_case(K[i], N[j]);
    return ok;
}

static int t_cumdecay_tail(void) {
    static const size_t T[] = {1, 7, 64};
    static const size_t C[] = {1, 3, 5, 17, 128, 129};
    int ok = 1;
    for (size_t i = 0; i < NELEM(T); ++i)
        for (size_t j = 0; j < NELEM(C); ++j) ok &= cumdecay_case(T[i], C[j], 0.1f, 0.99f, 1e-6f, 1e-5f);
    return ok;
}

static int t_scan_tail(void) {
    static const size_t C[] = {1, 3, 5, 17, 129, 255};
    int ok = 1;
    for (size_t j = 0; j < NELEM(C); ++j) ok &= scan_case(16, C[j]);
    return ok;
}

static int t_conv_tail(void) {
    static const size_t C[] = {1, 3, 5, 17, 129};
    int ok = 1;
    for (size_t j = 0; j < NELEM(C); ++j) ok &= conv_case(16, C[j]);
    return ok;
}

static int t_degenerate_cumdecay(void) {
    float a[1] = {0}, d[1] = {42.0f};
    kai_run_gdn_cumdecay_f32_sve(a, d, 0, 8);
    kai_run_gdn_cumdecay_f32_sve(a, d, 8, 0);
    return d[0] == 42.0f;
}

static int t_degenerate_scan(void) {
    float g[8] = {0}, x[8] = {0}, s[8];
    float st[4] = {1.0f, -2.0f, 3.0f, -4.0f}, st1[1] = {42.0f};
    kai_run_gdn_gated_scan_f32_sve(g, x, s, st, 0, 4);
    kai_run_gdn_gated_scan_f32_sve(g, x, s, st1, 8, 0);
    return st[0] == 1.0f && st[1] == -2.0f && st[2] == 3.0f && st[3] == -4.0f && st1[0] == 42.0f;
}

static int t_degenerate_conv(void) {
    float in[1] = {0}, w[12] = {0}, o[1];
    float h[6] = {1, 2, 3, 4, 5, 6}, h1[1] = {42.0f};
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in, w, o, h, 0, 2);
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(in, w, o, h1, 4, 0);
    for (int i = 0; i < 6; ++i)
        if (h[i] != (float)(i + 1)) return 0;
    return h1[0] == 42.0f;
}

static int t_degenerate_gemv(void) {
    float a[4] = {1, 2, 3, 4}, b[1] = {0}, c[8], c1[1] = {42.0f};
    memset(c, 0xFF, sizeof c);
    kai_run_gdn_gemv_f32_f32_f32_1x4_neon(a, b, c, 0, 8);
    kai_run_gdn_gemv_f32_f32_f32_1x4_neon(a, b, c1, 4, 0);
    for (int i = 0; i < 8; ++i)
        if (c[i] != 0.0f) return 0;
    return c1[0] == 42.0f;
}

/* ---- device-pointer entry points ------------------------------------------ */

#define HIPOK(x)                                                                    \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            printf("  %s: %s\n", #x, hipGetErrorString(e_));                        \
            return 0;                                                               \
        }                                                                           \
    } while (0)

static void *to_dev(const void *h, size_t n) {
    void *d = NULL;
    if (hipMalloc(&d, n ? n : 4) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        exit(1);
    }
    if (h && n && hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) {
        fprintf(stderr, "hipMemcpy failed\n");
        exit(1);
    }
    return d;
}

/* conv + SiLU (config-1 shape), device pointers, vs the naive reference */
static int t_dev_conv_silu(void) {
    const size_t T = 4096, C = 8192, n = T * C;
    float *in = alloc(n * 4), *w = alloc(16 * C), *o = alloc(n * 4), *ow = alloc(n * 4);
    float *h = alloc(12 * C), *hw = alloc(12 * C);
    fill(in, n, -2.0f, 2.0f);
    fill(w, 4 * C, -0.5f, 0.5f);
    memset(h, 0, 12 * C);
    memset(hw, 0, 12 * C);
    naive_conv(in, w, ow, hw, T, C, 1);
    float *din = to_dev(in, n * 4), *dw = to_dev(w, 16 * C), *dh = to_dev(h, 12 * C);
    float *dout = to_dev(NULL, n * 4);
    int rc = kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(din, dw, dout, dh, T, C, NULL);
    if (rc) {
        printf("  conv silu: %s\n", kai_gdn_hip_error_string(rc));
        return 0;
    }
    HIPOK(hipMemcpy(o, dout, n * 4, hipMemcpyDeviceToHost));
    HIPOK(hipMemcpy(h, dh, 12 * C, hipMemcpyDeviceToHost));
    int ok = compare(o, ow, n, "conv+silu", 1e-6f, 1e-5f) & compare(h, hw, 3 * C, "hist", 0, 0);
    hipFree(din), hipFree(dw), hipFree(dh), hipFree(dout);
    free(in), free(w), free(o), free(ow), free(h), free(hw);
    return ok;
}

/* matrix delta rule, one token: the reference validator's 4B case
 * (gdn_gpu_validate.c:623, 32 heads of 128x128, beta 0.5, decay 0.9) with
 * per-head arrays holding the scalar values and q_scale = 1 */
static void naive_delta(float *S, const float *k, const float *v, const float *q, float beta,
                        float decay, float *out, size_t dk, size_t dv) {
    for (size_t e = 0; e < dk * dv; ++e) S[e] = S[e] * decay;
    for (size_t i = 0; i < dv; ++i) {
        float kv = 0.0f, o = 0.0f;
        for (size_t j = 0; j < dk; ++j) kv = kv + S[j * dv + i] * k[j];
        float delta = (v[i] - kv) * beta;
        for (size_t j = 0; j < dk; ++j) S[j * dv + i] = S[j * dv + i] + k[j] * delta;
        for (size_t j = 0; j < dk; ++j) o = o + S[j * dv + i] * q[j];
        out[i] = o;
    }
}

static void l2n(float *x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    s = sqrtf(s);
    if (s > 0)
        for (size_t i = 0; i < n; ++i) x[i] /= s;
}

static int t_dev_delta_rule(void) {
    const int H = 32, d = 128;
    const size_t ns = (size_t)H * d * d;
    float *S = alloc(ns * 4), *Sw = alloc(ns * 4), *k = alloc(H * d * 4), *q = alloc(H * d * 4);
    float *v = alloc(H * d * 4), *o = alloc(H * d * 4), *ow = alloc(H * d * 4);
    float g[32], beta[32];
    fill(S, ns, -0.01f, 0.01f);
    memcpy(Sw, S, ns * 4);
    fill(k, H * d, -1.0f, 1.0f);
    fill(v, H * d, -0.5f, 0.5f);
    fill(q, H * d, -1.0f, 1.0f);
    for (int h = 0; h < H; ++h) {
        l2n(k + h * d, d);
        l2n(q + h * d, d);
        g[h] = logf(0.9f);
        beta[h] = 0.5f;
    }
    const float decay = expf(logf(0.9f));
    for (int h = 0; h < H; ++h)
        naive_delta(Sw + (size_t)h * d * d, k + h * d, v + h * d, q + h * d, 0.5f, decay,
                    ow + h * d, d, d);
    float *dS = to_dev(S, ns * 4), *dk = to_dev(k, H * d * 4), *dq = to_dev(q, H * d * 4);
    float *dv = to_dev(v, H * d * 4), *dg = to_dev(g, sizeof g), *db = to_dev(beta, sizeof beta);
    float *dout = to_dev(NULL, H * d * 4);
    int rc = kai_run_gdn_delta_rule_decode_f32_hip(dS, dq, dk, dv, dg, db, dout, 1, H, H, d, d,
                                                   1.0f, NULL);
    if (rc) {
        printf("  delta rule: %s\n", kai_gdn_hip_error_string(rc));
        return 0;
    }
    HIPOK(hipMemcpy(S, dS, ns * 4, hipMemcpyDeviceToHost));
    HIPOK(hipMemcpy(o, dout, H * d * 4, hipMemcpyDeviceToHost));
    int ok = compare(o, ow, H * d, "delta out", 1e-5f, 1e-4f) &
             compare(S, Sw, ns, "delta state", 1e-6f, 1e-4f);
    hipFree(dS), hipFree(dk), hipFree(dq), hipFree(dv), hipFree(dg), hipFree(db), hipFree(dout);
    free(S), free(Sw), free(k), free(q), free(v), free(o), free(ow);
    return ok;
}

int main(void) {
    setvbuf(stdout, NULL, _IOLBF, 0);
    printf("=== GDN kai entry points on MI355X (libkai_gdn_hip) ===\n\n");
    SUITE("test_cumdecay", t_cumdecay());
    SUITE("test_gated_scan", t_gated_scan());
    SUITE("test_causal_dwconv1d", t_conv());
    SUITE("test_gemv", t_gemv());
    SUITE("test_gated_scan_continuity", t_scan_continuity());
    SUITE("test_dwconv1d_continuity", t_conv_continuity());

    printf("\n--- Edge-case tests (tail handling) ---\n\n");
    SUITE("test_gemv_tail", t_gemv_tail());
    SUITE("test_cumdecay_tail", t_cumdecay_tail());
    SUITE("test_gated_scan_tail", t_scan_tail());
    SUITE("test_dwconv1d_tail", t_conv_tail());

    printf("\n--- Degenerate-input tests ---\n\n");
    SUITE("test_degenerate_cumdecay", t_degenerate_cumdecay());
    SUITE("test_degenerate_gated_scan", t_degenerate_scan());
    SUITE("test_degenerate_dwconv1d", t_degenerate_conv());
    SUITE("test_degenerate_gemv", t_degenerate_gemv());

    printf("\n--- Device-pointer entry points ---\n\n");
    SUITE("test_dwconv1d_silu_device", t_dev_conv_silu());
    SUITE("test_delta_rule_decode_device", t_dev_delta_rule());

    printf("=== Summary ===\n");
    printf("Tests run:    %d\n", n_run);
    printf("Tests failed: %d\n", n_failed);
    if (n_failed == 0) {
        printf("\nALL TESTS PASSED\n");
        return 0;
    }
    printf("\nSOME TESTS FAILED\n");
    return 1;
}

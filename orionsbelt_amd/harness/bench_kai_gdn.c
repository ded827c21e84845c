/*
 * bench_kai_gdn.c -- microbenchmark of the GDN kai entry points on MI355X.
 *
 * Keeps the reference harness's interface (kleidiai_submission/
 * bench_kai_gdn.c:248-298): `--repeats N` (default 30), `--csv`, CSV header
 *     kernel,shape,seq,channels,repeats,p50_us,gib_per_s_p50
 * p50 by nearest rank (bench_kai_gdn.c:55-60) and the reference's byte
 * formulas per kernel (bench_kai_gdn.c:311-380).
 *
 * Two kinds of rows:
 *   <kernel>       the drop-in kai symbol called with HOST buffers, as the
 *                  reference harness calls it: wall time per call including
 *                  the host<->device copies (PCIe), 20 warmups, each sample
 *                  a batch of calls (bench_kai_gdn.c:86-95);
 *   <kernel>_dev   the *_hip entry point on device buffers already in HBM:
 *                  hipEvent time per launch, 20 warmups.
 * The reference shapes (64/1 x 160/2560, GEMV K=128) are followed by the
 * MI355X-sized shapes of the measurement plan (conv [4096][8192] + SiLU,
 * cumdecay [4096][8192], decode B=64 x 32 heads x 128x128).
 */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <hip/hip_runtime_api.h>

#include "kai/ukernels/gdn/kai_gdn_causal_dwconv1d_f32_k4_sve.h"
#include "kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.h"
#include "kai/ukernels/gdn/kai_gdn_gated_scan_f32_sve.h"
#include "kai/ukernels/gdn/kai_gdn_gemv_f32_f32_f32_1x4_neon.h"
#include "kai_gdn_hip.h"

static int g_csv;

static double wall_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

static int by_value(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

static double median(double *v, int n) {
    qsort(v, (size_t)n, sizeof *v, by_value);
    int i = (int)(0.5 * (n - 1) + 0.5);
    return v[i < 0 ? 0 : (i >= n ? n - 1 : i)];
}

static void *xalloc(size_t n) {
    void *p = malloc(n);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(1);
    }
    return p;
}

static void *dalloc(size_t n) {
    void *p = NULL;
    if (hipMalloc(&p, n) != hipSuccess) {
        fprintf(stderr, "hipMalloc(%zu) failed\n", n);
        exit(1);
    }
    hipMemset(p, 0x3f, n); /* ~0.747f per float, as the reference fills */
    return p;
}

static void row(const char *name, const char *shape, long seq, long ch, int reps, double us,
                double bytes) {
    double gib = bytes / (us * 1e-6) / (1024.0 * 1024.0 * 1024.0);
    printf("%s,%s,%ld,%ld,%d,%.3f,%.2f\n", name, shape, seq, ch, reps, us, gib);
}

typedef void (*host_fn)(void *);
typedef int (*dev_fn)(void *);

static void bench_host(const char *name, const char *shape, long seq, long ch, int reps,
                       host_fn fn, void *ctx, double bytes) {
    for (int i = 0; i < 20; ++i) fn(ctx);
    int batch = 10;
    double *s = xalloc((size_t)reps * sizeof *s);
    for (int i = 0; i < reps; ++i) {
        double t0 = wall_us();
        for (int b = 0; b < batch; ++b) fn(ctx);
        s[i] = (wall_us() - t0) / batch;
    }
    row(name, shape, seq, ch, reps, median(s, reps), bytes);
    free(s);
}

static void bench_dev(const char *name, const char *shape, long seq, long ch, int reps,
                      dev_fn fn, void *ctx, double bytes) {
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    for (int i = 0; i < 20; ++i)
        if (fn(ctx)) {
            fprintf(stderr, "%s launch failed\n", name);
            exit(1);
        }
    double *s = xalloc((size_t)reps * sizeof *s);
    for (int i = 0; i < reps; ++i) {
        hipEventRecord(a, NULL);
        fn(ctx);
        hipEventRecord(b, NULL);
        hipEventSynchronize(b);
        float ms = 0;
        hipEventElapsedTime(&ms, a, b);
        s[i] = ms * 1e3;
    }
    row(name, shape, seq, ch, reps, median(s, reps), bytes);
    free(s);
    hipEventDestroy(a);
    hipEventDestroy(b);
}

/* ---- call wrappers ---------------------------------------------------------- */

typedef struct { float *a, *d, *x, *s, *st, *w, *h; size_t T, C; } sctx;
typedef struct { float *a, *b, *c; size_t k, n; } gctx;
typedef struct { float *S, *q, *k, *v, *g, *beta, *o; int B, Hv, Hk, d; } dctx;

static void h_cumdecay(void *p) { sctx *c = p; kai_run_gdn_cumdecay_f32_sve(c->a, c->d, c->T, c->C); }
static void h_scan(void *p) {
    sctx *c = p;
    kai_run_gdn_gated_scan_f32_sve(c->a, c->x, c->s, c->st, c->T, c->C);
}
static void h_conv(void *p) {
    sctx *c = p;
    kai_run_gdn_causal_dwconv1d_f32_k4_sve(c->x, c->w, c->s, c->h, c->T, c->C);
}
static void h_gemv(void *p) { gctx *c = p; kai_run_gdn_gemv_f32_f32_f32_1x4_neon(c->a, c->b, c->c, c->k, c->n); }

static int d_cumdecay(void *p) { sctx *c = p; return kai_run_gdn_cumdecay_f32_hip(c->a, c->d, c->T, c->C, NULL); }
static int d_scan(void *p) {
    sctx *c = p;
    return kai_run_gdn_gated_scan_f32_hip(c->a, c->x, c->s, c->st, c->T, c->C, NULL);
}
static int d_conv(void *p) {
    sctx *c = p;
    return kai_run_gdn_causal_dwconv1d_f32_k4_hip(c->x, c->w, c->s, c->h, c->T, c->C, NULL);
}
static int d_conv_silu(void *p) {
    sctx *c = p;
    return kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(c->x, c->w, c->s, c->h, c->T, c->C, NULL);
}
static int d_gemv(void *p) { gctx *c = p; return kai_run_gdn_gemv_f32_f32_f32_hip(c->a, c->b, c->c, c->k, c->n, NULL); }
static int d_decode(void *p) {
    dctx *c = p;
    return kai_run_gdn_delta_rule_decode_f32_hip(c->S, c->q, c->k, c->v, c->g, c->beta, c->o, c->B,
                                                 c->Hv, c->Hk, c->d, c->d, 0.08838835f, NULL);
}

static void host_shapes(int reps) {
    static const long shapes[][2] = {{64, 160}, {1, 160}, {64, 2560}, {1, 2560}};
    char lab[48];
    for (int si = 0; si < 4; ++si) {
        size_t T = (size_t)shapes[si][0], C = (size_t)shapes[si][1], n = T * C;
        sctx c = {0};
        c.T = T, c.C = C;
        c.a = xalloc(n * 4), c.d = xalloc(n * 4), c.x = xalloc(n * 4), c.s = xalloc(n * 4);
        c.st = xalloc(C * 4), c.w = xalloc(16 * C), c.h = xalloc(12 * C);
        memset(c.a, 0x3f, n * 4), memset(c.x, 0x3f, n * 4), memset(c.w, 0x3f, 16 * C);
        memset(c.st, 0, C * 4), memset(c.h, 0, 12 * C);
        snprintf(lab, sizeof lab, "%zux%zu", T, C);
        bench_host("cumdecay", lab, (long)T, (long)C, reps, h_cumdecay, &c, 2.0 * n * 4);
        bench_host("gated_scan", lab, (long)T, (long)C, reps, h_scan, &c, (3.0 * n + 2.0 * C) * 4);
        bench_host("dwconv1d", lab, (long)T, (long)C, reps, h_conv, &c, (2.0 * n + 4.0 * C + 6.0 * C) * 4);
        free(c.a), free(c.d), free(c.x), free(c.s), free(c.st), free(c.w), free(c.h);
    }
    static const long gs[][2] = {{128, 128}, {128, 2048}, {128, 2560}};
    for (int si = 0; si < 3; ++si) {
        gctx c = {xalloc(gs[si][0] * 4), xalloc(gs[si][0] * gs[si][1] * 4), xalloc(gs[si][1] * 4),
                  (size_t)gs[si][0], (size_t)gs[si][1]};
        memset(c.a, 0x3f, c.k * 4), memset(c.b, 0x3f, c.k * c.n * 4);
        snprintf(lab, sizeof lab, "K%ld_N%ld", gs[si][0], gs[si][1]);
        bench_host("gemv", lab, 0, gs[si][1], reps, h_gemv, &c,
                   ((double)c.k + (double)c.k * c.n + (double)c.n) * 4);
        free(c.a), free(c.b), free(c.c);
    }
}

static void dev_shapes(int reps) {
    static const long shapes[][2] = {{64, 160}, {1, 160}, {64, 2560}, {1, 2560}, {4096, 8192}};
    char lab[48];
    for (int si = 0; si < 5; ++si) {
        size_t T = (size_t)shapes[si][0], C = (size_t)shapes[si][1], n = T * C;
        sctx c = {0};
        c.T = T, c.C = C;
        c.a = dalloc(n * 4), c.d = dalloc(n * 4), c.x = dalloc(n * 4), c.s = dalloc(n * 4);
        c.st = dalloc(C * 4), c.w = dalloc(16 * C), c.h = dalloc(12 * C);
        snprintf(lab, sizeof lab, "%zux%zu", T, C);
        bench_dev("cumdecay_dev", lab, (long)T, (long)C, reps, d_cumdecay, &c, 2.0 * n * 4);
        bench_dev("gated_scan_dev", lab, (long)T, (long)C, reps, d_scan, &c, (3.0 * n + 2.0 * C) * 4);
        bench_dev("dwconv1d_dev", lab, (long)T, (long)C, reps, d_conv, &c, (2.0 * n + 4.0 * C + 6.0 * C) * 4);
        bench_dev("dwconv1d_silu_dev", lab, (long)T, (long)C, reps, d_conv_silu, &c,
                  (2.0 * n + 4.0 * C + 6.0 * C) * 4);
        hipFree(c.a), hipFree(c.d), hipFree(c.x), hipFree(c.s), hipFree(c.st), hipFree(c.w), hipFree(c.h);
    }
    static const long gs[][2] = {{128, 128}, {128, 2048}, {128, 2560}};
    for (int si = 0; si < 3; ++si) {
        gctx c = {dalloc(gs[si][0] * 4), dalloc(gs[si][0] * gs[si][1] * 4), dalloc(gs[si][1] * 4),
                  (size_t)gs[si][0], (size_t)gs[si][1]};
        snprintf(lab, sizeof lab, "K%ld_N%ld", gs[si][0], gs[si][1]);
        bench_dev("gemv_dev", lab, 0, gs[si][1], reps, d_gemv, &c,
                  ((double)c.k + (double)c.k * c.n + (double)c.n) * 4);
        hipFree(c.a), hipFree(c.b), hipFree(c.c);
    }
    /* decode step of one layer: B=64, 32 value heads, 16 key heads, 128x128 */
    dctx c = {0};
    c.B = 64, c.Hv = 32, c.Hk = 16, c.d = 128;
    size_t ns = (size_t)c.B * c.Hv * c.d * c.d;
    c.S = dalloc(ns * 4), c.q = dalloc((size_t)c.B * c.Hk * c.d * 4), c.k = dalloc((size_t)c.B * c.Hk * c.d * 4);
    c.v = dalloc((size_t)c.B * c.Hv * c.d * 4), c.o = dalloc((size_t)c.B * c.Hv * c.d * 4);
    c.g = dalloc((size_t)c.B * c.Hv * 4), c.beta = dalloc((size_t)c.B * c.Hv * 4);
    hipMemset(c.S, 0, ns * 4);
    hipMemset(c.g, 0, (size_t)c.B * c.Hv * 4);
    double bytes = 2.0 * ns * 4 + 2.0 * c.B * c.Hk * c.d * 4 + 2.0 * c.B * c.Hv * c.d * 4 + 2.0 * c.B * c.Hv * 4;
    bench_dev("delta_decode_dev", "B64_H32_128x128", 1, (long)c.B * c.Hv * c.d, reps, d_decode, &c, bytes);
    hipFree(c.S), hipFree(c.q), hipFree(c.k), hipFree(c.v), hipFree(c.o), hipFree(c.g), hipFree(c.beta);
}

int main(int argc, char **argv) {
    int reps = 30;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--repeats") && i + 1 < argc) reps = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--csv")) g_csv = 1;
    }
    if (reps < 1) reps = 1;
    if (kai_gdn_hip_init() != 0) {
        fprintf(stderr, "HIP initialisation failed\n");
        return 1;
    }
    if (!g_csv) {
        printf("GDN kai entry points on MI355X\n");
        printf("  repeats per shape : %d (after 20 warmups)\n\n", reps);
    } else {
        printf("kernel,shape,seq,channels,repeats,p50_us,gib_per_s_p50\n");
    }
    host_shapes(reps);
    dev_shapes(reps);
    if (kai_gdn_hip_check_device_error() != 0) {
        fprintf(stderr, "scan watchdog fired\n");
        return 1;
    }
    return 0;
}

/*
 * gdn_e2e_decode.c -- the end-to-end hybrid decode benchmark on MI355X,
 * driving include/kai_gdn_hybrid.h (Qwen3.5-4B shape, int8 weights).
 *
 * Keeps the interface of the reference program
 * (src/orionsbelt/engines/cpu/kernels/gdn_e2e_decode.c:1921-1974, output at
 * :2733-2860 and the context sweep at :2590-2620):
 *   --tokens N           decode N tokens per sequence (default 8)
 *   --csv                CSV instead of the text report
 *   --ctx-sweep L1,L2..  decode cost at growing context lengths
 *   --help
 * with the reference's CSV headers, so its parser (bench/convert_e2e_decode.py)
 * reads these rows.  The reference's per-phase timers (:1365-1371) are filled
 * from a separate timing pass after the measured one (the library's timing
 * mode, kai_gdn_hybrid_set_timing: HIP events between the kernel groups,
 * whose own cost would perturb the measured pass): GDN input projection,
 * GDN out projection, full attention and FFN as in the reference.  The
 * reference's conv1d, cumdecay and gated-scan phases are one fused kernel in
 * a GPU decode step; its time is reported as gdn_scan and the conv and decay
 * columns as 0.  Added:
 *   --prefill M          process M prompt tokens in one pass
 *                        (kai_gdn_hybrid_prefill) and report TTFT and prefill
 *                        throughput (:2644-2730: 2 warm-up passes, then one
 *                        measured; its CSV header with the GDN / full
 *                        attention / FFN split of a timing pass)
 *   --batch B            sequences decoded together (default 1, at most 16)
 *   --ctx L              a drawn context of L positions before the timed
 *                        tokens (KV caches, recurrent and conv states)
 * The reference's other flags (--pure-gdn, --verify-*, --naive) select CPU
 * code paths that do not exist here; they are reported and ignored.
 *
 * As in the reference: 3 warm-up tokens, then a reset and the measured
 * tokens, each timed on its own (HIP events around the step, synchronised),
 * TTFT = the first token's time, percentiles by sorted rank.  Tokens stay on
 * the device: each step's greedy argmax is the next step's input.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "kai_gdn_hybrid.h"

#define MODEL_NAME "Qwen3.5-4B"

#define HIP_OK(x)                                                                    \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                    __LINE__);                                                       \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)
#define KAI_OK(x)                                                                    \
    do {                                                                             \
        int r_ = (x);                                                                \
        if (r_ != 0) {                                                               \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString((hipError_t)r_)); \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)

static int cmp_double(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

typedef struct {
    kai_gdn_hybrid *m;
    int32_t *tok[2];
    int batch, vocab, which;
    hipStream_t st;
    hipEvent_t e0, e1;
} runner;

static void first_tokens(runner *r, uint32_t seed) {
    int32_t host[16];
    for (int b = 0; b < r->batch; ++b) {
        seed = seed * 1664525u + 1013904223u;
        host[b] = (int32_t)(seed % (uint32_t)r->vocab);
    }
    HIP_OK(hipMemcpy(r->tok[0], host, sizeof(int32_t) * (size_t)r->batch, hipMemcpyHostToDevice));
    r->which = 0;
}

/* `n` untimed steps with the library's timing mode on, from a fresh drawn
 * context; ph[] gets each phase's sum over them (microseconds). */
static void phase_pass(runner *r, int ctx, int n, double *ph) {
    KAI_OK(kai_gdn_hybrid_reset(r->m, r->batch, ctx, 7));
    first_tokens(r, 42u);
    KAI_OK(kai_gdn_hybrid_set_timing(r->m, 1));
    for (int t = 0; t < n; ++t) {
        KAI_OK(kai_gdn_hybrid_step(r->m, r->tok[r->which], r->tok[r->which ^ 1], NULL, r->st));
        r->which ^= 1;
    }
    KAI_OK(kai_gdn_hybrid_phase_times(r->m, ph, KAI_GDN_PHASE_COUNT));
    KAI_OK(kai_gdn_hybrid_set_timing(r->m, 0));
}

/* One step, timed on its own; returns microseconds. */
static double timed_step(runner *r) {
    HIP_OK(hipEventRecord(r->e0, r->st));
    KAI_OK(kai_gdn_hybrid_step(r->m, r->tok[r->which], r->tok[r->which ^ 1], NULL, r->st));
    HIP_OK(hipEventRecord(r->e1, r->st));
    HIP_OK(hipEventSynchronize(r->e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, r->e0, r->e1));
    r->which ^= 1;
    return ms * 1e3;
}

/* --prefill M: M uniform-random prompt tokens per sequence through every
 * layer in one pass; 2 warm-up passes, then the measured one (HIP events
 * around the call, synchronised). */
static int run_prefill(int M, int batch, int csv) {
    kai_gdn_hybrid_config cfg = kai_gdn_hybrid_qwen35_4b(batch, M + 1);
    kai_gdn_hybrid *m = NULL;
    KAI_OK(kai_gdn_hybrid_create(&cfg, 12345, &m));
    hipStream_t st;
    hipEvent_t e0, e1;
    HIP_OK(hipStreamCreate(&st));
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    const size_t n = (size_t)batch * (size_t)M;
    int32_t *host = malloc(sizeof(int32_t) * n), *tok = NULL, *next = NULL;
    if (!host) {
        fprintf(stderr, "Error: out of host memory\n");
        return 1;
    }
    uint32_t seed = 42u;
    for (size_t i = 0; i < n; ++i) {
        seed = seed * 1664525u + 1013904223u;
        host[i] = (int32_t)(seed % (uint32_t)cfg.vocab);
    }
    HIP_OK(hipMalloc((void **)&tok, sizeof(int32_t) * n));
    HIP_OK(hipMalloc((void **)&next, sizeof(int32_t) * 16));
    HIP_OK(hipMemcpy(tok, host, sizeof(int32_t) * n, hipMemcpyHostToDevice));
    if (!csv) {
        printf(MODEL_NAME " MI355X prefill benchmark (M=%d)\n", M);
        printf("  layers=%d (GDN=%d, full=%d), hidden=%d, int8 weights, batch=%d\n", cfg.layers,
               cfg.layers - cfg.layers / cfg.attn_every, cfg.layers / cfg.attn_every, cfg.hidden, batch);
        printf("  tokens/prefill=%d\n\n", M);
    }
    for (int r = 0; r < 2; ++r) KAI_OK(kai_gdn_hybrid_prefill(m, tok, batch, M, next, NULL, st));
    HIP_OK(hipStreamSynchronize(st));
    HIP_OK(hipEventRecord(e0, st));
    KAI_OK(kai_gdn_hybrid_prefill(m, tok, batch, M, next, NULL, st));
    HIP_OK(hipEventRecord(e1, st));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    const double total_us = ms * 1e3, ttft_ms = ms, tps = (double)n * 1e6 / total_us;
    /* the per-layer-type split, from a timing pass */
    double ph[KAI_GDN_PHASE_COUNT];
    KAI_OK(kai_gdn_hybrid_set_timing(m, 1));
    KAI_OK(kai_gdn_hybrid_prefill(m, tok, batch, M, next, NULL, st));
    KAI_OK(kai_gdn_hybrid_phase_times(m, ph, KAI_GDN_PHASE_COUNT));
    KAI_OK(kai_gdn_hybrid_set_timing(m, 0));
    const double gdn_us = ph[KAI_GDN_PHASE_GDN_PROJ] + ph[KAI_GDN_PHASE_GDN_CORE] + ph[KAI_GDN_PHASE_GDN_OPROJ];
    if (csv) {
        printf("model,prefill_M,ttft_ms,tok_per_sec_prefill,gdn_us,full_us,ffn_us\n");
        printf(MODEL_NAME ",%d,%.2f,%.2f,%.0f,%.0f,%.0f\n", M, ttft_ms, tps, gdn_us, ph[KAI_GDN_PHASE_ATTN],
               ph[KAI_GDN_PHASE_FFN]);
    } else {
        printf("Results (prefill M=%d, %d sequences):\n", M, batch);
        printf("  TTFT (prefill total):  %.2f ms  (%.0f us)\n", ttft_ms, total_us);
        printf("  Prefill throughput:    %.2f tok/s  (%.4f ms/tok)\n", tps, ttft_ms / (double)n);
        printf("  Layer types (timing pass): GDN %.0f us, full attention %.0f us, FFN %.0f us, other %.0f us\n",
               gdn_us, ph[KAI_GDN_PHASE_ATTN], ph[KAI_GDN_PHASE_FFN], ph[KAI_GDN_PHASE_OTHER]);
    }
    free(host);
    HIP_OK(hipFree(tok));
    HIP_OK(hipFree(next));
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    HIP_OK(hipStreamDestroy(st));
    kai_gdn_hybrid_destroy(m);
    return 0;
}

int main(int argc, char **argv) {
    int num_tokens = 8, csv = 0, batch = 1, ctx = 0, sweep = 0, prefill_m = 0;
    const char *ctx_lens_str = NULL;
    for (int i = 1; i < argc; ++i) {
        if (strcmp(argv[i], "--tokens") == 0 && i + 1 < argc)
            num_tokens = atoi(argv[++i]);
        else if (strcmp(argv[i], "--csv") == 0)
            csv = 1;
        else if (strcmp(argv[i], "--batch") == 0 && i + 1 < argc)
            batch = atoi(argv[++i]);
        else if (strcmp(argv[i], "--ctx") == 0 && i + 1 < argc)
            ctx = atoi(argv[++i]);
        else if (strcmp(argv[i], "--ctx-sweep") == 0) {
            sweep = 1;
            if (i + 1 < argc && argv[i + 1][0] != '-') ctx_lens_str = argv[++i];
        } else if (strcmp(argv[i], "--help") == 0) {
            printf("Usage: %s [OPTIONS]\n", argv[0]);
            printf("  --tokens N        Decode N tokens per sequence (default 8)\n");
            printf("  --csv             CSV output\n");
            printf("  --ctx-sweep L1,L2,...  Decode cost at growing context lengths\n");
            printf("  --batch B         Sequences decoded together (default 1, at most 16)\n");
            printf("  --ctx L           Drawn context of L positions before the timed tokens\n");
            printf("  --prefill M       Process M tokens in one pass (measures TTFT / prefill cost)\n");
            return 0;
        } else if (strcmp(argv[i], "--pure-gdn") == 0 || strcmp(argv[i], "--naive") == 0 ||
                   strncmp(argv[i], "--verify-", 9) == 0) {
            fprintf(stderr, "Warning: '%s' selects a CPU code path of the reference; ignored\n", argv[i]);
        } else if (strcmp(argv[i], "--prefill") == 0 && i + 1 < argc) {
            char *end = NULL;
            const long v = strtol(argv[++i], &end, 10);
            if (end == argv[i] || *end != '\0' || v < 1 || v > 16777215) {
                fprintf(stderr, "Error: --prefill must be an integer in 1..16777215 (got '%s')\n", argv[i]);
                return 1;
            }
            prefill_m = (int)v;
        } else {
            fprintf(stderr, "Warning: unrecognized argument '%s' (ignored)\n", argv[i]);
        }
    }
    if (num_tokens < 1) {
        fprintf(stderr, "Error: --tokens must be >= 1 (got %d)\n", num_tokens);
        return 1;
    }
    if (batch < 1 || batch > 16 || ctx < 0) {
        fprintf(stderr, "Error: --batch must be in 1..16 and --ctx >= 0\n");
        return 1;
    }
    if (prefill_m > 0) return run_prefill(prefill_m, batch, csv);
    /* context lengths of the sweep (default: the reference's list, :2447-2449) */
    int lens[64], nlens = 0;
    if (sweep) {
        const char *s = ctx_lens_str ? ctx_lens_str : "1,64,256,1024,4096";
        while (*s && nlens < 64) {
            lens[nlens++] = atoi(s);
            while (*s && *s != ',') ++s;
            if (*s == ',') ++s;
        }
    }
    int max_ctx = ctx;
    for (int i = 0; i < nlens; ++i)
        if (lens[i] > max_ctx) max_ctx = lens[i];
    const int reps = 8;
    kai_gdn_hybrid_config cfg =
        kai_gdn_hybrid_qwen35_4b(batch, max_ctx + (num_tokens > reps ? num_tokens : reps) + 4);
    runner r = {0};
    r.batch = batch;
    r.vocab = cfg.vocab;
    KAI_OK(kai_gdn_hybrid_create(&cfg, 12345, &r.m));
    HIP_OK(hipStreamCreate(&r.st));
    HIP_OK(hipEventCreate(&r.e0));
    HIP_OK(hipEventCreate(&r.e1));
    HIP_OK(hipMalloc((void **)&r.tok[0], sizeof(int32_t) * 16));
    HIP_OK(hipMalloc((void **)&r.tok[1], sizeof(int32_t) * 16));

    if (sweep) {
        if (csv) printf("model,ctx_len,gdn_layer_us,full_attn_us,ffn_us,total_us,tok_per_sec,kv_cache_mb\n");
        else printf(MODEL_NAME " MI355X decode cost vs context (batch %d)\n", batch);
        for (int i = 0; i < nlens; ++i) {
            KAI_OK(kai_gdn_hybrid_reset(r.m, batch, lens[i], 7));
            first_tokens(&r, 42u);
            for (int t = 0; t < 3; ++t) timed_step(&r);
            KAI_OK(kai_gdn_hybrid_reset(r.m, batch, lens[i], 7));
            double total = 0.0;
            for (int t = 0; t < reps; ++t) total += timed_step(&r);
            total /= reps;
            const double tps = batch * 1e6 / total;
            const double kv_mb = (double)(cfg.layers / cfg.attn_every) * batch * cfg.attn_kv_heads * lens[i] *
                                 256 * 2 * 2 / (1024.0 * 1024.0);
            double ph[KAI_GDN_PHASE_COUNT];
            phase_pass(&r, lens[i], reps, ph);
            const double gdn = (ph[KAI_GDN_PHASE_GDN_PROJ] + ph[KAI_GDN_PHASE_GDN_CORE] +
                                ph[KAI_GDN_PHASE_GDN_OPROJ]) / reps;
            const double full = ph[KAI_GDN_PHASE_ATTN] / reps, ffn = ph[KAI_GDN_PHASE_FFN] / reps;
            if (csv)
                printf(MODEL_NAME ",%d,%.0f,%.0f,%.0f,%.0f,%.2f,%.1f\n", lens[i], gdn, full, ffn, total, tps, kv_mb);
            else
                printf("  ctx=%5d  GDN=%7.0f us  full_attn=%7.0f us  FFN=%7.0f us  total=%7.0f us  %.2f tok/s"
                       "  KV=%7.1f MB\n", lens[i], gdn, full, ffn, total, tps, kv_mb);
        }
    } else {
        if (!csv) {
            printf(MODEL_NAME " MI355X decode benchmark\n");
            printf("  layers=%d (GDN=%d, full=%d), hidden=%d, int8 weights, batch=%d, context=%d\n", cfg.layers,
                   cfg.layers - cfg.layers / cfg.attn_every, cfg.layers / cfg.attn_every, cfg.hidden, batch, ctx);
            printf("  tokens=%d\n\n", num_tokens);
        }
        KAI_OK(kai_gdn_hybrid_reset(r.m, batch, ctx, 7));
        first_tokens(&r, 42u);
        for (int t = 0; t < 3; ++t) timed_step(&r); /* warm-up */
        KAI_OK(kai_gdn_hybrid_reset(r.m, batch, ctx, 7));
        first_tokens(&r, 42u);
        double *tok_times = malloc(sizeof(double) * (size_t)num_tokens);
        double total_us = 0.0;
        for (int t = 0; t < num_tokens; ++t) {
            tok_times[t] = timed_step(&r);
            total_us += tok_times[t];
        }
        const double ttft_ms = tok_times[0] / 1e3, mean_us = total_us / num_tokens;
        qsort(tok_times, (size_t)num_tokens, sizeof(double), cmp_double);
        const double p50 = tok_times[num_tokens / 2], p95 = tok_times[(int)(num_tokens * 0.95)],
                     p99 = tok_times[(int)(num_tokens * 0.99)];
        const double tok_per_sec = batch * 1e6 / mean_us;
        /* the reference's bottleneck breakdown (:2820-2857), from a timing
         * pass: conv1d, cumdecay and the scan are one fused kernel here
         * (reported as the scan; conv and decay 0) */
        double ph[KAI_GDN_PHASE_COUNT];
        phase_pass(&r, ctx, num_tokens, ph);
        const double t_proj = ph[KAI_GDN_PHASE_GDN_PROJ], t_scan = ph[KAI_GDN_PHASE_GDN_CORE],
                     t_oproj = ph[KAI_GDN_PHASE_GDN_OPROJ], t_full = ph[KAI_GDN_PHASE_ATTN],
                     t_ffn = ph[KAI_GDN_PHASE_FFN];
        const double phase_sum = t_proj + t_scan + t_oproj + t_full + t_ffn;
        if (csv) {
            printf("model,tokens,ttft_ms,tok_per_sec_mean,p50_us,p95_us,p99_us,mean_us,"
                   "gdn_proj_pct,gdn_conv_pct,gdn_decay_pct,gdn_scan_pct,gdn_oproj_pct,full_pct,ffn_pct\n");
            printf(MODEL_NAME ",%d,%.2f,%.2f,%.0f,%.0f,%.0f,%.0f,%.1f,%.1f,%.1f,%.1f,%.1f,%.1f,%.1f\n", num_tokens,
                   ttft_ms, tok_per_sec, p50, p95, p99, mean_us, 100.0 * t_proj / phase_sum, 0.0, 0.0,
                   100.0 * t_scan / phase_sum, 100.0 * t_oproj / phase_sum, 100.0 * t_full / phase_sum,
                   100.0 * t_ffn / phase_sum);
        } else {
            printf("Results (%d tokens x %d sequences):\n", num_tokens, batch);
            printf("  TTFT (first token):  %.2f ms\n", ttft_ms);
            printf("  Tokens/sec (mean):   %.2f\n", tok_per_sec);
            printf("  Per-token latency:\n");
            printf("    p50:  %.0f us  (%.2f ms)\n", p50, p50 / 1e3);
            printf("    p95:  %.0f us  (%.2f ms)\n", p95, p95 / 1e3);
            printf("    p99:  %.0f us  (%.2f ms)\n", p99, p99 / 1e3);
            printf("    mean: %.0f us  (%.2f ms)\n", mean_us, mean_us / 1e3);
            printf("  Total decode time:   %.2f s\n", total_us / 1e6);
            printf("  Bottleneck breakdown (timing pass, share of the summed phases):\n");
            printf("    GDN q/k/v proj:  %5.1f%%  (%.0f us/tok)\n", 100.0 * t_proj / phase_sum, t_proj / num_tokens);
            printf("    GDN conv1d + cumdecay + gated_scan (one fused kernel): %5.1f%%  (%.0f us/tok)\n",
                   100.0 * t_scan / phase_sum, t_scan / num_tokens);
            printf("    GDN out proj:    %5.1f%%  (%.0f us/tok)\n", 100.0 * t_oproj / phase_sum,
                   t_oproj / num_tokens);
            printf("    Full-attention:  %5.1f%%  (%.0f us/tok)\n", 100.0 * t_full / phase_sum, t_full / num_tokens);
            printf("    FFN:             %5.1f%%  (%.0f us/tok)\n", 100.0 * t_ffn / phase_sum, t_ffn / num_tokens);
        }
        free(tok_times);
    }
    HIP_OK(hipFree(r.tok[0]));
    HIP_OK(hipFree(r.tok[1]));
    HIP_OK(hipEventDestroy(r.e0));
    HIP_OK(hipEventDestroy(r.e1));
    HIP_OK(hipStreamDestroy(r.st));
    kai_gdn_hybrid_destroy(r.m);
    return 0;
}

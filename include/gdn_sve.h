/*
 * gdn_sve.h -- the reference's internal gdn_* ABI for the diagonal GDN
 * kernels (src/orionsbelt/engines/cpu/kernels/gdn_sve.h:30-86), served by
 * libkai_gdn_hip.so on gfx950.
 *
 * Same names, argument order and meaning as the reference, so its callers
 * (bench_gdn.c, test_gdn_sve.c, test_gdn_mixed.c, test_gdn2_scan.c) compile
 * against this header and link the HIP library unchanged.  Like the kai
 * drop-in symbols: synchronous; each pointer may be host or device memory
 * (device pointers are used in place, host buffers are copied through the
 * library's device staging buffers); seq == 0 or channels == 0 writes
 * nothing; a HIP failure prints the failing call and exits(1).
 *
 * fp16 arrays are IEEE binary16 storage: __fp16 where the compiler has it
 * (clang, Arm), else uint16_t -- the same pointer ABI.  bf16 arrays are
 * uint16_t, the upper half of a binary32, rounded to nearest even by the
 * reference's rule (gdn_sve.c:81-87).
 */
#ifndef GDN_SVE_H
#define GDN_SVE_H

#include <stddef.h>
#include <stdint.h>

#if defined(__clang__) || defined(__ARM_FP16_FORMAT_IEEE)
#define GDN_SVE_F16 __fp16
#else
#define GDN_SVE_F16 uint16_t
#endif

#ifdef __cplusplus
#define GDN_SVE_RESTRICT __restrict__
extern "C" {
#else
#define GDN_SVE_RESTRICT restrict
#endif

/* decay[t][c] = prod_{i<=t} a[i][c]; a, decay [seq][channels]
 * (gdn_sve.h:30-31; the kai symbol kai_run_gdn_cumdecay_f32_sve). */
void gdn_cumdecay_f32(const float *GDN_SVE_RESTRICT a, float *GDN_SVE_RESTRICT decay,
                      size_t seq, size_t channels);

/* s[t][c] = g[t][c] * s[t-1][c] + x[t][c], state[] carried across calls
 * (gdn_sve.h:36-38). */
void gdn_gated_scan_f32(const float *GDN_SVE_RESTRICT g, const float *GDN_SVE_RESTRICT x,
                        float *GDN_SVE_RESTRICT s, float *GDN_SVE_RESTRICT state,
                        size_t seq, size_t channels);

/* out[t][c] = sum_{j<4} w[j][c] * in[t-3+j][c], hist [3][channels] carried
 * (gdn_sve.h:44-46). */
void gdn_causal_dwconv1d_f32(const float *GDN_SVE_RESTRICT in, const float *GDN_SVE_RESTRICT w,
                             float *GDN_SVE_RESTRICT out, float *GDN_SVE_RESTRICT hist,
                             size_t seq, size_t channels);

/* Mixed precision: fp32 accumulation, narrow storage (gdn_sve.h:57-72). */
void gdn_cumdecay_f16(const float *GDN_SVE_RESTRICT a, GDN_SVE_F16 *GDN_SVE_RESTRICT decay,
                      size_t seq, size_t channels);
void gdn_gated_scan_f16(const float *GDN_SVE_RESTRICT g, const float *GDN_SVE_RESTRICT x,
                        float *GDN_SVE_RESTRICT s, GDN_SVE_F16 *GDN_SVE_RESTRICT state,
                        size_t seq, size_t channels);
void gdn_cumdecay_bf16(const float *GDN_SVE_RESTRICT a, uint16_t *GDN_SVE_RESTRICT decay,
                       size_t seq, size_t channels);
void gdn_gated_scan_bf16(const float *GDN_SVE_RESTRICT g, const float *GDN_SVE_RESTRICT x,
                         float *GDN_SVE_RESTRICT s, uint16_t *GDN_SVE_RESTRICT state,
                         size_t seq, size_t channels);

/* GDN-2 decoupled-gating scan (gdn_sve.h:83-86):
 *   s[t][c] = w[t][c] * x[t][c] + s[t-1][c] * (g[t][c] * b[t][c])
 * with both products rounded before the sum, as the reference's portable
 * branch computes it (gdn_sve.c:861-874); state[] carried across calls. */
void gdn2_gated_scan_f32(const float *GDN_SVE_RESTRICT g, const float *GDN_SVE_RESTRICT b_gate,
                         const float *GDN_SVE_RESTRICT w_gate, const float *GDN_SVE_RESTRICT x,
                         float *GDN_SVE_RESTRICT s, float *GDN_SVE_RESTRICT state,
                         size_t seq, size_t channels);

#ifdef __cplusplus
}
#endif
#endif /* GDN_SVE_H */

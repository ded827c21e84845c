/*
 * GEMV (M = 1) -- drop-in declaration for the MI355X build.
 *
 * Same symbol, prototype and semantics as the reference kai ukernel
 * (kleidiai_submission/kai/ukernels/gdn/kai_gdn_gemv_f32_f32_f32_1x4_neon.h:40-42):
 *     c[j] = sum_{kk<k} a[kk] * b[kk][j],   j < n
 * b is [k][n] row-major fp32; k == 0 writes zeros, n == 0 writes nothing.
 * Implemented by libkai_gdn_hip.so (host or device pointers; synchronous).
 */
#ifndef KAI_GDN_GEMV_F32_F32_F32_1X4_NEON_H
#define KAI_GDN_GEMV_F32_F32_F32_1X4_NEON_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void kai_run_gdn_gemv_f32_f32_f32_1x4_neon(const float *a, const float *b,
                                            float *c, size_t k, size_t n);

#ifdef __cplusplus
}
#endif

#endif

/*
 * Diagonal gated scan -- drop-in declaration for the MI355X build.
 *
 * Same symbol, prototype and semantics as the reference kai ukernel
 * (kleidiai_submission/kai/ukernels/gdn/kai_gdn_gated_scan_f32_sve.h:35-36):
 *     s[t][c] = g[t][c] * s[t-1][c] + x[t][c],   s[-1][c] = state[c]
 * and state[c] = s[seq-1][c] on return.  g, x, s are [seq][channels]
 * row-major fp32.  Implemented by libkai_gdn_hip.so (host or device
 * pointers; synchronous).  seq == 0 or channels == 0 leaves state untouched.
 */
#ifndef KAI_GDN_GATED_SCAN_F32_SVE_H
#define KAI_GDN_GATED_SCAN_F32_SVE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void kai_run_gdn_gated_scan_f32_sve(const float *g, const float *x, float *s,
                                    float *state, size_t seq, size_t channels);

#ifdef __cplusplus
}
#endif

#endif

/*
 * Gated cumulative decay -- drop-in declaration for the MI355X build.
 *
 * Same symbol, prototype and semantics as the reference kai ukernel
 * (kleidiai_submission/kai/ukernels/gdn/kai_gdn_cumdecay_f32_sve.h:33-34):
 *     decay[t][c] = a[0][c] * a[1][c] * ... * a[t][c]
 * a and decay are [seq][channels] row-major fp32.  Here the symbol is
 * implemented by libkai_gdn_hip.so on a gfx950 GPU; pointers may be host
 * (copied in and out, synchronous) or device memory (run in place).
 * seq == 0 or channels == 0 writes nothing.  A HIP failure prints a message
 * and exits(1), the reference's convention for fatal errors.
 */
#ifndef KAI_GDN_CUMDECAY_F32_SVE_H
#define KAI_GDN_CUMDECAY_F32_SVE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void kai_run_gdn_cumdecay_f32_sve(const float *a, float *decay, size_t seq,
                                  size_t channels);

#ifdef __cplusplus
}
#endif

#endif

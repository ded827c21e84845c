/*
 * Causal depthwise Conv1D, kernel width 4 -- drop-in declaration for the
 * MI355X build.
 *
 * Same symbol, prototype and semantics as the reference kai ukernel
 * (kleidiai_submission/kai/ukernels/gdn/kai_gdn_causal_dwconv1d_f32_k4_sve.h:39-41):
 *     out[t][c] = w[0][c]*h0 + w[1][c]*h1 + w[2][c]*h2 + w[3][c]*in[t][c]
 * with h0 the oldest of the three previous inputs of channel c.  hist is
 * [3][channels] (oldest row first), read on entry and replaced by the last
 * three inputs on return.  in/out are [seq][channels], w is [4][channels].
 * Implemented by libkai_gdn_hip.so (host or device pointers; synchronous).
 */
#ifndef KAI_GDN_CAUSAL_DWCONV1D_F32_K4_SVE_H
#define KAI_GDN_CAUSAL_DWCONV1D_F32_K4_SVE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void kai_run_gdn_causal_dwconv1d_f32_k4_sve(const float *in, const float *w,
                                            float *out, float *hist, size_t seq,
                                            size_t channels);

#ifdef __cplusplus
}
#endif

#endif

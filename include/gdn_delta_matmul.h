/*
 * gdn_delta_matmul.h -- the reference's delta-rule matmul C = A . B
 * (src/orionsbelt/engines/cpu/kernels/gdn_delta_matmul.h:15-16), served by
 * libkai_gdn_hip.so on gfx950.
 *
 * Same name, argument order and meaning as the reference, so its callers
 * (test_gdn_delta_matmul.c, bench/bench_delta_matmul.c) compile against this
 * header and link the HIP library unchanged.  A is row-major [M][K], B
 * row-major [K][N], C row-major [M][N]; no bias, no clamp.  Like the kai
 * drop-in symbols: synchronous; each pointer may be host or device memory
 * (device pointers are used in place, host buffers are copied through the
 * library's device staging buffers); M == 0 or N == 0 writes nothing, K == 0
 * writes zeros; a HIP failure prints the failing call and exits(1).
 *
 * Each C[i][j] is the k-ordered fp32 sum of A[i][k] * B[k][j], each product
 * rounded before it is added (the reference test's naive loop,
 * test_gdn_delta_matmul.c:32-41).
 */
#ifndef GDN_DELTA_MATMUL_H
#define GDN_DELTA_MATMUL_H

#include <stddef.h>

#ifdef __cplusplus
#define GDN_DM_RESTRICT __restrict__
extern "C" {
#else
#define GDN_DM_RESTRICT restrict
#endif

/* C = A @ B (gdn_delta_matmul.h:15-16). */
void gdn_delta_rule_matmul(const float *GDN_DM_RESTRICT A, const float *GDN_DM_RESTRICT B,
                           float *GDN_DM_RESTRICT C, size_t M, size_t K, size_t N);

#ifdef __cplusplus
}
#endif

#endif /* GDN_DELTA_MATMUL_H */

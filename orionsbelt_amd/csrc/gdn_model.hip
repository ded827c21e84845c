// gdn_model.hip -- the matmuls of the hybrid decode loop for gfx950: int8
// weight-only GEMM (fp16 activations, per-output-channel symmetric scales)
// and the weight quantiser.
//
// Weights are stored output-major, Wq[N][K] int8 with scale[N] fp32 (the
// reference quantises per output column, gdn_e2e_decode.c:175-199; its
// [K][N] layout is transposed here so that the 8 k-values an MFMA lane
// needs are 8 contiguous bytes).  y[m][n] = scale[n] sum_k x[m][k] Wq[n][k],
// m < M <= 16 (the decode batch).
//
// One wave computes a 16-channel x 16-row tile on fp16 MFMA 16x16x32: A =
// 16 weight rows (int8 -> fp16 exactly: the byte u = q + 128 placed under
// the fp16 exponent of 1024 reads as 1024 + u, minus 1152 is q), B = the
// activation rows.  Per 64-k step a lane loads 16 weight bytes (one
// 16-byte load; the four lane groups cover 64 contiguous bytes of a row)
// and 32 activation bytes.  The four waves of a block split the block's
// k-range and reduce through LDS; narrow layers (few 16-channel tiles) also
// split k across blocks, into a partial-sum workspace that a second kernel
// reduces in a fixed order (deterministic).  The layer is HBM-bound on the
// weight bytes at decode sizes; the activations are L2-resident.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kW8Threads = 256;  // four waves
constexpr int kKStep = 64;       // k per wave iteration (two MFMAs)

GDN_DEV f32x4_t mfma_f16(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Four int8 (one dword) -> four fp16, exactly.
GDN_DEV void i8x4_to_f16(uint32_t w, f16x2_t &lo, f16x2_t &hi) {
    const uint32_t t = w ^ 0x80808080u;  // u = q + 128 per byte
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u);  // [u0, 0x64, u1, 0x64]
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u);  // [u2, 0x64, u3, 0x64]
    const f16x2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(f16x2_t, a) - bias;
    hi = __builtin_bit_cast(f16x2_t, b) - bias;
}
// 16 int8 -> two MFMA operands of 8 fp16 (k = 0..7 and 8..15 of the 16).
GDN_DEV void i8x16_to_f16(const u32x4_t &w, f16x8_t &k0, f16x8_t &k1) {
    f16x2_t p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) i8x4_to_f16(w[i], p[2 * i], p[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k0[2 * i] = p[i][0];
        k0[2 * i + 1] = p[i][1];
        k1[2 * i] = p[4 + i][0];
        k1[2 * i + 1] = p[4 + i][1];
    }
}

// Block (tile t = blockIdx.x, split s = blockIdx.y): channels 16t .. 16t+15,
// k in [s * kblk, (s + 1) * kblk), wave w taking the w-th quarter.
// Output: S == 1: y[m][n] fp32, scaled; S > 1: part[s][m][n], unscaled.
__global__ __launch_bounds__(kW8Threads) void w8_gemm_kernel(const uint16_t *__restrict__ x,
                                                             const int8_t *__restrict__ W,
                                                             const float *__restrict__ scale,
                                                             float *__restrict__ out, int M, int N,
                                                             int K, int kblk, int S) {
    __shared__ f32x4_t red[3][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int n0 = 16 * blockIdx.x;
    const int kq = kblk / 4;  // multiple of kKStep
    const int kb = blockIdx.y * kblk + wave * kq;
    const int8_t *wp = W + (size_t)(n0 + r) * K + kb + 16 * g;
    const bool row_ok = r < M;
    const uint16_t *xp = x + (size_t)(row_ok ? r : 0) * K + kb + 16 * g;
    f32x4_t acc = zero4();
#pragma unroll 4
    for (int k = 0; k < kq; k += kKStep) {
        const u32x4_t wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(wp + k));
        u32x4_t xa = *reinterpret_cast<const u32x4_t *>(xp + k);
        u32x4_t xb = *reinterpret_cast<const u32x4_t *>(xp + k + 8);
        if (!row_ok) xa = xb = u32x4_t{0u, 0u, 0u, 0u};
        f16x8_t w0, w1;
        i8x16_to_f16(wv, w0, w1);
        acc = mfma_f16(w0, __builtin_bit_cast(f16x8_t, xa), acc);
        acc = mfma_f16(w1, __builtin_bit_cast(f16x8_t, xb), acc);
    }
    // C lane (g, r): C[4g + e][r] = sum over this wave's k of W[n0+4g+e] . x[r]
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int i = 0; i < 3; ++i) acc += red[i][lane];
    if (r >= M) return;
    const int n = n0 + 4 * g;
    if (S == 1) {
        const f32x4_t sc = *reinterpret_cast<const f32x4_t *>(scale + n);
        *reinterpret_cast<f32x4_t *>(out + (size_t)r * N + n) = acc * sc;
    } else {
        *reinterpret_cast<f32x4_t *>(out + ((size_t)blockIdx.y * M + r) * N + n) = acc;
    }
}

// y[m][n] = scale[n] * sum_{s < S} part[s][m][n], the splits in order.
__global__ __launch_bounds__(256) void w8_reduce_kernel(const float *__restrict__ part,
                                                        const float *__restrict__ scale,
                                                        float *__restrict__ y, int M, int N, int S) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * N) return;
    float s = 0.f;
    for (int j = 0; j < S; ++j) s += part[(size_t)j * M * N + i];
    y[i] = s * scale[i % N];
}

// Per-output-channel symmetric quantisation of W[N][K] fp32 (the
// reference's quantize_weight, gdn_e2e_decode.c:175-199, on rows instead of
// columns): scale = max|w| / 127 (1 for an all-zero row), q =
// clamp(round_half_away(w * (1 / scale)), -128, 127).  One block per row.
__global__ __launch_bounds__(256) void w8_quantize_kernel(const float *__restrict__ W,
                                                          int8_t *__restrict__ Wq,
                                                          float *__restrict__ scale, int K) {
    __shared__ float wmax[4];
    const size_t n = blockIdx.x;
    const float *row = W + n * K;
    float m = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(row[k]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float s = m > 0.f ? m / 127.0f : 1.0f;
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) scale[n] = s;
    for (int k = threadIdx.x; k < K; k += 256) {
        float v = roundf(row[k] * inv);
        v = fminf(fmaxf(v, -128.f), 127.f);
        Wq[n * K + k] = (int8_t)(int)v;
    }
}

}  // namespace

int w8_splits(int N, int K) {
    const int tiles = N / 16;
    int S = 1;
    // enough blocks to fill 256 CUs several times over; each block keeps at
    // least 4 x 256 k
    while (tiles * S < 1024 && K % (4 * kKStep * S * 2) == 0 && K / (S * 2) >= 1024) S *= 2;
    return S;
}

size_t w8_workspace_bytes(int M, int N, int K) {
    const int S = w8_splits(N, K);
    return S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
}

hipError_t launch_w8_gemm(const uint16_t *x, const int8_t *W, const float *scale, float *y, int M,
                          int N, int K, float *workspace, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const int S = w8_splits(N, K);
    const int kblk = K / S;
    float *out = S > 1 ? workspace : y;
    if (S > 1 && !workspace) return hipErrorInvalidValue;
    w8_gemm_kernel<<<dim3(N / 16, S), kW8Threads, 0, st>>>(x, W, scale, out, M, N, K, kblk, S);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const size_t n = (size_t)M * N;
    w8_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(workspace, scale, y, M, N, S);
    return hipGetLastError();
}

hipError_t launch_w8_quantize(const float *W, int8_t *Wq, float *scale, int N, int K, hipStream_t st) {
    if (N == 0 || K == 0) return hipSuccess;
    w8_quantize_kernel<<<N, 256, 0, st>>>(W, Wq, scale, K);
    return hipGetLastError();
}

}  // namespace gdn

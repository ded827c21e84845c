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

constexpr int kW8Threads = 256;  // four waves
constexpr int kKStep = 64;       // k per wave iteration (two MFMAs)

GDN_DEV f32x4_t mfma_f16(f16x8_t a, f16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
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


// ---------------------------------------------------------------------------
// The model's int8 GEMM: the matmuls of one layer that read the same input
// are one weight matrix (their rows concatenated), one launch.
//
// Weights are pre-tiled (w8f_tile_kernel) so that every wave load is one
// contiguous 1 KB: for channel group c (64 channels, four 16-channel MFMA
// tiles) and 64-k step s, the 4 KB at ((c * K / 64) + s) * 4096 hold tile
// j's 1 KB at j * 1024, lane (g, r)'s 16 bytes at (16 g + r) * 16 = row
// 64 c + 16 j + r, k = 64 s + 16 g .. +15.
//
// Block (group c = blockIdx.x, split s = blockIdx.y) takes k in [s kblk,
// (s + 1) kblk); its WAVES waves split that range, each streaming its steps
// with DEPTH steps of loads in flight; one activation load feeds the four
// tiles.  The waves reduce through LDS, wave j finishing tile j.  With S > 1
// splits, each block stores its partial (agent-scope, written through) and
// the last of the group's S blocks to arrive (counter cnt[c], returned to
// 0) sums the S partials in split order -- the result does not depend on
// which block is last -- and runs the epilogue:
//   kW8Segments: y = acc * scale into up to four output arrays, channel
//                ranges of 16-multiples, each with its own row stride;
//   kW8SwiGLU:   the rows are gate/up interleaved in groups of 8 (tile rows
//                0..7 gate channels 8t..8t+7, rows 8..15 the up channels),
//                out16[m][c] = fp16(silu(gate) * up) (Qwen3_5MLP,
//                modeling_qwen3_5.py:704-717).
// With W8Out::nin_h set, the input is formed in each block instead of read:
// the decoder layer's "h = h + branch; x = norm(h)" (Qwen3_5RMSNorm, weight
// 1 + w) ahead of the matrix that reads x, without a launch of its own.
// ---------------------------------------------------------------------------
namespace {

constexpr int kW8fGroup = 64;  // channels per block
constexpr int kBufFlags = 0x00020000;  // buffer descriptor word 3 (raw dword access)
constexpr int kSc1 = 16;               // cache policy: agent-coherent (sc1)

// row-major Wq [N][K] -> the tiled layout above; one thread per 16 bytes
__global__ __launch_bounds__(256) void w8f_tile_kernel(const int8_t *__restrict__ src, int8_t *__restrict__ dst,
                                                       int K, size_t chunks) {
    const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= chunks) return;
    const int lane = (int)(q & 63), j = (int)((q >> 6) & 3);
    const size_t cs = q >> 8;  // c * (K / 64) + s
    const int steps = K / 64;
    const size_t c = cs / steps, s = cs % steps;
    const size_t n = 64 * c + 16 * j + (lane & 15);
    const size_t k = 64 * s + 16 * (lane >> 4);
    *reinterpret_cast<uint4 *>(dst + q * 16) = *reinterpret_cast<const uint4 *>(src + n * K + k);
}

// The normalised input of a block (W8Out::nin_*), threads 0..255 with the
// arithmetic of the hybrid model's addnorm kernel (the same per-thread
// chunks and wave-sum pairing, so the rows are bit-identical): xs[b][k] = fp16(h'[b][k] * inv * (1 + w[k])), h' = h + add;
// `writer` stores h'.  Every thread of the block calls it (barriers).
__device__ void w8f_norm_input(const W8Out &out, int M, int K, uint16_t *xs, float *s_ss, bool writer) {
    const int n4 = K / 4, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int b = 0; b < M; ++b) {
        f32x4_t x[4];
        float ss = 0.f;
        if (tid < 256) {
            const float4 *hr = reinterpret_cast<const float4 *>(out.nin_h + (size_t)b * K);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = tid + 256 * j;
                if (i < n4) {
                    const float4 hv = hr[i];
                    x[j] = f32x4_t{hv.x, hv.y, hv.z, hv.w};
                    if (out.nin_add) {
                        const float4 dv = reinterpret_cast<const float4 *>(out.nin_add + (size_t)b * K)[i];
                        x[j] += f32x4_t{dv.x, dv.y, dv.z, dv.w};
                        if (writer)
                            reinterpret_cast<float4 *>(out.nin_hout + (size_t)b * K)[i] =
                                make_float4(x[j][0], x[j][1], x[j][2], x[j][3]);
                    }
                    ss += x[j][0] * x[j][0] + x[j][1] * x[j][1] + x[j][2] * x[j][2] + x[j][3] * x[j][3];
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if (lane == 0) s_ss[wave] = ss;
        }
        __syncthreads();
        const float inv = 1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)K + out.nin_eps);
        __syncthreads();  // s_ss is rewritten by the next row
        if (tid < 256) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = tid + 256 * j;
                if (i < n4) {
                    const float4 wv = reinterpret_cast<const float4 *>(out.nin_w)[i];
                    uint2 o;
                    o.x = (uint32_t)f32_to_f16_rne(x[j][0] * inv * (1.0f + wv.x)) |
                          ((uint32_t)f32_to_f16_rne(x[j][1] * inv * (1.0f + wv.y)) << 16);
                    o.y = (uint32_t)f32_to_f16_rne(x[j][2] * inv * (1.0f + wv.z)) |
                          ((uint32_t)f32_to_f16_rne(x[j][3] * inv * (1.0f + wv.w)) << 16);
                    *reinterpret_cast<uint2 *>(&xs[(size_t)b * K + 4 * i]) = o;
                }
            }
        }
    }
    __syncthreads();
}

template <int WAVES, int DEPTH, bool NORM_IN = false>
__global__ __launch_bounds__(64 * WAVES) void w8f_kernel(const uint16_t *__restrict__ x,
                                                         const int8_t *__restrict__ W,
                                                         const float *__restrict__ scale, int M, int N, int K,
                                                         int kblk, int S, float *__restrict__ part,
                                                         uint32_t *__restrict__ cnt, W8Out out) {
    __shared__ f32x4_t red[WAVES][4][64];
    __shared__ float s_ss[4];
    __shared__ bool last;
    extern __shared__ __align__(16) uint16_t xs[];  // NORM_IN: the normalised rows [M][K] (dynamic)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int c = blockIdx.x;
    const int n0 = kW8fGroup * c;
    const int kq = kblk / WAVES;      // this wave's k-range
    const int nsteps = kq / kKStep;   // a multiple of DEPTH
    const int kb = blockIdx.y * kblk + wave * kq;
    const int8_t *wp = W + ((size_t)c * (K / kKStep) + kb / kKStep) * 4096 + lane * 16;
    const bool row_ok = r < M;
    // rows past M read row 0 (in bounds, one cache line per wave) and are zeroed
    const uint16_t *xp = NORM_IN ? &xs[(size_t)(row_ok ? r : 0) * K + kb + 16 * g]
                                 : x + (size_t)(row_ok ? r : 0) * K + kb + 16 * g;
    f32x4_t acc[4] = {zero4(), zero4(), zero4(), zero4()};
    u32x4_t buf[DEPTH][4];
    auto load_w = [&](u32x4_t (&w)[4], int st) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(wp + (size_t)st * 4096 + j * 1024));
    };
    auto mult = [&](const u32x4_t (&w)[4], int st) {
        u32x4_t xa = *reinterpret_cast<const u32x4_t *>(xp + st * kKStep);
        u32x4_t xb = *reinterpret_cast<const u32x4_t *>(xp + st * kKStep + 8);
        if (!row_ok) xa = xb = u32x4_t{0u, 0u, 0u, 0u};
        const f16x8_t fa = __builtin_bit_cast(f16x8_t, xa), fb = __builtin_bit_cast(f16x8_t, xb);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f16x8_t w0, w1;
            i8x16_to_f16(w[j], w0, w1);
            acc[j] = mfma_f16(w0, fa, acc[j]);
            acc[j] = mfma_f16(w1, fb, acc[j]);
        }
    };
    // DEPTH steps in flight: step st + DEPTH is requested as step st is used
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) load_w(buf[i], i);
    // the normalised input forms while the first weight steps are in flight
    if constexpr (NORM_IN) w8f_norm_input(out, M, K, xs, s_ss, blockIdx.x == 0 && blockIdx.y == 0);
    int base = 0;
    for (; base + DEPTH < nsteps; base += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            mult(buf[i], base + i);
            load_w(buf[i], base + DEPTH + i);
        }
    }
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) mult(buf[i], base + i);
    // reduce over the waves; wave j (< 4) ends with tile j of the block
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave >= 4) return;
    const int j = wave;
    f32x4_t t = red[0][j][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) t += red[w][j][lane];
    const int n = n0 + 16 * j + 4 * g;  // C lane (g, r): channels n .. n+3 of batch row r
    if (S > 1) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(part, 0, 0x7FFFFFFF, kBufFlags);
        const int row_stride = N * 4;
        if (row_ok)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, t), rs,
                                                   ((blockIdx.y * M + r) * row_stride) + n * 4, 0, kSc1);
        stores_done();
        __syncthreads();
        if (threadIdx.x == 0) last = arrive_last(&cnt[c], (uint32_t)S);
        __syncthreads();
        if (!last) return;
        t = zero4();
        if (row_ok) {
            // every split's partial requested before any is summed
            constexpr int kBatch = 8;
            for (int s0 = 0; s0 < S; s0 += kBatch) {
                u32x4_t v[kBatch];
#pragma unroll
                for (int q = 0; q < kBatch; ++q)
                    if (s0 + q < S)
                        v[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, (((s0 + q) * M + r) * row_stride) + n * 4, 0,
                                                                     kSc1);
#pragma unroll
                for (int q = 0; q < kBatch; ++q)
                    if (s0 + q < S) t += __builtin_bit_cast(f32x4_t, v[q]);
            }
        }
    }
    // epilogue (wave j, tile j)
    f32x4_t y = t * *reinterpret_cast<const f32x4_t *>(scale + n);
    if (out.mode == kW8SwiGLU) {
        f32x4_t up;
#pragma unroll
        for (int e = 0; e < 4; ++e) up[e] = __shfl_xor(y[e], 32);
        if (g < 2 && row_ok) {
            uint32_t h[2];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float a = y[e] / (1.0f + expf(-y[e])) * up[e];
                const float b = y[e + 1] / (1.0f + expf(-y[e + 1])) * up[e + 1];
                h[e / 2] = (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
            }
            const int cc = (n0 + 16 * j) / 2 + 4 * g;
            *reinterpret_cast<uint2 *>(out.x16 + (size_t)r * (N / 2) + cc) = make_uint2(h[0], h[1]);
        }
    } else if (row_ok && n < out.seg[out.nseg - 1].n_end) {  // channels past the last segment: padding
        int sgi = 0, nb = 0;
#pragma unroll
        for (int q = 0; q < kW8MaxSegs - 1; ++q)
            if (q < out.nseg - 1 && n >= out.seg[q].n_end) {
                sgi = q + 1;
                nb = out.seg[q].n_end;
            }
        float *dst = out.seg[0].dst;
        int ld = out.seg[0].ld;
#pragma unroll
        for (int q = 1; q < kW8MaxSegs; ++q)
            if (q == sgi) {
                dst = out.seg[q].dst;
                ld = out.seg[q].ld;
            }
        if (out.add_in) y = *reinterpret_cast<const f32x4_t *>(out.add_in + (size_t)r * out.add_ld + n) + y;
        *reinterpret_cast<f32x4_t *>(dst + (size_t)r * ld + (n - nb)) = y;
    }
}

// The narrow branch matrices at small M (out_proj, down: N = 2560): one
// 16-channel tile per block and no k-split.  Wave w takes NS consecutive
// 64-k steps, all its weight fragments requested up front; the waves' tiles
// are summed in LDS in wave order and wave 0 stores.  Against the k-split
// form (whose last block sums the splits), at N = 2560: K = 4096 5.3
// against 7.3 us (M = 1) and 7.2 against 8.0 us (M = 16); K = 9216 7.6
// against 8.9 us (M <= 3), but 12.8 against 9.8 us at M = 16 (its 18 steps
// per wave spill), where the k-split form stays.
template <int WAVES, int NS>
__global__ __launch_bounds__(64 * WAVES) void w8n_kernel(const uint16_t *__restrict__ x, const int8_t *__restrict__ W,
                                                         const float *__restrict__ scale, int M, int N, int K,
                                                         W8Out out) {
    __shared__ f32x4_t red[WAVES][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int t = blockIdx.x;         // 16-channel tile
    const int c = t >> 2, j = t & 3;  // its 64-channel group and place in the group
    const int steps = K / kKStep;
    const int s0 = wave * NS;         // this wave's first 64-k step
    const int8_t *wp = W + ((size_t)c * steps + s0) * 4096 + j * 1024 + lane * 16;
    const bool row_ok = r < M;
    // rows past M read row 0 (in bounds) and are zeroed
    const uint16_t *xp = x + (size_t)(row_ok ? r : 0) * K + s0 * kKStep + 16 * g;
    u32x4_t wv[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i)
        wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(wp + (size_t)i * 4096));
    f32x4_t acc = zero4();
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        u32x4_t xa = *reinterpret_cast<const u32x4_t *>(xp + i * kKStep);
        u32x4_t xb = *reinterpret_cast<const u32x4_t *>(xp + i * kKStep + 8);
        if (!row_ok) xa = xb = u32x4_t{0u, 0u, 0u, 0u};
        f16x8_t w0, w1;
        i8x16_to_f16(wv[i], w0, w1);
        acc = mfma_f16(w0, __builtin_bit_cast(f16x8_t, xa), acc);
        acc = mfma_f16(w1, __builtin_bit_cast(f16x8_t, xb), acc);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4_t y = red[0][lane];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) y += red[w][lane];
    const int n = 16 * t + 4 * g;  // C lane (g, r): channels n .. n+3 of batch row r
    if (row_ok && n < out.seg[0].n_end) {
        y = y * *reinterpret_cast<const f32x4_t *>(scale + n);
        if (out.add_in) y = *reinterpret_cast<const f32x4_t *>(out.add_in + (size_t)r * out.add_ld + n) + y;
        *reinterpret_cast<f32x4_t *>(out.seg[0].dst + (size_t)r * out.seg[0].ld + n) = y;
    }
}

// The decode GEMM at batch <= kW8vRows: one 16-channel tile per block, WPT
// waves over k, each wave NS consecutive 64-k steps (WPT * NS = K / 64).
// The block's input reaches LDS before any weight is requested: the
// activation rows (the block's threads copy x[M][K] in 16-byte pieces), or,
// for NR = M <= kW8NormInRows rows with W8Out::nin_h (and no pending
// branch), the loads of the residual norm's inputs, whose arithmetic
// finishes after the weights are requested.  Vector loads complete in issue order, so the input lands
// first and the norm runs while the weights stream.  Every weight step of
// a wave is requested up front, only the lanes of real rows read the input
// from LDS, and the kernel stays near 64 VGPRs, so that several blocks
// share a CU (the form that held 222 VGPRs ran at half the rate).  Each
// wave sums its steps in order (two MFMAs per step) and the tile's waves
// are added in wave order, the same for every M <= kW8vRows.  Epilogues as
// in w8f_kernel (segments, SwiGLU on the interleaved rows).
constexpr int kW8vRows = 3;
constexpr int kW8vPieces = 4;  // 16-byte pieces of x per thread: M K <= 32 * threads
constexpr int kW8vNormJ = 3;   // norm pieces per thread (of 256): K <= 3072

// The first half of w8f_norm_input's work for NR rows without a pending
// branch (W8Out::nin_add null: the branch matrix added it in its
// epilogue): threads 0..255 request their pieces of h and w;
// w8v_norm_finish does the arithmetic.  Pieces past K / 4 are not
// requested and not used.
template <int NR> struct NormPieces {
    f32x4_t h[NR][kW8vNormJ], w[kW8vNormJ];
};
template <int NR> GDN_DEV void w8v_norm_load(const W8Out &out, int K, NormPieces<NR> &p) {
    const int n4 = K / 4, tid = threadIdx.x;
    if (tid >= 256) return;
#pragma unroll
    for (int j = 0; j < kW8vNormJ; ++j) {
        const int i = tid + 256 * j;
        if (i < n4) {
            const float4 wv = reinterpret_cast<const float4 *>(out.nin_w)[i];
            p.w[j] = f32x4_t{wv.x, wv.y, wv.z, wv.w};
        }
    }
#pragma unroll
    for (int b = 0; b < NR; ++b)
#pragma unroll
        for (int j = 0; j < kW8vNormJ; ++j) {
            const int i = tid + 256 * j;
            if (i < n4) {
                const float4 hv = reinterpret_cast<const float4 *>(out.nin_h + (size_t)b * K)[i];
                p.h[b][j] = f32x4_t{hv.x, hv.y, hv.z, hv.w};
            }
        }
}
// w8f_norm_input's arithmetic on pieces already requested (the same sums in
// the same order); every thread of the block calls it (barriers).
template <int NR>
GDN_DEV void w8v_norm_finish(const W8Out &out, int K, NormPieces<NR> &p, uint16_t *xs, float *s_ss) {
    const int n4 = K / 4, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int b = 0; b < NR; ++b) {
        f32x4_t x[kW8vNormJ];
        float ss = 0.f;
        if (tid < 256) {
#pragma unroll
            for (int j = 0; j < kW8vNormJ; ++j) {
                const int i = tid + 256 * j;
                if (i < n4) {
                    x[j] = p.h[b][j];
                    ss += x[j][0] * x[j][0] + x[j][1] * x[j][1] + x[j][2] * x[j][2] + x[j][3] * x[j][3];
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
            if (lane == 0) s_ss[wave] = ss;
        }
        __syncthreads();
        const float inv = 1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) / (float)K + out.nin_eps);
        __syncthreads();  // s_ss is rewritten by the next row
        if (tid < 256) {
#pragma unroll
            for (int j = 0; j < kW8vNormJ; ++j) {
                const int i = tid + 256 * j;
                if (i < n4) {
                    const f32x4_t wv = p.w[j];
                    uint2 o;
                    o.x = (uint32_t)f32_to_f16_rne(x[j][0] * inv * (1.0f + wv[0])) |
                          ((uint32_t)f32_to_f16_rne(x[j][1] * inv * (1.0f + wv[1])) << 16);
                    o.y = (uint32_t)f32_to_f16_rne(x[j][2] * inv * (1.0f + wv[2])) |
                          ((uint32_t)f32_to_f16_rne(x[j][3] * inv * (1.0f + wv[3])) << 16);
                    *reinterpret_cast<uint2 *>(&xs[(size_t)b * K + 4 * i]) = o;
                }
            }
        }
    }
    __syncthreads();
}

// NR = 0: input x[M][K]; NR = M (1 or 2): the normalised rows of W8Out::nin_h
template <int WPT, int NS, int NR>
__global__ __launch_bounds__(64 * WPT) void w8v_kernel(const uint16_t *__restrict__ x, const int8_t *__restrict__ W,
                                                       const float *__restrict__ scale, int M, int N, int K,
                                                       W8Out out) {
    __shared__ f32x4_t red[WPT][64];
    __shared__ float s_ss[4];
    extern __shared__ __align__(16) uint16_t xs[];  // the block's input rows [M][K] fp16 (dynamic)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int t = blockIdx.x;        // 16-channel tile
    const int c = t >> 2, j = t & 3;  // its 64-channel group and place in the group
    const int steps = K / kKStep;     // WPT * NS
    const int s0 = wave * NS;         // this wave's first 64-k step
    const bool row_ok = r < M;
    // 1. the input's loads, ahead of every weight load
    NormPieces<NR == 0 ? 1 : NR> np;
    u32x4_t xin[kW8vPieces];
    const int npieces = M * K / 8;  // 16-byte pieces of x
    if constexpr (NR > 0) {
        w8v_norm_load<NR>(out, K, np);
    } else {
#pragma unroll
        for (int q = 0; q < kW8vPieces; ++q) {
            const int i = threadIdx.x + q * 64 * WPT;
            if (i < npieces) xin[q] = reinterpret_cast<const u32x4_t *>(x)[i];
        }
    }
    // 2. every weight step of this wave
    const int8_t *wp = W + ((size_t)c * steps + s0) * 4096 + j * 1024 + lane * 16;
    u32x4_t wv[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i)
        wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(wp + (size_t)i * 4096));
    // 3. the input rows into LDS
    if constexpr (NR > 0) {
        w8v_norm_finish<NR>(out, K, np, xs, s_ss);
    } else {
#pragma unroll
        for (int q = 0; q < kW8vPieces; ++q) {
            const int i = threadIdx.x + q * 64 * WPT;
            if (i < npieces) reinterpret_cast<u32x4_t *>(xs)[i] = xin[q];
        }
        __syncthreads();
    }
    // 4. the tile: lane (g, r) holds row r's k = 64 s + 16 g .. +15; lanes
    // of rows past M read nothing and multiply zeros
    const uint16_t *xp = &xs[(size_t)(row_ok ? r : 0) * K + s0 * kKStep + 16 * g];
    f32x4_t acc = zero4();
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        u32x4_t xa = u32x4_t{0u, 0u, 0u, 0u}, xb = xa;
        if (row_ok) {
            xa = *reinterpret_cast<const u32x4_t *>(xp + i * kKStep);
            xb = *reinterpret_cast<const u32x4_t *>(xp + i * kKStep + 8);
        }
        f16x8_t w0, w1;
        i8x16_to_f16(wv[i], w0, w1);
        acc = mfma_f16(w0, __builtin_bit_cast(f16x8_t, xa), acc);
        acc = mfma_f16(w1, __builtin_bit_cast(f16x8_t, xb), acc);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4_t y = red[0][lane];
#pragma unroll
    for (int w = 1; w < WPT; ++w) y += red[w][lane];
    const int n = 16 * t + 4 * g;  // C lane (g, r): channels n .. n+3 of batch row r
    y = y * *reinterpret_cast<const f32x4_t *>(scale + n);
    if (out.mode == kW8SwiGLU) {
        f32x4_t up;
#pragma unroll
        for (int e = 0; e < 4; ++e) up[e] = __shfl_xor(y[e], 32);
        if (g < 2 && row_ok) {
            uint32_t h[2];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float a = y[e] / (1.0f + expf(-y[e])) * up[e];
                const float b = y[e + 1] / (1.0f + expf(-y[e + 1])) * up[e + 1];
                h[e / 2] = (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
            }
            const int cc = 8 * t + 4 * g;
            *reinterpret_cast<uint2 *>(out.x16 + (size_t)r * (N / 2) + cc) = make_uint2(h[0], h[1]);
        }
    } else if (row_ok && n < out.seg[out.nseg - 1].n_end) {  // channels past the last segment: padding
        int sgi = 0, nb = 0;
#pragma unroll
        for (int q = 0; q < kW8MaxSegs - 1; ++q)
            if (q < out.nseg - 1 && n >= out.seg[q].n_end) {
                sgi = q + 1;
                nb = out.seg[q].n_end;
            }
        float *dst = out.seg[0].dst;
        int ld = out.seg[0].ld;
#pragma unroll
        for (int q = 1; q < kW8MaxSegs; ++q)
            if (q == sgi) {
                dst = out.seg[q].dst;
                ld = out.seg[q].ld;
            }
        if (out.add_in) y = *reinterpret_cast<const f32x4_t *>(out.add_in + (size_t)r * out.add_ld + n) + y;
        *reinterpret_cast<f32x4_t *>(dst + (size_t)r * ld + (n - nb)) = y;
    }
}

}  // namespace

// Launch shape from a sweep over the Qwen3.5-4B matrices at M = 1 and 16
// (weights rotated through 1.5 GB so none comes from the Infinity Cache):
// one step in flight per wave; eight waves per block when there are fewer
// blocks than CUs (each block must pull more bytes), four when there are
// more (a CU then holds several blocks at once: gate|up 10.7 us against
// 12.3 us); k-splits only for narrow matrices, the fewest that give 160
// blocks (the cross-block hand-off costs more than the extra parallelism
// beyond that).
W8fShape w8f_shape(int N, int K) {
    const int groups = N / kW8fGroup;
    W8fShape sh{K % 512 == 0 && groups <= 256 ? 8 : 4, 1, 1};
    for (int S = 2; S <= 32 && groups * sh.splits < 160; ++S)
        if (K % (S * sh.waves * kKStep) == 0) sh.splits = S;
    return sh;
}

size_t w8f_workspace_floats(int M, int N, int K) {
    const W8fShape sh = w8f_shape(N, K);
    return sh.splits > 1 ? (size_t)sh.splits * M * N : 0;
}

hipError_t launch_w8f_tile(const int8_t *src, int8_t *dst, int N, int K, hipStream_t st) {
    if (N % kW8fGroup != 0 || K % kKStep != 0) return hipErrorInvalidValue;
    const size_t chunks = (size_t)N * K / 16;
    w8f_tile_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, st>>>(src, dst, K, chunks);
    return hipGetLastError();
}

// The small-batch form's launch: hipErrorNotSupported where it has no
// instantiation for the shape (the caller then takes another form).  Eight
// waves per tile at K = 2560 (the hidden size: in-projections, gate|up),
// sixteen at K = 4096 and 9216 (out_proj, o_proj, down: 160 tiles, fewer
// blocks than CUs, so each block splits k finer).  The LM head (9496 tiles)
// keeps w8f_kernel, whose 64-channel blocks form the norm a quarter as often.
hipError_t launch_w8v(const uint16_t *x, const int8_t *W, const float *scale, int M, int N, int K,
                      const W8Out &out, hipStream_t st) {
    const int steps = K / kKStep, tiles = N / 16;
    if (M > kW8vRows || N % kW8fGroup || K % kKStep || tiles > 2048) return hipErrorNotSupported;
    const size_t lds = (size_t)M * K * 2;
    if (out.nin_h) {
        if (steps != 40 || K / 4 > 256 * kW8vNormJ || M != 1 || out.nin_add) return hipErrorNotSupported;
        w8v_kernel<8, 5, 1><<<tiles, 512, lds, st>>>(x, W, scale, M, N, K, out);
        return hipGetLastError();
    }
    const int wpt = steps == 40 ? 8 : 16;
    if ((size_t)M * K / 8 > (size_t)kW8vPieces * 64 * wpt) return hipErrorNotSupported;
    if (steps == 40) w8v_kernel<8, 5, 0><<<tiles, 512, lds, st>>>(x, W, scale, M, N, K, out);
    else if (steps == 64) w8v_kernel<16, 4, 0><<<tiles, 1024, lds, st>>>(x, W, scale, M, N, K, out);
    else if (steps == 144) w8v_kernel<16, 9, 0><<<tiles, 1024, lds, st>>>(x, W, scale, M, N, K, out);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

hipError_t launch_w8f(const uint16_t *x, const int8_t *W, const float *scale, int M, int N, int K,
                      const W8Out &out, float *part, uint32_t *cnt, hipStream_t st, W8fShape sh) {
    if (M == 0 || N == 0) return hipSuccess;
    if (out.nin_h && (M > kW8NormInRows || K > kW8NormInMaxK || K % 4 || !out.nin_w ||
                      (out.nin_add && !out.nin_hout)))
        return hipErrorInvalidValue;
    if (out.add_in && (out.mode != kW8Segments || out.nseg != 1)) return hipErrorInvalidValue;
    // batch <= kW8vRows: the small-batch form where it has one for the shape
    if (sh.splits == 0) {
        const hipError_t e = launch_w8v(x, W, scale, M, N, K, out, st);
        if (e != hipErrorNotSupported) return e;
    }
    // the narrow single-output matrices: one tile per block, no k-split
    // (w8n_kernel), when no launch shape is asked for
    if (sh.splits == 0 && out.mode == kW8Segments && out.nseg == 1 && !out.nin_h && N % kW8fGroup == 0 &&
        ((K == 8 * 8 * kKStep && M <= 16) || (K == 8 * 18 * kKStep && M <= 3))) {
        if (K == 8 * 8 * kKStep) w8n_kernel<8, 8><<<N / 16, 512, 0, st>>>(x, W, scale, M, N, K, out);
        else w8n_kernel<8, 18><<<N / 16, 512, 0, st>>>(x, W, scale, M, N, K, out);
        return hipGetLastError();
    }
    if (sh.splits == 0) sh = w8f_shape(N, K);
    const int S = sh.splits;
    if (M > 16 || N % kW8fGroup != 0 || K % (S * sh.waves * sh.depth * kKStep) != 0) return hipErrorInvalidValue;
    if (S > 1 && (!part || !cnt || (size_t)S * M * N * 4 > 0x7FFFFFFFull)) return hipErrorInvalidValue;
    const dim3 grid(N / kW8fGroup, S);
#define W8F_CASE(WV, DP)                                                                                  \
    if (sh.waves == WV && sh.depth == DP) {                                                                \
        if (out.nin_h)                                                                                     \
            w8f_kernel<WV, DP, true><<<grid, 64 * WV, (size_t)M * K * 2, st>>>(x, W, scale, M, N, K, K / S, S, \
                                                                               part, cnt, out);             \
        else                                                                                               \
            w8f_kernel<WV, DP><<<grid, 64 * WV, 0, st>>>(x, W, scale, M, N, K, K / S, S, part, cnt, out); \
        return hipGetLastError();                                                                          \
    }
    W8F_CASE(4, 1)
    W8F_CASE(4, 2)
    W8F_CASE(4, 4)
    W8F_CASE(8, 1)
    W8F_CASE(8, 2)
    W8F_CASE(8, 4)
#undef W8F_CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Attention decode (HF Qwen3_5Attention with a KV cache, one new token per
// sequence; eager_attention_forward, modeling_qwen3_5.py:606-627): for query
// head h of sequence b, with kv = h / (Hq / Hkv) (repeat_kv),
//   o[b][h] = softmax_t(scaling * q[b][h] . K[b][kv][t]) . V[b][kv][t],  t < L
// q [B][Hq][256] fp16, K, V [B][Hkv][Tmax][256] fp16, fp32 softmax and sums.
// Split over the sequence: block (span, kv, b) takes positions [256 span,
// 256 span + 256) and every query head of kv; wave w takes 64 of them in
// groups of 16.  Scores on fp16 MFMA 16x16x32 (A = 16 key rows, B = the
// group's query heads as columns); online softmax per head in exp2; P.V on
// the VALU, lane l holding dims 4l .. 4l+3 of every head's output.  The
// block's four waves merge through LDS into one partial (max, sum, o) per
// head; attn_combine_kernel merges the spans.  With a tiled K cache (the
// hybrid model's own) each group's 16 rows are 8 contiguous KB laid out in
// MFMA-lane order, so every K load of a wave is one contiguous 1 KB (10%
// faster at B=16 and 32K than the 16 x 64-byte row pieces of the row-major
// cache).
// ---------------------------------------------------------------------------
namespace {

constexpr int kAttD = 256;
constexpr int kAttSpan = 256;   // positions per block
constexpr int kAttRepMax = 4;   // query heads per kv head handled (Hq / Hkv <= 4)
constexpr int kAttPart = kAttD + 2;

template <bool KTILED>
__global__ __launch_bounds__(256) void attn_decode_kernel(const uint16_t *__restrict__ q,
                                                          const uint16_t *__restrict__ Kc,
                                                          const uint16_t *__restrict__ Vc,
                                                          float *__restrict__ part, int Hq, int Hkv,
                                                          int Tmax, int L, int nspan, int G, float sc_log2) {
    __shared__ float s_m[4][kAttRepMax], s_l[4][kAttRepMax];
    __shared__ float s_o[4][kAttRepMax][kAttD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int span = blockIdx.x, kv = blockIdx.y, b = blockIdx.z;
    const int rep = Hq / Hkv;
    const size_t kvrow = ((size_t)b * Hkv + kv) * Tmax;  // row of position 0
    // B operand: query head r of the group (zero columns past rep), dims
    // 32 j + 8 g .. +7
    f16x8_t qb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        u32x4_t u = {0u, 0u, 0u, 0u};
        if (r < rep) u = *reinterpret_cast<const u32x4_t *>(q + ((size_t)b * Hq + kv * rep + r) * kAttD + 32 * j + 8 * g);
        qb[j] = __builtin_bit_cast(f16x8_t, u);
    }
    float m[kAttRepMax], l[kAttRepMax], o[kAttRepMax][4];
#pragma unroll
    for (int h = 0; h < kAttRepMax; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[h][i] = 0.f;
    }
    // Each wave takes G groups of 16 positions (the span is 64 G),
    // double-buffered: the K rows and V rows of the next group are in
    // flight while a group is scored and accumulated.  Rows past L are
    // clamped to L - 1 (in bounds; masked by p = 0).
    const int t_begin = span * (64 * G) + wave * (16 * G);
    const int t_end = min(t_begin + 16 * G, L);
    u32x4_t kbuf[2][8];
    u32x2_t vbuf[2][16];
    auto load_group = [&](int t0, u32x4_t (&kb)[8], u32x2_t (&vb)[16]) {
        if constexpr (KTILED) {
            // the group's 16 rows as 8 contiguous KB (kv_tiled_offset)
            const uint16_t *kp = Kc + (kvrow + t0) * kAttD + lane * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                kb[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(kp + 512 * j));
        } else {
            const uint16_t *kp = Kc + (kvrow + min(t0 + r, L - 1)) * kAttD + 8 * g;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                kb[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(kp + 32 * j));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            vb[i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x2_t *>(Vc + (kvrow + min(t0 + i, L - 1)) * kAttD + 4 * lane));
    };
    auto process = [&](const u32x4_t (&kb)[8], const u32x2_t (&vb)[16], int t0) {
        f32x4_t acc = zero4();
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, kb[j]), qb[j], acc, 0, 0, 0);
        // lane (g, r): scores of positions t0 + 4g + e for head r, in log2 units
        float s[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = (t0 + 4 * g + e < L) ? acc[e] * sc_log2 : -INFINITY;
        float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // per head r (all lanes of column r agree); the new running max
        float p[4], mrow = -INFINITY;
#pragma unroll
        for (int h = 0; h < kAttRepMax; ++h)
            if (h == r) mrow = m[h];
        const float mnew = fmaxf(mrow, mx);
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            p[e] = __builtin_amdgcn_exp2f(s[e] - mnew);
            ps += p[e];
        }
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);  // 0 on the first group
        // every lane: the running state of each head from lane h
#pragma unroll
        for (int h = 0; h < kAttRepMax; ++h) {
            if (h >= rep) break;
            const float a_h = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
            const float mn_h = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mnew), h));
            const float ps_h = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ps), h));
            m[h] = mn_h;
            l[h] = l[h] * a_h + ps_h;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[h][i] *= a_h;
        }
        // P.V: position t0 + 4gg + e, head h: p in lane 16 gg + h, element e
        // (p = 0 for positions past L)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const u32x2_t vv = vb[4 * gg + e];
                const float v[4] = {f16_to_f32((uint16_t)(vv[0] & 0xFFFFu)), f16_to_f32((uint16_t)(vv[0] >> 16)),
                                    f16_to_f32((uint16_t)(vv[1] & 0xFFFFu)), f16_to_f32((uint16_t)(vv[1] >> 16))};
#pragma unroll
                for (int h = 0; h < kAttRepMax; ++h) {
                    if (h >= rep) break;
                    const float ph = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p[e]), 16 * gg + h));
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[h][i] += ph * v[i];
                }
            }
    };
    if (t_begin < t_end) load_group(t_begin, kbuf[0], vbuf[0]);
    for (int t0 = t_begin; t0 < t_end; t0 += 32) {  // uniform over the wave
        const int t1 = t0 + 16;
        if (t1 < t_end) load_group(t1, kbuf[1], vbuf[1]);
        process(kbuf[0], vbuf[0], t0);
        if (t1 >= t_end) break;
        if (t1 + 16 < t_end) load_group(t1 + 16, kbuf[0], vbuf[0]);
        process(kbuf[1], vbuf[1], t1);
    }
    // merge the four waves (each may have seen no position: m = -inf, l = 0)
    if (lane == 0)
#pragma unroll
        for (int h = 0; h < kAttRepMax; ++h) {
            s_m[wave][h] = m[h];
            s_l[wave][h] = l[h];
        }
#pragma unroll
    for (int h = 0; h < kAttRepMax; ++h)
        *reinterpret_cast<float4 *>(&s_o[wave][h][4 * lane]) = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
    __syncthreads();
    // thread (h, d): h = tid / 64, dims 4 (tid % 64) .. +3
    const int h = threadIdx.x >> 6;
    if (h >= rep) return;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w][h]);
    float lsum = 0.f, acc4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float f = s_m[w][h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w][h] - M);
        lsum += f * s_l[w][h];
        const float4 ow = *reinterpret_cast<const float4 *>(&s_o[w][h][4 * lane]);
        acc4[0] += f * ow.x;
        acc4[1] += f * ow.y;
        acc4[2] += f * ow.z;
        acc4[3] += f * ow.w;
    }
    float *pp = part + (((size_t)b * Hq + kv * rep + h) * nspan + span) * kAttPart;
    *reinterpret_cast<float4 *>(pp + 4 * lane) = make_float4(acc4[0], acc4[1], acc4[2], acc4[3]);
    if (lane == 0) {
        pp[kAttD] = M;
        pp[kAttD + 1] = lsum;
    }
}

// o[b][h][d] = sum_s e^{m_s - M} o_s[d] / sum_s e^{m_s - M} l_s (log2 units),
// one block per (b, h): wave j takes the spans s = j mod 4, lane l dims
// 4l .. 4l+3; the four waves merge in a fixed order.  With `gate`, the
// output is fp16(o * sigmoid(gate[bh * gate_stride + d])) into out16
// (the sigmoid output gate of Qwen3_5Attention), else fp32 into out.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *__restrict__ part,
                                                           float *__restrict__ out, const float *__restrict__ gate,
                                                           int gate_stride, uint16_t *__restrict__ out16,
                                                           int nspan) {
    __shared__ float s_red[4];
    __shared__ float s_l[4];
    __shared__ float4 s_o[4][64];
    const size_t bh = blockIdx.x;
    const float *pp = part + bh * nspan * kAttPart;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float M = -INFINITY;
    for (int s = tid; s < nspan; s += 256) M = fmaxf(M, pp[s * kAttPart + kAttD]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    if (lane == 0) s_red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float lsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int s = wave; s < nspan; s += 4) {
        const float *ps = pp + s * kAttPart;
        const float ms = ps[kAttD];
        const float f = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - M);
        lsum += f * ps[kAttD + 1];
        const float4 v = *reinterpret_cast<const float4 *>(ps + 4 * lane);
        acc.x += f * v.x;
        acc.y += f * v.y;
        acc.z += f * v.z;
        acc.w += f * v.w;
    }
    s_o[wave][lane] = acc;
    if (lane == 0) s_l[wave] = lsum;
    __syncthreads();
    const int d = tid;
    const float *so = reinterpret_cast<const float *>(s_o);
    const float num = ((so[d] + so[256 + d]) + so[512 + d]) + so[768 + d];
    const float den = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];
    const float y = num / den;
    if (gate) {
        const float gt = gate[bh * gate_stride + d];
        out16[bh * kAttD + d] = f32_to_f16_rne(y * (1.0f / (1.0f + expf(-gt))));
    } else {
        out[bh * kAttD + d] = y;
    }
}

}  // namespace

size_t attn_workspace_bytes(int B, int Hq, int L) {
    const int nspan = (L + kAttSpan - 1) / kAttSpan;
    return (size_t)B * Hq * nspan * kAttPart * sizeof(float);
}

// Groups of 16 positions per wave.  256-position spans (G = 4) for a
// row-major K cache.  For a tiled-K cache the span is sized for a block
// count: a grid of fewer than 2048 blocks of 256 positions fills 512 slots
// (2 per CU on 256 CUs) in one round -- at B = 1 and 32K, 129 x 4 = 516
// blocks of 256 positions would leave 4 blocks for a second round that
// doubles the kernel's time -- and a larger grid is cut into about 2048
// blocks: at B = 16 and 32K, spans of 16 groups (2112 blocks) took 356.5
// against 381.4 us per layer with 4 groups (8256 blocks), decode and
// combine, with 8 to 24 groups all within 364 us (longer spans read the
// KV stream faster and leave fewer partials to combine).
int attn_groups(int B, int Hkv, int L, bool k_tiled) {
    const long blocks256 = (long)B * Hkv * ((L + kAttSpan - 1) / kAttSpan);
    if (!k_tiled) return 4;
    const int target = blocks256 >= 2048 ? 2048 : 512;
    const int per_kv = max(1, target / (B * Hkv));
    return max(1, (L + 64 * per_kv - 1) / (64 * per_kv));
}

size_t attn_workspace_bytes_tiled(int B, int Hq, int L) {
    const int nspan = (L + 63) / 64;  // enough for any span of a whole number of 64 positions
    return (size_t)B * Hq * nspan * kAttPart * sizeof(float);
}

hipError_t launch_attn_decode(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, float *out,
                              int B, int Hq, int Hkv, int Tmax, int L, float scaling, float *workspace,
                              hipStream_t st, const float *gate, int gate_stride, uint16_t *out16, bool k_tiled) {
    if (B == 0) return hipSuccess;
    if (k_tiled && Tmax % 16 != 0) return hipErrorInvalidValue;
    const int G = attn_groups(B, Hkv, L, k_tiled);
    const int nspan = (L + 64 * G - 1) / (64 * G);
    const float sc_log2 = scaling * 1.4426950408889634f;
    if (k_tiled)
        attn_decode_kernel<true><<<dim3(nspan, Hkv, B), 256, 0, st>>>(q, Kc, Vc, workspace, Hq, Hkv, Tmax, L, nspan,
                                                                      G, sc_log2);
    else
        attn_decode_kernel<false><<<dim3(nspan, Hkv, B), 256, 0, st>>>(q, Kc, Vc, workspace, Hq, Hkv, Tmax, L,
                                                                       nspan, G, sc_log2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_combine_kernel<<<dim3(B * Hq), kAttD, 0, st>>>(workspace, out, gate, gate_stride, out16, nspan);
    return hipGetLastError();
}

}  // namespace gdn

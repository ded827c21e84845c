// gdn_probe.hip -- measurement probes for the roofline figures: what this
// GPU actually delivers for a streaming copy, a streaming read, and dense
// bf16 MFMA, next to the datasheet peaks (HBM 8 TB/s, bf16 2.5 PFLOP/s).
// They compute nothing of the GDN path.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeWords = 4 * kProbeThreads;  // 16-byte words per block
constexpr int kProbeBlocksPerCU = 16;

// Block b copies (or reads) words [1024 b, 1024 b + 1024): four
// non-temporal 16-byte loads in flight per thread, then the stores.  A sweep
// of probe forms on MI355X gave 6.2 TB/s copy and 7.0 TB/s read for this
// one, against 4.6 and 6.0 TB/s for a grid-stride loop.
__global__ __launch_bounds__(kProbeThreads) void probe_copy_kernel(const u32x4_t *__restrict__ src,
                                                                   u32x4_t *__restrict__ dst, size_t n) {
    const size_t base = (size_t)blockIdx.x * kProbeWords + threadIdx.x;
    u32x4_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (base + kProbeThreads * i < n) v[i] = __builtin_nontemporal_load(src + base + kProbeThreads * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (base + kProbeThreads * i < n) __builtin_nontemporal_store(v[i], dst + base + kProbeThreads * i);
}

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const u32x4_t *__restrict__ src,
                                                                   uint32_t *__restrict__ sink, size_t n) {
    const size_t base = (size_t)blockIdx.x * kProbeWords + threadIdx.x;
    u32x4_t acc = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (base + kProbeThreads * i < n) acc ^= __builtin_nontemporal_load(src + base + kProbeThreads * i);
    // keep the loads: a store that practically never happens
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9E3779B9u) sink[threadIdx.x] = 1u;
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Independent bf16 MFMA chains per wave, iters steps each: SHAPE 0 is
// 32x32x16 (four chains), 1 is 16x16x32 (eight chains); the accumulators'
// sum goes to sink[thread].
template <int SHAPE>
__global__ __launch_bounds__(kProbeThreads) void probe_mfma_kernel(float *__restrict__ sink, int iters, float seed) {
    const float x = seed * (float)(threadIdx.x + 1);
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = x * (float)(i + 1);
    const bf16x8_t a = pack_bf16x8(f), b = pack_bf16x8(f);
    float s = 0.f;
    if constexpr (SHAPE == 0) {
        f32x16_t acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[c][e] = 0.f;
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < 4; ++c) s += acc[c][0] + acc[c][15];
    } else {
        f32x4_t acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = zero4();
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = mfma_16x16x32_bf16(a, b, acc[c]);
#pragma unroll
        for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][3];
    }
    sink[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

}  // namespace

size_t probe_sink_words(int cu_count) { return (size_t)cu_count * kProbeBlocksPerCU * kProbeThreads; }

hipError_t launch_probe_stream(const void *src, void *dst, size_t bytes, int mode, uint32_t *sink, int cu_count,
                               hipStream_t st) {
    (void)cu_count;
    const size_t n = bytes / 16;
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + kProbeWords - 1) / kProbeWords;
    if (blocks > 0x7FFFFFFFu) return hipErrorInvalidValue;
    if (mode == 0)
        probe_copy_kernel<<<(unsigned)blocks, kProbeThreads, 0, st>>>(static_cast<const u32x4_t *>(src),
                                                                       static_cast<u32x4_t *>(dst), n);
    else
        probe_read_kernel<<<(unsigned)blocks, kProbeThreads, 0, st>>>(static_cast<const u32x4_t *>(src), sink, n);
    return hipGetLastError();
}

hipError_t launch_probe_mfma(float *sink, int iters, int shape, int cu_count, unsigned long long *flops,
                             hipStream_t st) {
    const unsigned blocks = (unsigned)cu_count * kProbeBlocksPerCU;
    const unsigned long long waves = (unsigned long long)blocks * (kProbeThreads / 64);
    if (shape == 0) {
        probe_mfma_kernel<0><<<blocks, kProbeThreads, 0, st>>>(sink, iters, 1e-3f);
        *flops = waves * (unsigned long long)iters * 4ull * (2ull * 32 * 32 * 16);
    } else {
        probe_mfma_kernel<1><<<blocks, kProbeThreads, 0, st>>>(sink, iters, 1e-3f);
        *flops = waves * (unsigned long long)iters * 8ull * (2ull * 16 * 16 * 32);
    }
    return hipGetLastError();
}

}  // namespace gdn

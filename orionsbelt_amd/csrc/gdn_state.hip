// gdn_state.hip -- the state formats of the prefill -> decode hand-off and the
// decode-step conv, for gfx950.
//
// HF keeps a GDN layer's cache as (transformers cache_utils.py,
// LinearAttentionLayer.update_conv_state:1032-1070, and
// modeling_qwen3_5.py causal_conv1d_update:199-217):
//   conv_state [B][C][4]: the last four conv inputs of each sequence, newest
//                         last, zero-padded on the left after a short prefill;
//   recurrent state [B][Hv][128][128] in the model dtype.
// The kai conv (kai_gdn_causal_dwconv1d_f32_k4_sve.h:28-36) instead carries
// hist [3][C]: the last three inputs, oldest first, channel-major.  The
// kernels here convert between the two and run HF's one-token conv update
// on the HF layout for a batch of sequences, with the kai conv's arithmetic:
// ((s1*w0 + s2*w1) + s3*w2) + x*w3 without contraction (the reference's
// scalar order), so a sequence continued by decode steps is bit-identical
// to the kai conv run over the whole sequence.  All of it is index work or
// a 4-tap dot product: one thread per (sequence, channel), 16-byte state
// accesses, launch-bound at decode sizes.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int kThreads = 256;

GDN_DEV float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
GDN_DEV void st4(float *p, float4 x) { *reinterpret_cast<float4 *>(p) = x; }

// One thread per (sequence b = blockIdx.y, channel c): x and out [B][T][C],
// conv_state [B][C][4], w [C][4] (HF's conv1d.weight.squeeze(1)).
template <bool SILU>
__global__ __launch_bounds__(kThreads) void conv_update_kernel(const float *__restrict__ x,
                                                               float *__restrict__ conv_state,
                                                               const float *__restrict__ w,
                                                               float *__restrict__ out, int T,
                                                               int64_t C) {
#pragma clang fp contract(off)
    const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (c >= C) return;
    const int64_t b = blockIdx.y;
    float *sp = conv_state + (b * C + c) * 4;
    const float4 s = ld4(sp), wv = ld4(w + c * 4);
    float s1 = s.y, s2 = s.z, s3 = s.w, s0 = s.x;
    for (int t = 0; t < T; ++t) {
        const int64_t i = (b * T + t) * C + c;
        const float cur = x[i];
        float acc = s1 * wv.x + s2 * wv.y + s3 * wv.z + cur * wv.w;
        if (SILU) acc = acc / (1.0f + expf(-acc));
        out[i] = acc;
        s0 = s1;
        s1 = s2;
        s2 = s3;
        s3 = cur;
    }
    st4(sp, make_float4(s0, s1, s2, s3));
}

// conv_state [B][C][4] = the last four rows of x [B][T][C], zero where the
// sequence is shorter than four (HF's prefill path of update_conv_state).
__global__ __launch_bounds__(kThreads) void conv_state_from_inputs_kernel(
    const float *__restrict__ x, float *__restrict__ conv_state, int64_t T, int64_t C) {
    const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (c >= C) return;
    const int64_t b = blockIdx.y;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t t = T - 4 + j;
        v[j] = t >= 0 ? x[(b * T + t) * C + c] : 0.0f;
    }
    st4(conv_state + (b * C + c) * 4, make_float4(v[0], v[1], v[2], v[3]));
}

// hist [B][3][C] (oldest first) <-> conv_state [B][C][4]: the three newest
// entries.  Entry 0 of the HF state (the input four steps back) feeds no
// later output; hist -> state writes it as 0.
template <bool TO_HIST>
__global__ __launch_bounds__(kThreads) void conv_hist_state_kernel(float *__restrict__ hist,
                                                                   float *__restrict__ conv_state,
                                                                   int64_t C) {
    const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (c >= C) return;
    const int64_t b = blockIdx.y;
    float *sp = conv_state + (b * C + c) * 4;
    float *hp = hist + b * 3 * C + c;
    if constexpr (TO_HIST) {
        const float4 s = ld4(sp);
        hp[0] = s.y;
        hp[C] = s.z;
        hp[2 * C] = s.w;
    } else {
        st4(sp, make_float4(0.0f, hp[0], hp[C], hp[2 * C]));
    }
}

// Element format conversion of a recurrent state (or any array): fp32,
// IEEE fp16 and bf16 bit patterns, through fp32; narrowing rounds to nearest
// even (bf16 by the reference's bias-and-truncate rule, gdn_sve.c:81-87).
GDN_DEV float fmt_load(const void *p, int fmt, size_t i) {
    if (fmt == kF32) return static_cast<const float *>(p)[i];
    const uint16_t u = static_cast<const uint16_t *>(p)[i];
    return fmt == kF16 ? f16_to_f32(u) : bf16_to_f32(u);
}
GDN_DEV void fmt_store(void *p, int fmt, size_t i, float x) {
    if (fmt == kF32) static_cast<float *>(p)[i] = x;
    else static_cast<uint16_t *>(p)[i] = fmt == kF16 ? f32_to_f16_rne(x) : f32_to_bf16_rne(x);
}
__global__ __launch_bounds__(kThreads) void convert_kernel(const void *__restrict__ src, int sf,
                                                           void *__restrict__ dst, int df,
                                                           size_t n) {
    const size_t stride = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        fmt_store(dst, df, i, fmt_load(src, sf, i));
}

dim3 per_channel_grid(int B, size_t C) {
    return dim3((unsigned)((C + kThreads - 1) / kThreads), (unsigned)B);
}

}  // namespace

hipError_t launch_conv_update(const float *x, float *conv_state, const float *w, float *out, int B,
                              int T, size_t C, bool silu, hipStream_t st) {
    if (B == 0 || C == 0 || T == 0) return hipSuccess;
    if (silu)
        conv_update_kernel<true><<<per_channel_grid(B, C), kThreads, 0, st>>>(x, conv_state, w, out, T,
                                                                              (int64_t)C);
    else
        conv_update_kernel<false><<<per_channel_grid(B, C), kThreads, 0, st>>>(x, conv_state, w, out, T,
                                                                               (int64_t)C);
    return hipGetLastError();
}

hipError_t launch_conv_state_from_inputs(const float *x, float *conv_state, int B, size_t T, size_t C,
                                         hipStream_t st) {
    if (B == 0 || C == 0) return hipSuccess;
    conv_state_from_inputs_kernel<<<per_channel_grid(B, C), kThreads, 0, st>>>(x, conv_state, (int64_t)T,
                                                                                (int64_t)C);
    return hipGetLastError();
}

hipError_t launch_conv_hist_state(bool to_hist, float *hist, float *conv_state, int B, size_t C,
                                  hipStream_t st) {
    if (B == 0 || C == 0) return hipSuccess;
    if (to_hist)
        conv_hist_state_kernel<true><<<per_channel_grid(B, C), kThreads, 0, st>>>(hist, conv_state,
                                                                                  (int64_t)C);
    else
        conv_hist_state_kernel<false><<<per_channel_grid(B, C), kThreads, 0, st>>>(hist, conv_state,
                                                                                   (int64_t)C);
    return hipGetLastError();
}

hipError_t launch_convert(const void *src, int sf, void *dst, int df, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t want = (n + kThreads - 1) / kThreads;
    const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
    convert_kernel<<<blocks, kThreads, 0, st>>>(src, sf, dst, df, n);
    return hipGetLastError();
}

}  // namespace gdn

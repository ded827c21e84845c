// gdn_layer.hip -- the layer glue on either side of the recurrence kernels
// for gfx950: the gating prologue (conv output -> normalised q, k, v and the
// gates g, beta) and the gated RMSNorm epilogue (recurrence output, gate z ->
// the input of out_proj).  Both are elementwise with one reduction over a
// 128-value head row, so they are HBM-bound: every value is read once and
// written once with 16-byte non-temporal accesses, one 16-lane DPP row per
// 128-value row (8 values per lane), and a block keeps several rows' loads in
// flight per group before it reduces any of them.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int D = kHeadDim;    // 128 values per head row
constexpr int kThreads = 256;  // sixteen 16-lane rows
constexpr int kGroups = kThreads / 16;
constexpr int kPass = 4;       // head rows in flight per 16-lane group (prologue)
// rows in flight per 16-lane group (RMSNorm): 8 bf16 or 4 fp32 rows of o and
// z, 64 registers per lane either way
template <typename T> constexpr int kRowsPass = sizeof(T) == 2 ? 8 : 4;

// Eight consecutive values of a 128-value row per lane: lane l of a 16-lane
// group holds values 8l .. 8l+7, moved as 16-byte accesses (one for bf16, two
// for fp32) with non-temporal hints (every value is touched once).
struct V8 {
    float f[8];
};
GDN_DEV V8 load8(const float *p) {
    const float4 a = load_f4<true>(p), b = load_f4<true>(p + 4);
    return V8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}
// bf16 rows stay packed (four registers) until they are used.
struct Raw16 {
    u32x4_t u;
};
struct Raw32 {
    float4 a, b;
};
GDN_DEV Raw16 load_raw(const uint16_t *p) {
    return Raw16{__builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p))};
}
GDN_DEV Raw32 load_raw(const float *p) { return Raw32{load_f4<true>(p), load_f4<true>(p + 4)}; }
GDN_DEV V8 unpack(const Raw32 &r) {
    return V8{{r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w}};
}
GDN_DEV V8 unpack(const Raw16 &r) {
    const u32x4_t u = r.u;
    V8 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v.f[2 * i] = __uint_as_float(u[i] << 16);
        v.f[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
    }
    return v;
}
GDN_DEV V8 load8(const uint16_t *p) { return unpack(load_raw(p)); }
GDN_DEV void store8(float *p, const V8 &v) {
    store_f4<true>(p, make_float4(v.f[0], v.f[1], v.f[2], v.f[3]));
    store_f4<true>(p + 4, make_float4(v.f[4], v.f[5], v.f[6], v.f[7]));
}
// bf16 by the hardware convert (round to nearest even).
GDN_DEV void store8(uint16_t *p, const V8 &v) {
    u32x4_t u;
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = pack2_bf16_hw(v.f[2 * i], v.f[2 * i + 1]);
    __builtin_nontemporal_store(u, reinterpret_cast<u32x4_t *>(p));
}
GDN_DEV float sumsq8(const V8 &v) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v.f[i] * v.f[i];
    return s;
}

// Sum over the 16 lanes of a row group.
GDN_DEV float group_sum(float x) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) x += __shfl_xor(x, m, 16);
    return x;
}

// x rounded to bf16 (nearest even) and widened back.
GDN_DEV float round_bf16(float x) { return bf16_to_f32(f32_to_bf16_hw(x)); }
// SiLU with the hardware exp2 and reciprocal: t / (1 + exp(-t)) within a few
// fp32 ulps (the exponent's product rounding and one ulp each for v_exp and
// v_rcp), far inside one bf16 ulp; the division and expf of the plain form
// cost about 25 VALU operations per value, which made the kernel VALU-bound.
GDN_DEV float silu_fast(float t) {
    constexpr float kLog2e = 1.4426950408889634f;
    return t * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-t * kLog2e));
}

// ---------------------------------------------------------------------------
// Gating prologue (HF transformers modeling_qwen3_5.py, Qwen3_5GatedDeltaNet.
// forward:481-502 and l2norm:242-245).  One block per token: its conv output
// row holds H = 2 Hk + Hv heads of 128 channels (q heads, k heads, v heads);
// 16-lane group s takes heads s, s + 16, ...  q and k heads are scaled by
// 1 / sqrt(sum x^2 + 1e-6); v heads are copied.  Threads h < Hv also form the
// gates of value head h:
//   g = -exp(A_log) softplus(a + dt_bias)   (softplus(y) = y > 20 ? y : log1p(exp(y)))
//   beta = 1 / (1 + exp(-b))
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(kThreads) void gating_prologue_kernel(
    const float *__restrict__ x, const float *__restrict__ a, const float *__restrict__ b,
    const float *__restrict__ A_log, const float *__restrict__ dt_bias, OutT *__restrict__ q,
    OutT *__restrict__ k, OutT *__restrict__ v, float *__restrict__ g, float *__restrict__ beta,
    int Hk, int Hv) {
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 15, grp = tid >> 4;
    const int H = 2 * Hk + Hv;
    const float *xr = x + row * (size_t)H * D + 8 * lane;
    for (int h0 = 0; h0 < H; h0 += kGroups * kPass) {
        V8 xv[kPass];
#pragma unroll
        for (int j = 0; j < kPass; ++j) {
            const int h = h0 + grp + kGroups * j;
            if (h < H) xv[j] = load8(xr + (size_t)h * D);
        }
#pragma unroll
        for (int j = 0; j < kPass; ++j) {
            const int h = h0 + grp + kGroups * j;  // uniform over the group
            if (h >= H) break;
            V8 y = xv[j];
            OutT *dst;
            if (h < 2 * Hk) {
                const float inv = 1.0f / sqrtf(group_sum(sumsq8(y)) + 1e-6f);
#pragma unroll
                for (int i = 0; i < 8; ++i) y.f[i] *= inv;
                dst = h < Hk ? q + (row * Hk + h) * D : k + (row * Hk + (h - Hk)) * D;
            } else {
                dst = v + (row * Hv + (h - 2 * Hk)) * D;
            }
            store8(dst + 8 * lane, y);
        }
    }
    for (int h = tid; h < Hv; h += kThreads) {
        const size_t i = row * Hv + h;
        const float y = a[i] + dt_bias[h];
        const float sp = y > 20.f ? y : log1pf(expf(y));
        g[i] = -expf(A_log[h]) * sp;
        beta[i] = 1.0f / (1.0f + expf(-b[i]));
    }
}

// ---------------------------------------------------------------------------
// The causal conv (K = 4, SiLU) of a prompt's rows fused with the gating
// prologue, so that the conv's fp32 output never reaches HBM.  Block (row
// segment of kConvRows rows, 16 heads): 16-lane group s takes head
// 16 blockIdx.y + s, lane l its channels 8l .. 8l+7, for every row of the
// segment in order, with the three previous inputs in registers (from the
// rows before the segment, or from `hist` for the first).  Each value is
// conv_k4_kernel's (the same tap sum in the same order, no contraction, and
// its SiLU), and each head row then gets gating_prologue_kernel's arithmetic,
// so q, k, v, g and beta are bit for bit those of the two kernels in turn.
// The block of head group 0 also forms the segment's gates.
// ---------------------------------------------------------------------------
constexpr int kConvRows = 64;  // rows per block
constexpr int kConvU = 4;      // rows in flight per lane

GDN_DEV float conv_silu(float h0, float h1, float h2, float cur, float w0, float w1, float w2, float w3) {
#pragma clang fp contract(off)
    const float acc = h0 * w0 + h1 * w1 + h2 * w2 + cur * w3;
    return acc / (1.0f + expf(-acc));
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void conv_gating_kernel(
    const float *__restrict__ x, const float *__restrict__ wt, const float *__restrict__ hist,
    const float *__restrict__ a, const float *__restrict__ b, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, OutT *__restrict__ q, OutT *__restrict__ k, OutT *__restrict__ v,
    float *__restrict__ g, float *__restrict__ beta, int64_t T, int Hk, int Hv) {
    const int tid = threadIdx.x, lane = tid & 15, grp = tid >> 4;
    const int H = 2 * Hk + Hv;
    const int64_t C = (int64_t)H * D;
    const int h = blockIdx.y * kGroups + grp;  // uniform over the group
    const int64_t t0 = (int64_t)blockIdx.x * kConvRows, t1 = min(T, t0 + kConvRows);
    if (h < H) {
        const int64_t c = (int64_t)h * D + 8 * lane;
        V8 w[4], hh[3];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = load8(wt + j * C + c);
#pragma unroll
        for (int j = 0; j < 3; ++j) hh[j] = t0 == 0 ? load8(hist + j * C + c) : load8(x + (t0 - 3 + j) * C + c);
        OutT *dst;
        int64_t ld;
        if (h < Hk) {
            dst = q + (int64_t)h * D;
            ld = (int64_t)Hk * D;
        } else if (h < 2 * Hk) {
            dst = k + (int64_t)(h - Hk) * D;
            ld = (int64_t)Hk * D;
        } else {
            dst = v + (int64_t)(h - 2 * Hk) * D;
            ld = (int64_t)Hv * D;
        }
        for (int64_t t = t0; t < t1; t += kConvU) {
            // unconditional loads (rows past the end clamp to the last row and
            // are not used), so the kConvU rows issue back to back
            V8 cur[kConvU];
#pragma unroll
            for (int i = 0; i < kConvU; ++i) cur[i] = load8(x + min(t + i, T - 1) * C + c);
#pragma unroll
            for (int i = 0; i < kConvU; ++i) {
                if (t + i >= t1) break;  // uniform over the block
                V8 y;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    y.f[e] = conv_silu(hh[0].f[e], hh[1].f[e], hh[2].f[e], cur[i].f[e], w[0].f[e], w[1].f[e],
                                       w[2].f[e], w[3].f[e]);
                hh[0] = hh[1];
                hh[1] = hh[2];
                hh[2] = cur[i];
                if (h < 2 * Hk) {
                    const float inv = 1.0f / sqrtf(group_sum(sumsq8(y)) + 1e-6f);
#pragma unroll
                    for (int e = 0; e < 8; ++e) y.f[e] *= inv;
                }
                store8(dst + (t + i) * ld + 8 * lane, y);
            }
        }
    }
    if (blockIdx.y == 0) {
        const int64_t n = (t1 - t0) * Hv;
        for (int64_t i0 = tid; i0 < n; i0 += kThreads) {
            const int64_t i = t0 * Hv + i0;
            const int hv = (int)(i0 % Hv);
            const float y = a[i] + dt_bias[hv];
            const float sp = y > 20.f ? y : log1pf(expf(y));
            g[i] = -expf(A_log[hv]) * sp;
            beta[i] = 1.0f / (1.0f + expf(-b[i]));
        }
    }
}

// ---------------------------------------------------------------------------
// Gated RMSNorm with the SiLU gate (HF Qwen3_5RMSNormGated.forward,
// modeling_qwen3_5.py:175-184) over rows of 128 values; 16-lane group s of
// block B takes rows 16 NP B + s + 16 j, j < NP.
//   fp32: y = (w * (o / sqrt(mean(o^2) + eps))) * silu(z)
//   bf16: h = bf16(o / sqrt(mean(o^2) + eps)); h = bf16(w * h);
//         y = bf16(h * silu(z))      (HF's roundings in a bf16 model)
// silu(z) = z / (1 + exp(-z)) in fp32 (hardware exp2 and reciprocal).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(
    const T *__restrict__ o, const T *__restrict__ z, const T *__restrict__ w, T *__restrict__ y,
    size_t rows, float eps) {
    constexpr bool kBF16 = sizeof(T) == 2;
    const int tid = threadIdx.x, lane = tid & 15, grp = tid >> 4;
    constexpr int NP = kRowsPass<T>;
    const size_t r0 = (size_t)blockIdx.x * (kGroups * NP) + grp;
    const V8 wv = unpack(load_raw(w + 8 * lane));
    decltype(load_raw(o)) ov[NP], zv[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const size_t r = r0 + kGroups * j;
        if (r < rows) {
            ov[j] = load_raw(o + r * D + 8 * lane);
            zv[j] = load_raw(z + r * D + 8 * lane);
        }
    }
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const size_t r = r0 + kGroups * j;  // uniform over the group
        if (r >= rows) break;
        const V8 x = unpack(ov[j]), s = unpack(zv[j]);
        const float inv = 1.0f / sqrtf(group_sum(sumsq8(x)) / (float)D + eps);
        V8 out;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (kBF16)
                out.f[i] = round_bf16(wv.f[i] * round_bf16(x.f[i] * inv)) * silu_fast(s.f[i]);
            else
                out.f[i] = (wv.f[i] * (x.f[i] * inv)) * silu_fast(s.f[i]);
        }
        store8(y + r * D + 8 * lane, out);
    }
}

}  // namespace

hipError_t launch_gating_prologue(bool bf16, const float *x, const float *a, const float *b,
                                  const float *A_log, const float *dt_bias, void *q, void *k,
                                  void *v, float *g, float *beta, size_t rows, int Hk, int Hv,
                                  hipStream_t st) {
    if (rows == 0) return hipSuccess;
    if (rows > 0x7FFFFFFFu) return hipErrorInvalidValue;
    const dim3 grid((unsigned)rows);
    if (bf16)
        gating_prologue_kernel<uint16_t><<<grid, kThreads, 0, st>>>(
            x, a, b, A_log, dt_bias, static_cast<uint16_t *>(q), static_cast<uint16_t *>(k),
            static_cast<uint16_t *>(v), g, beta, Hk, Hv);
    else
        gating_prologue_kernel<float><<<grid, kThreads, 0, st>>>(
            x, a, b, A_log, dt_bias, static_cast<float *>(q), static_cast<float *>(k),
            static_cast<float *>(v), g, beta, Hk, Hv);
    return hipGetLastError();
}

hipError_t launch_conv_gating(const float *x, const float *conv_wt, const float *hist, const float *a,
                              const float *b, const float *A_log, const float *dt_bias, uint16_t *q, uint16_t *k,
                              uint16_t *v, float *g, float *beta, int64_t T, int Hk, int Hv, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (Hk <= 0 || Hv <= 0) return hipErrorInvalidValue;
    const int H = 2 * Hk + Hv;
    const dim3 grid((unsigned)((T + kConvRows - 1) / kConvRows), (unsigned)((H + kGroups - 1) / kGroups));
    conv_gating_kernel<uint16_t><<<grid, kThreads, 0, st>>>(x, conv_wt, hist, a, b, A_log, dt_bias, q, k, v, g, beta,
                                                            T, Hk, Hv);
    return hipGetLastError();
}

hipError_t launch_gated_rmsnorm(bool bf16, const void *o, const void *z, const void *w, void *y,
                                size_t rows, float eps, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const size_t per_block = (size_t)kGroups * (bf16 ? kRowsPass<uint16_t> : kRowsPass<float>);
    const size_t blocks = (rows + per_block - 1) / per_block;
    if (blocks > 0x7FFFFFFFu) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
    if (bf16)
        gated_rmsnorm_kernel<uint16_t><<<grid, kThreads, 0, st>>>(
            static_cast<const uint16_t *>(o), static_cast<const uint16_t *>(z),
            static_cast<const uint16_t *>(w), static_cast<uint16_t *>(y), rows, eps);
    else
        gated_rmsnorm_kernel<float><<<grid, kThreads, 0, st>>>(
            static_cast<const float *>(o), static_cast<const float *>(z),
            static_cast<const float *>(w), static_cast<float *>(y), rows, eps);
    return hipGetLastError();
}

}  // namespace gdn

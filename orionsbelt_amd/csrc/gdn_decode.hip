// gdn_decode.hip -- single-token matrix-state gated delta rule for gfx950.
//
// Semantics: the OpenCL gdn_delta_rule_decode (gpu/gdn_gpu_kernels.cl:158-206)
// and its host oracle ref_delta_rule (gpu/gdn_gpu_validate.c:100-118), with
// per-(sequence, value-head) decay exp(g) and beta and a q scale, as HF
// torch_recurrent_gated_delta_rule runs one step (modeling_qwen3_5.py:364-375).
//
// Mapping: one workgroup per (sequence, value head); the 128x128 fp32 state
// (64 KiB) is read from HBM once into registers, decayed, updated and written
// back once -- the step moves 2 x 64 KiB per head and is HBM-bound (about
// 0.9 FLOP per byte), so it uses plain FMAs, no MFMA.  256 threads: thread
// (rg, cg) owns 4 consecutive value columns (one float4) of rows rg, rg+RG,
// ...; a wavefront reads whole rows, 1 KiB contiguous per load instruction.
// The two column reductions (k^T S and q^T S over the key dimension) are
// per-thread partial sums over its rows followed by a reduction across the
// RG row groups in LDS.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

// State I/O.  NT selects non-temporal loads and stores: the state is touched
// once per step, so it need not be kept in L2 or the Infinity Cache.
template <int NARROW, bool NT> struct StateIO;
template <bool NT> struct StateIO<kF32, NT> {
    static GDN_DEV float4 load(const void *S, int64_t i) {
        return load_f4<NT>(static_cast<const float *>(S) + i);
    }
    static GDN_DEV void store(void *S, int64_t i, float4 v) {
        store_f4<NT>(static_cast<float *>(S) + i, v);
    }
};
template <bool NT> struct StateIO<kF16, NT> {
    static GDN_DEV float4 load(const void *S, int64_t i) {
        const u32x2_t u = load_u2<NT>(static_cast<const uint16_t *>(S) + i);
        return make_float4(f16_to_f32((uint16_t)(u[0] & 0xFFFF)), f16_to_f32((uint16_t)(u[0] >> 16)),
                           f16_to_f32((uint16_t)(u[1] & 0xFFFF)), f16_to_f32((uint16_t)(u[1] >> 16)));
    }
    static GDN_DEV void store(void *S, int64_t i, float4 v) {
        u32x2_t u;
        u[0] = (uint32_t)f32_to_f16_rne(v.x) | ((uint32_t)f32_to_f16_rne(v.y) << 16);
        u[1] = (uint32_t)f32_to_f16_rne(v.z) | ((uint32_t)f32_to_f16_rne(v.w) << 16);
        store_u2<NT>(static_cast<uint16_t *>(S) + i, u);
    }
};

GDN_DEV float4 f4_fma(float a, float4 b, float4 c) {
    return make_float4(fmaf(a, b.x, c.x), fmaf(a, b.y, c.y), fmaf(a, b.z, c.z), fmaf(a, b.w, c.w));
}
GDN_DEV float4 f4_add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// MINW: minimum waves per SIMD the register allocation must allow.
// NT:   non-temporal state traffic.
// CS:   column splits -- CS workgroups per (sequence, head), each owning
//       DV/CS value columns (the update of column j reads only column j).
template <int DK, int DV, int NARROW, int MINW, bool NT, int CS>
__global__ __launch_bounds__(256, MINW) void delta_decode_kernel(
    void *S, const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ g, const float *__restrict__ beta,
    float *__restrict__ o, int Hv, int Hk, float q_scale) {
    constexpr int TPR = DV / CS / 4;   // threads per state row (segment)
    constexpr int RG = 256 / TPR;      // row groups
    constexpr int RPT = DK / RG;       // rows per thread
    static_assert(TPR >= 1 && RPT >= 1 && DK % RG == 0, "unsupported head shape");
    __shared__ float4 red[RG][TPR];

    const int bh = blockIdx.x / CS;
    const int b = bh / Hv, h = bh % Hv;
    const int kh = h / (Hv / Hk);
    const int cgi = threadIdx.x % TPR;
    const int rg = threadIdx.x / TPR;
    const int c = (blockIdx.x % CS) * (DV / CS) + cgi * 4;
    const int64_t sbase = (int64_t)bh * DK * DV;
    const float *kp = k + ((int64_t)b * Hk + kh) * DK;
    const float *qp = q + ((int64_t)b * Hk + kh) * DK;

    float4 s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = StateIO<NARROW, NT>::load(S, sbase + (int64_t)(rg + RG * i) * DV + c);
    float kj[RPT], qj[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        kj[i] = kp[rg + RG * i];
        qj[i] = qp[rg + RG * i] * q_scale;
    }
    const float decay = expf(g[bh]);
    const float bt = beta[bh];
    const float4 vv = *reinterpret_cast<const float4 *>(v + (int64_t)bh * DV + c);

    // S *= decay ; partial kv = sum_rows S[j][c] k[j]
    float4 kv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        s[i] = make_float4(s[i].x * decay, s[i].y * decay, s[i].z * decay, s[i].w * decay);
        kv = f4_fma(kj[i], s[i], kv);
    }
    red[rg][cgi] = kv;
    __syncthreads();
    kv = red[0][cgi];
#pragma unroll
    for (int r = 1; r < RG; ++r) kv = f4_add(kv, red[r][cgi]);
    const float4 delta = make_float4((vv.x - kv.x) * bt, (vv.y - kv.y) * bt,
                                     (vv.z - kv.z) * bt, (vv.w - kv.w) * bt);

    // S += k (x) delta ; store S ; partial o = sum_rows S[j][c] q[j]
    float4 op = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        s[i] = f4_fma(kj[i], delta, s[i]);
        StateIO<NARROW, NT>::store(S, sbase + (int64_t)(rg + RG * i) * DV + c, s[i]);
        op = f4_fma(qj[i], s[i], op);
    }
    __syncthreads();  // everyone has read red[] for kv
    red[rg][cgi] = op;
    __syncthreads();
    if (rg == 0) {
        float4 acc = red[0][cgi];
#pragma unroll
        for (int r = 1; r < RG; ++r) acc = f4_add(acc, red[r][cgi]);
        *reinterpret_cast<float4 *>(o + (int64_t)bh * DV + c) = acc;
    }
}

}  // namespace

// Production configuration of the decode kernel, measured on MI355X over 24
// rotating 128 MiB states (B=64, 32 heads, 128x128): 2 column splits with
// non-temporal state traffic run 47.1 us per layer (5.77 TB/s) against
// 55.4 us for one workgroup per head with cached traffic.
constexpr int kDecodeMinW = 1;
constexpr bool kDecodeNT = true;
constexpr int kDecodeCS = 2;

template <int NARROW, int MINW, bool NT, int CS>
hipError_t launch_decode_cfg(void *S, const float *q, const float *k, const float *v,
                             const float *g, const float *beta, float *o, int B, int Hv, int Hk,
                             int dk, int dv, float q_scale, hipStream_t st) {
#define GDN_DEC(DK, DV)                                                                      \
    if (dk == DK && dv == DV) {                                                              \
        constexpr int cs = (CS * 1024 <= DK * DV && DV / CS >= 4) ? CS : 1;                  \
        dim3 grid((unsigned)(B * Hv * cs)), block(256);                                      \
        delta_decode_kernel<DK, DV, NARROW, MINW, NT, cs><<<grid, block, 0, st>>>(            \
            S, q, k, v, g, beta, o, Hv, Hk, q_scale);                                        \
        return hipGetLastError();                                                            \
    }
    GDN_DEC(128, 128)
    GDN_DEC(64, 64)
    GDN_DEC(32, 32)
    GDN_DEC(128, 64)
    GDN_DEC(64, 128)
    GDN_DEC(128, 32)
    GDN_DEC(32, 128)
    GDN_DEC(64, 32)
    GDN_DEC(32, 64)
#undef GDN_DEC
    return hipErrorInvalidValue;
}

hipError_t launch_delta_decode(int narrow_state, void *S, const float *q, const float *k,
                               const float *v, const float *g, const float *beta, float *o,
                               int B, int Hv, int Hk, int dk, int dv, float q_scale,
                               hipStream_t st) {
    if (B <= 0 || Hv <= 0) return hipSuccess;
    if (narrow_state == kF32)
        return launch_decode_cfg<kF32, kDecodeMinW, kDecodeNT, kDecodeCS>(
            S, q, k, v, g, beta, o, B, Hv, Hk, dk, dv, q_scale, st);
    if (narrow_state == kF16)
        return launch_decode_cfg<kF16, kDecodeMinW, kDecodeNT, kDecodeCS>(
            S, q, k, v, g, beta, o, B, Hv, Hk, dk, dv, q_scale, st);
    return hipErrorInvalidValue;
}

}  // namespace gdn

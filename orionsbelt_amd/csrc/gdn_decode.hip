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
#include <type_traits>

#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

// State I/O of V consecutive value columns.  NT selects non-temporal loads
// and stores: the state is touched once per step, so it need not be kept in
// L2 or the Infinity Cache.  fp32 moves 4 columns (16 bytes) per lane; fp16
// 4 (8 bytes) or 8 (16 bytes).
template <int NARROW, bool NT, int V> struct StateIO;
template <bool NT> struct StateIO<kF32, NT, 4> {
    typedef float4 Raw;
    static GDN_DEV Raw load_raw(const void *S, int64_t i) {
        return load_f4<NT>(static_cast<const float *>(S) + i);
    }
    static GDN_DEV void unpack(Raw v, float (&x)[4]) {
        x[0] = v.x;
        x[1] = v.y;
        x[2] = v.z;
        x[3] = v.w;
    }
    static GDN_DEV void load(const void *S, int64_t i, float (&x)[4]) { unpack(load_raw(S, i), x); }
    static GDN_DEV void store(void *S, int64_t i, const float (&x)[4]) {
        store_f4<NT>(static_cast<float *>(S) + i, make_float4(x[0], x[1], x[2], x[3]));
    }
};
template <bool NT, int V> struct StateIO<kF16, NT, V> {
    static_assert(V == 4 || V == 8, "fp16 state: 4 or 8 columns per lane");
    static constexpr int W = V / 2;  // 32-bit words
    typedef std::conditional_t<V == 8, u32x4_t, u32x2_t> Vec;
    typedef Vec Raw;
    static GDN_DEV Raw load_raw(const void *S, int64_t i) {
        if constexpr (V == 8) return load_u4<NT>(static_cast<const uint16_t *>(S) + i);
        else return load_u2<NT>(static_cast<const uint16_t *>(S) + i);
    }
    static GDN_DEV void unpack(Raw u, float (&x)[V]) {
#pragma unroll
        for (int j = 0; j < W; ++j) {
            x[2 * j] = f16_to_f32((uint16_t)(u[j] & 0xFFFF));
            x[2 * j + 1] = f16_to_f32((uint16_t)(u[j] >> 16));
        }
    }
    static GDN_DEV void load(const void *S, int64_t i, float (&x)[V]) { unpack(load_raw(S, i), x); }
    static GDN_DEV void store(void *S, int64_t i, const float (&x)[V]) {
        Vec u;
#pragma unroll
        for (int j = 0; j < W; ++j)
            u[j] = (uint32_t)f32_to_f16_rne(x[2 * j]) | ((uint32_t)f32_to_f16_rne(x[2 * j + 1]) << 16);
        if constexpr (V == 8) store_u4<NT>(static_cast<uint16_t *>(S) + i, u);
        else store_u2<NT>(static_cast<uint16_t *>(S) + i, u);
    }
};

GDN_DEV float4 f4_fma(float a, float4 b, float4 c) {
    return make_float4(fmaf(a, b.x, c.x), fmaf(a, b.y, c.y), fmaf(a, b.z, c.z), fmaf(a, b.w, c.w));
}
GDN_DEV float4 f4_add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Sum of acc over the row groups of the workgroup, for this thread's V
// columns (the lanes rg * TPR + cgi of every wave hold the same columns).
// SHFL: first within each wave by lane exchanges (xor TPR, 2 TPR, ... 32),
// then the 4 wave sums in LDS, in wave order; otherwise every row group's
// partial goes through LDS and each thread adds them in row-group order.
// ALL: every thread receives the sum; otherwise only row group 0 does.
template <int TPR, int RG, int V, bool SHFL, bool ALL>
GDN_DEV void row_group_sum(float (&acc)[V], float *red, int rg, int cgi) {
    if constexpr (SHFL) {
        constexpr int W = 4;  // waves
#pragma unroll
        for (int m = TPR; m < 64; m <<= 1)
#pragma unroll
            for (int j = 0; j < V; ++j) acc[j] += __shfl_xor(acc[j], m);
        const int wave = (int)threadIdx.x >> 6;
        if (((int)threadIdx.x & 63) < TPR)
#pragma unroll
            for (int j = 0; j < V; ++j) red[(wave * TPR + cgi) * V + j] = acc[j];
        __syncthreads();
        if (!ALL && rg != 0) return;
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] = red[cgi * V + j];
#pragma unroll
        for (int w = 1; w < W; ++w)
#pragma unroll
            for (int j = 0; j < V; ++j) acc[j] += red[(w * TPR + cgi) * V + j];
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j) red[(rg * TPR + cgi) * V + j] = acc[j];
        __syncthreads();
        if (!ALL && rg != 0) return;
#pragma unroll
        for (int j = 0; j < V; ++j) acc[j] = red[cgi * V + j];
#pragma unroll
        for (int r = 1; r < RG; ++r)
#pragma unroll
            for (int j = 0; j < V; ++j) acc[j] += red[(r * TPR + cgi) * V + j];
    }
}

// MINW: minimum waves per SIMD the register allocation must allow.
// NT:   non-temporal state traffic.
// CS:   column splits -- CS workgroups per (sequence, head), each owning
//       DV/CS value columns (the update of column j reads only column j).
// SHFL: row-group reduction through lane exchanges first (row_group_sum).
// V:    value columns per thread (StateIO).
template <int DK, int DV, int NARROW, int V, int MINW, bool NT, int CS, bool SHFL>
__global__ __launch_bounds__(256, MINW) void delta_decode_kernel(
    void *S, const float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ g, const float *__restrict__ beta,
    float *__restrict__ o, int Hv, int Hk, float q_scale) {
    using IO = StateIO<NARROW, NT, V>;
    constexpr int TPR = DV / CS / V;   // threads per state row (segment)
    constexpr int RG = 256 / TPR;      // row groups
    constexpr int RPT = DK / RG;       // rows per thread
    static_assert(TPR >= 1 && RPT >= 1 && DK % RG == 0 && 64 % TPR == 0, "unsupported head shape");
    __shared__ float red[(SHFL ? 4 : RG) * TPR * V];

    const int bh = blockIdx.x / CS;
    const int b = bh / Hv, h = bh % Hv;
    const int kh = h / (Hv / Hk);
    const int cgi = threadIdx.x % TPR;
    const int rg = threadIdx.x / TPR;
    const int c = (blockIdx.x % CS) * (DV / CS) + cgi * V;
    const int64_t sbase = (int64_t)bh * DK * DV;
    const float *kp = k + ((int64_t)b * Hk + kh) * DK;
    const float *qp = q + ((int64_t)b * Hk + kh) * DK;

    float s[RPT][V];
#pragma unroll
    for (int i = 0; i < RPT; ++i) IO::load(S, sbase + (int64_t)(rg + RG * i) * DV + c, s[i]);
    float kj[RPT], qj[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        kj[i] = kp[rg + RG * i];
        qj[i] = qp[rg + RG * i] * q_scale;
    }
    const float decay = expf(g[bh]);
    const float bt = beta[bh];
    float vv[V];
#pragma unroll
    for (int j = 0; j < V; j += 4) {
        const float4 t = *reinterpret_cast<const float4 *>(v + (int64_t)bh * DV + c + j);
        vv[j] = t.x;
        vv[j + 1] = t.y;
        vv[j + 2] = t.z;
        vv[j + 3] = t.w;
    }

    // S *= decay ; partial kv = sum_rows S[j][c] k[j]
    float kv[V];
#pragma unroll
    for (int j = 0; j < V; ++j) kv[j] = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int j = 0; j < V; ++j) {
            s[i][j] = s[i][j] * decay;
            kv[j] = fmaf(kj[i], s[i][j], kv[j]);
        }
    row_group_sum<TPR, RG, V, SHFL, true>(kv, red, rg, cgi);
    float delta[V];
#pragma unroll
    for (int j = 0; j < V; ++j) delta[j] = (vv[j] - kv[j]) * bt;

    // S += k (x) delta ; store S ; partial o = sum_rows S[j][c] q[j]
    float op[V];
#pragma unroll
    for (int j = 0; j < V; ++j) op[j] = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
        for (int j = 0; j < V; ++j) s[i][j] = fmaf(kj[i], delta[j], s[i][j]);
        IO::store(S, sbase + (int64_t)(rg + RG * i) * DV + c, s[i]);
#pragma unroll
        for (int j = 0; j < V; ++j) op[j] = fmaf(qj[i], s[i][j], op[j]);
    }
    __syncthreads();  // everyone has read red[] for kv
    row_group_sum<TPR, RG, V, SHFL, false>(op, red, rg, cgi);
    if (rg == 0) {
#pragma unroll
        for (int j = 0; j < V; j += 4)
            *reinterpret_cast<float4 *>(o + (int64_t)bh * DV + c + j) =
                make_float4(op[j], op[j + 1], op[j + 2], op[j + 3]);
    }
}

// One GDN layer's decode step after its in-projection, fused for the hybrid
// loop: block (sequence b, value head h), 256 threads, fp32 state, d = 128.
//   1. the conv update on HF's cache with SiLU (conv_update_kernel's
//      arithmetic) for the block's 384 channels: q and k of key head
//      kh = h / (Hv / Hk), v of head h.  The cache is read from conv_in and
//      the shifted cache written to conv_out (a different array: the value
//      heads that share a key head all read its q/k state); the first value
//      head of a key head writes the q/k entries, every head its v entries;
//   2. q, k L2-normalised (eps 1e-6), q scaled; g = -exp(A_log) *
//      softplus(a + dt_bias), beta = sigmoid(b) (the gating prologue);
//   3. the delta-rule step of delta_decode_kernel with one block owning all
//      128 value columns;
//   4. the gated RMSNorm of the output row with z (weight w [128]) and the
//      fp16 rounding the out-projection reads: out16[b][h * 128 + c].
// x holds the in-projection's qkv rows [B][(2 Hk + Hv) * 128].
__global__ __launch_bounds__(256) void gdn_step_fused_kernel(
    const float *__restrict__ x, const float *__restrict__ conv_in, float *__restrict__ conv_out,
    const float *__restrict__ conv_w, const float *__restrict__ a_in, const float *__restrict__ b_in,
    const float *__restrict__ A_log, const float *__restrict__ dt_bias, float *__restrict__ S,
    const float *__restrict__ z, const float *__restrict__ norm_w, uint16_t *__restrict__ out16, int Hk, int Hv,
    float q_scale, float eps) {
#pragma clang fp contract(off)
    constexpr int D = 128, TPR = 32, RG = 8, RPT = 16;
    __shared__ float qs[D], ks[D], vs[D];
    __shared__ float red_ss[4];
    __shared__ float gate[2];
    __shared__ float4 red[RG][TPR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bh = blockIdx.x;
    const int b = bh / Hv, h = bh % Hv;
    const int rep = Hv / Hk, kh = h / rep;
    const int64_t C = (int64_t)(2 * Hk + Hv) * D;
    const int cgi = tid % TPR, rg = tid / TPR;
    const int c = cgi * 4;
    const int64_t sbase = (int64_t)bh * D * D;
    // Loads in the order they are needed (vector loads complete in issue
    // order): the conv inputs and gate scalars, the epilogue's z and norm
    // weight (row group 0), then the 64 KB state, which streams in while the
    // conv, the norms and the gates are formed.
    // 1. conv + SiLU: thread t < 128 takes q channel t and v channel t,
    //    thread t >= 128 k channel t - 128
    struct ConvIn {
        float4 st, wv;
        float cur;
    };
    auto conv_load = [&](int64_t ch) {
        const int64_t si = ((int64_t)b * C + ch) * 4;
        return ConvIn{*reinterpret_cast<const float4 *>(conv_in + si), *reinterpret_cast<const float4 *>(conv_w + ch * 4),
                      x[(int64_t)b * C + ch]};
    };
    auto conv = [&](int64_t ch, const ConvIn &in, bool write) {
        const int64_t si = ((int64_t)b * C + ch) * 4;
        float acc = in.st.y * in.wv.x + in.st.z * in.wv.y + in.st.w * in.wv.z + in.cur * in.wv.w;
        acc = acc / (1.0f + expf(-acc));
        if (write) *reinterpret_cast<float4 *>(conv_out + si) = make_float4(in.st.y, in.st.z, in.st.w, in.cur);
        return acc;
    };
    const bool qk_writer = h % rep == 0;
    const int64_t ch0 = tid < D ? (int64_t)kh * D + tid : (int64_t)Hk * D + (int64_t)kh * D + (tid - D);
    const int64_t chv = (int64_t)2 * Hk * D + (int64_t)h * D + (tid & (D - 1));
    const ConvIn in0 = conv_load(ch0);
    ConvIn inv_;
    if (tid < D) inv_ = conv_load(chv);
    float ga = 0.f, gb = 0.f, gA = 0.f, gdt = 0.f;
    if (tid == 0) {
        ga = a_in[bh];
        gdt = dt_bias[h];
        gA = A_log[h];
        gb = b_in[bh];
    }
    float4 zz = make_float4(0.f, 0.f, 0.f, 0.f), ww = zz;
    if (rg == 0) {
        zz = *reinterpret_cast<const float4 *>(z + (int64_t)bh * D + c);
        ww = *reinterpret_cast<const float4 *>(norm_w + c);
    }
    float4 s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = load_f4<true>(S + sbase + (int64_t)(rg + RG * i) * D + c);

    float mine;
    if (tid < D) {
        mine = conv(ch0, in0, qk_writer);
        vs[tid] = conv(chv, inv_, true);
    } else {
        mine = conv(ch0, in0, qk_writer);
    }
    // 2. L2 norms (q: waves 0-1, k: waves 2-3) and the gates
    float ss = mine * mine;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) red_ss[wave] = ss;
    if (tid == 0) {
        const float y = ga + gdt;
        const float sp = y > 20.f ? y : log1pf(expf(y));
        gate[0] = -expf(gA) * sp;
        gate[1] = 1.0f / (1.0f + expf(-gb));
    }
    __syncthreads();
    if (tid < D) qs[tid] = mine * (1.0f / sqrtf(red_ss[0] + red_ss[1] + 1e-6f)) * q_scale;
    else ks[tid - D] = mine * (1.0f / sqrtf(red_ss[2] + red_ss[3] + 1e-6f));
    __syncthreads();

    // 3. the delta-rule step (delta_decode_kernel, one block per head)
    float kj[RPT], qj[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        kj[i] = ks[rg + RG * i];
        qj[i] = qs[rg + RG * i];
    }
    const float decay = expf(gate[0]);
    const float bt = gate[1];
    const float4 vv = *reinterpret_cast<const float4 *>(vs + c);
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
    const float4 delta = make_float4((vv.x - kv.x) * bt, (vv.y - kv.y) * bt, (vv.z - kv.z) * bt, (vv.w - kv.w) * bt);
    float4 op = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        s[i] = f4_fma(kj[i], delta, s[i]);
        store_f4<true>(S + sbase + (int64_t)(rg + RG * i) * D + c, s[i]);
        op = f4_fma(qj[i], s[i], op);
    }
    __syncthreads();
    red[rg][cgi] = op;
    __syncthreads();
    if (rg != 0) return;
    // 4. gated RMSNorm over the row (threads 0..31 of wave 0, 4 columns each)
    float4 o4 = red[0][cgi];
#pragma unroll
    for (int r = 1; r < RG; ++r) o4 = f4_add(o4, red[r][cgi]);
    float q2 = o4.x * o4.x + o4.y * o4.y + o4.z * o4.z + o4.w * o4.w;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) q2 += __shfl_xor(q2, o, 32);
    const float inv = 1.0f / sqrtf(q2 / (float)D + eps);
    auto gn = [&](float ov, float zv, float wv) { return (wv * (ov * inv)) * (zv / (1.0f + expf(-zv))); };
    uint2 o;
    o.x = (uint32_t)f32_to_f16_rne(gn(o4.x, zz.x, ww.x)) | ((uint32_t)f32_to_f16_rne(gn(o4.y, zz.y, ww.y)) << 16);
    o.y = (uint32_t)f32_to_f16_rne(gn(o4.z, zz.z, ww.z)) | ((uint32_t)f32_to_f16_rne(gn(o4.w, zz.w, ww.w)) << 16);
    *reinterpret_cast<uint2 *>(out16 + (int64_t)bh * D + c) = o;
}

}  // namespace

hipError_t launch_gdn_step_fused(const float *x, const float *conv_in, float *conv_out, const float *conv_w,
                                 const float *a, const float *b, const float *A_log, const float *dt_bias, float *S,
                                 const float *z, const float *norm_w, uint16_t *out16, int B, int Hk, int Hv,
                                 float q_scale, float eps, hipStream_t st) {
    if (B <= 0) return hipSuccess;
    if (Hk <= 0 || Hv % Hk != 0 || conv_in == conv_out) return hipErrorInvalidValue;
    gdn_step_fused_kernel<<<dim3((unsigned)(B * Hv)), 256, 0, st>>>(x, conv_in, conv_out, conv_w, a, b, A_log,
                                                                    dt_bias, S, z, norm_w, out16, Hk, Hv, q_scale,
                                                                    eps);
    return hipGetLastError();
}

// Production configuration of the decode kernel, measured on MI355X over 24
// rotating states (B=64, 32 heads, 128x128):
//  * fp32 state: 2 column splits with non-temporal state traffic, 47.1 us
//    per layer (5.77 TB/s) against 55.4 us for one workgroup per head with
//    cached traffic; lane exchanges in the reductions change nothing
//    measurable (46.48 against 46.56 us), so the LDS reduction stays.
//  * fp16 state: 2 column splits, lane exchanges first, 24.4 us (5.6 TB/s)
//    against 24.9 us with the LDS reduction alone.  Rejected: 8 columns per
//    lane (16-byte accesses, 29.0 us), one or four workgroups per head
//    (25.7 / 38.8 us), and a persistent form that loads the next head's
//    state while it works on the current one (27-32 us; fp32 48-52 us).
constexpr int kDecodeMinW = 1;
constexpr bool kDecodeNT = true;
template <int NARROW> struct DecodeCfg;
template <> struct DecodeCfg<kF32> { static constexpr int CS = 2; static constexpr bool SHFL = false; };
template <> struct DecodeCfg<kF16> { static constexpr int CS = 2; static constexpr bool SHFL = true; };

template <int NARROW>
hipError_t launch_decode_cfg(void *S, const float *q, const float *k, const float *v,
                             const float *g, const float *beta, float *o, int B, int Hv, int Hk,
                             int dk, int dv, float q_scale, hipStream_t st) {
    constexpr int CS = DecodeCfg<NARROW>::CS;
    constexpr bool SHFL = DecodeCfg<NARROW>::SHFL;
    // fits(DK, DV, cs, vec): at least 4 threads per row, row groups <= rows
#define GDN_FITS(DK, DV, cs, vec) ((DV) / (cs) / (vec) >= 4 && 256 / ((DV) / (cs) / (vec)) <= (DK))
#define GDN_DEC(DK, DV)                                                                      \
    if (dk == DK && dv == DV) {                                                              \
        constexpr int vec = 4;                                                               \
        constexpr int cs = GDN_FITS(DK, DV, CS, vec) ? CS : 1;                               \
        static_assert(GDN_FITS(DK, DV, cs, vec), "decode shape");                            \
        dim3 grid((unsigned)(B * Hv * cs)), block(256);                                      \
        delta_decode_kernel<DK, DV, NARROW, vec, kDecodeMinW, kDecodeNT, cs, SHFL>           \
            <<<grid, block, 0, st>>>(S, q, k, v, g, beta, o, Hv, Hk, q_scale);               \
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
#undef GDN_FITS
    return hipErrorInvalidValue;
}

hipError_t launch_delta_decode(int narrow_state, void *S, const float *q, const float *k,
                               const float *v, const float *g, const float *beta, float *o,
                               int B, int Hv, int Hk, int dk, int dv, float q_scale,
                               hipStream_t st) {
    if (B <= 0 || Hv <= 0) return hipSuccess;
    if (narrow_state == kF32)
        return launch_decode_cfg<kF32>(S, q, k, v, g, beta, o, B, Hv, Hk, dk, dv, q_scale, st);
    if (narrow_state == kF16)
        return launch_decode_cfg<kF16>(S, q, k, v, g, beta, o, B, Hv, Hk, dk, dv, q_scale, st);
    return hipErrorInvalidValue;
}

}  // namespace gdn

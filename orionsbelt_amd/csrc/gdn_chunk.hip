// gdn_chunk.hip -- chunkwise (WY) gated delta rule prefill for gfx950.
//
// Algorithm: HF torch_chunk_gated_delta_rule (transformers
// modeling_qwen3_5.py:248-328), chunk size 64, head dims 128.  Per
// (sequence b, value head h, chunk n) with G = cumsum(g) inside the chunk and
// Gamma_ij = exp(G_i - G_j) (i >= j):
//   M  = tril(beta_i (k_i . k_j) Gamma_ij, -1)        T = (I + M)^-1
//   W  = T (beta k e^G)    U = T (beta v)    A = tril((q_i . k_j) Gamma_ij) * scale
// then sequentially over chunks, with S the [128 x 128] state:
//   v_new = U - W S ;  o = (q e^G scale) S + A v_new ;
//   S = e^{G_last} S + (k e^{G_last - G})^T v_new
//
// Phase A (chunk_prep_kernel) computes everything that does not depend on S,
// fully parallel over (chunk, head): K K^T and Q K^T on bf16 MFMA, the unit
// lower-triangular inverse T in fp32 (column-parallel forward substitution),
// W and U on MFMA.  It writes W (bf16), U (fp32), A (bf16), Q e^G (bf16),
// (K e^{G_last-G})^T (bf16) and e^{G_last} to a workspace.
//
// Phase B (chunk_state_kernel) runs the recurrence.  The update of column j
// of S needs only column j of S, U and v_new, so the 128 value columns are
// split in 8 tiles of 16: one workgroup per (b, h, column tile), 4 waves.
// Wave w owns rows 32w..32w+31 of the fp32 state tile as MFMA accumulators
// and computes v_new / o for chunk rows 16w..16w+15.  S (bf16) and v_new
// (bf16) are exchanged through LDS, transposed so every MFMA operand is one
// 16-byte read.  Operands of chunk n+1 are fetched while chunk n computes.
//
// Long sequences run as segments of up to kSegChunks chunks (phase A then
// phase B per segment) so the workspace stays bounded.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int C = kChunk;      // 64
constexpr int D = kHeadDim;    // 128
constexpr int kSegChunks = 64; // chunks per segment
constexpr int kColTile = 16;   // value columns per phase-B workgroup
constexpr int kNColTiles = D / kColTile;

// Workspace layout of one segment: arrays indexed by cn = (b*NCs + n)*Hv + h.
struct ChunkWs {
    uint16_t *W;    // [cn][C][D]   bf16
    float *U;       // [cn][C][D]   fp32
    uint16_t *A;    // [cn][C][C]   bf16 (masked, scaled Q K^T)
    uint16_t *Qg;   // [cn][C][D]   bf16
    uint16_t *KgT;  // [cn][D][C]   bf16
    float *gam;     // [cn]         e^{G_last}
    float *S32;     // [B][Hv][D][D] fp32 carried state between segments
};

constexpr size_t kWsW = (size_t)C * D * 2, kWsU = (size_t)C * D * 4, kWsA = (size_t)C * C * 2,
                 kWsQ = (size_t)C * D * 2, kWsK = (size_t)D * C * 2;

GDN_DEV uint32_t pack2_bf16(float a, float b) {
    return (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
}

// ---------------------------------------------------------------------------
// Phase A
// ---------------------------------------------------------------------------
// LDS: rows padded by 8 bf16 (16 B) so row-strided 16-byte fragment reads
// fall in different banks.
constexpr int PD = D + 8;   // padded row of a [.][D] bf16 tile
constexpr int PC = C + 8;   // padded row of a [.][C] bf16 tile
constexpr int PF = C + 1;   // padded row of a [.][C] fp32 tile

struct PrepSmem {
    union {
        struct {
            uint16_t K[C][PD];  // raw k rows
            uint16_t Q[C][PD];  // raw q rows
        } in;
        struct {
            float M[C][PF];     // strictly lower beta K K^T Gamma
            float X[C][PF];     // T = (I + M)^-1
        } tri;
    } u;
    uint16_t KBGt[D][PC];       // (beta k e^G)^T  [d][i]
    uint16_t VBt[D][PC];        // (beta v)^T      [d][i]
    uint16_t Tb[C][PC];         // T in bf16       [i][m]
    float G[C];
    float Bt[C];
    float graw[C];
};

__global__ __launch_bounds__(256) void chunk_prep_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *__restrict__ g, const float *__restrict__ beta,
    int T, int Hv, int Hk, int n0, int NCs, float q_scale, ChunkWs ws) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    PrepSmem &sm = *reinterpret_cast<PrepSmem *>(smem_raw);
    const int nl = blockIdx.x;           // chunk within the segment
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int n = n0 + nl;               // global chunk index
    const int kh = h / (Hv / Hk);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, r = lane & 15;
    const size_t cn = ((size_t)b * NCs + nl) * Hv + h;

    // 1. gates and the in-chunk cumulative sum (sequential order, as cumsum)
    if (tid < C) {
        const int t = n * C + tid;
        const bool live = t < T;
        sm.graw[tid] = live ? g[((size_t)b * T + t) * Hv + h] : 0.f;
        sm.Bt[tid] = live ? beta[((size_t)b * T + t) * Hv + h] : 0.f;
    }
    __syncthreads();
    if (tid < C) {
        float acc = 0.f;
        for (int i = 0; i <= tid; ++i) acc = acc + sm.graw[i];
        sm.G[tid] = acc;
    }
    __syncthreads();
    const float Glast = sm.G[C - 1];

    // 2. load q, k, v rows (16 B = 8 bf16 per load), scatter into LDS layouts
    for (int it = tid; it < C * (D / 8); it += 256) {
        const int i = it / (D / 8);
        const int d0 = (it % (D / 8)) * 8;
        const int t = n * C + i;
        uint4 kv4 = make_uint4(0, 0, 0, 0), qv4 = kv4, vv4 = kv4;
        if (t < T) {
            kv4 = *reinterpret_cast<const uint4 *>(k + (((size_t)b * T + t) * Hk + kh) * D + d0);
            qv4 = *reinterpret_cast<const uint4 *>(q + (((size_t)b * T + t) * Hk + kh) * D + d0);
            vv4 = *reinterpret_cast<const uint4 *>(v + (((size_t)b * T + t) * Hv + h) * D + d0);
        }
        *reinterpret_cast<uint4 *>(&sm.u.in.K[i][d0]) = kv4;
        *reinterpret_cast<uint4 *>(&sm.u.in.Q[i][d0]) = qv4;
        const float eg = expf(sm.G[i]);
        const float bt = sm.Bt[i];
        const float qs = q_scale * eg;
        const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
        const uint32_t qw[4] = {qv4.x, qv4.y, qv4.z, qv4.w};
        const uint32_t vw[4] = {vv4.x, vv4.y, vv4.z, vv4.w};
        uint32_t qo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float k0 = bf16_to_f32((uint16_t)(kw[e] & 0xFFFF));
            const float k1 = bf16_to_f32((uint16_t)(kw[e] >> 16));
            const float v0 = bf16_to_f32((uint16_t)(vw[e] & 0xFFFF));
            const float v1 = bf16_to_f32((uint16_t)(vw[e] >> 16));
            sm.KBGt[d0 + 2 * e][i] = f32_to_bf16_rne(k0 * bt * eg);
            sm.KBGt[d0 + 2 * e + 1][i] = f32_to_bf16_rne(k1 * bt * eg);
            sm.VBt[d0 + 2 * e][i] = f32_to_bf16_rne(v0 * bt);
            sm.VBt[d0 + 2 * e + 1][i] = f32_to_bf16_rne(v1 * bt);
            qo[e] = pack2_bf16(bf16_to_f32((uint16_t)(qw[e] & 0xFFFF)) * qs,
                               bf16_to_f32((uint16_t)(qw[e] >> 16)) * qs);
        }
        *reinterpret_cast<uint4 *>(ws.Qg + cn * (C * D) + (size_t)i * D + d0) =
            make_uint4(qo[0], qo[1], qo[2], qo[3]);
    }
    if (tid == 0) ws.gam[cn] = expf(Glast);
    __syncthreads();

    // 2b. (K e^{G_last - G})^T -> workspace [d][i], 8 consecutive i per store
    for (int it = tid; it < D * (C / 8); it += 256) {
        const int d = it / (C / 8);
        const int i0 = (it % (C / 8)) * 8;
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 2 * e;
            w4[e] = pack2_bf16(bf16_to_f32(sm.u.in.K[i][d]) * expf(Glast - sm.G[i]),
                               bf16_to_f32(sm.u.in.K[i + 1][d]) * expf(Glast - sm.G[i + 1]));
        }
        *reinterpret_cast<uint4 *>(ws.KgT + cn * (D * C) + (size_t)d * C + i0) =
            make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }

    // 3. K K^T and Q K^T: wave w -> row block w, column blocks 0..3
    f32x4_t kk[4], qk[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) { kk[cb] = zero4(); qk[cb] = zero4(); }
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        const bf16x8_t ak = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.u.in.K[16 * wave + r][kb * 32 + 8 * gq]));
        const bf16x8_t aq = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.u.in.Q[16 * wave + r][kb * 32 + 8 * gq]));
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const bf16x8_t bk = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.u.in.K[16 * cb + r][kb * 32 + 8 * gq]));
            kk[cb] = mfma_16x16x32_bf16(ak, bk, kk[cb]);
            qk[cb] = mfma_16x16x32_bf16(aq, bk, qk[cb]);
        }
    }
    __syncthreads();  // K/Q tiles are dead from here (tri aliases them)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int j = 16 * cb + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 16 * wave + 4 * gq + e;
            const float gam_ij = expf(sm.G[i] - sm.G[j]);
            sm.u.tri.M[i][j] = (j < i) ? sm.Bt[i] * kk[cb][e] * gam_ij : 0.f;
            const float a = (j <= i) ? q_scale * qk[cb][e] * gam_ij : 0.f;
            ws.A[cn * (C * C) + (size_t)i * C + j] = f32_to_bf16_rne(a);
        }
    }
    __syncthreads();

    // 4. T = (I + M)^-1: lane j solves column j by forward substitution,
    //    X[i][j] = delta_ij - sum_{m<i} M[i][m] X[m][j]  (fp32)
    if (wave == 0) {
        const int j = lane;
        for (int i = 0; i < C; ++i) {
            float acc = 0.f;
            for (int m = 0; m < i; ++m) acc = fmaf(sm.u.tri.M[i][m], sm.u.tri.X[m][j], acc);
            const float x = (i == j) ? 1.f : -acc;
            sm.u.tri.X[i][j] = x;
            sm.Tb[i][j] = f32_to_bf16_rne(x);
        }
    }
    __syncthreads();

    // 5. W = T (beta k e^G), U = T (beta v): wave w -> row block w, 8 column blocks
    f32x4_t wacc[8], uacc[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) { wacc[cb] = zero4(); uacc[cb] = zero4(); }
#pragma unroll
    for (int kb = 0; kb < C / 32; ++kb) {
        const bf16x8_t at = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.Tb[16 * wave + r][kb * 32 + 8 * gq]));
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            const bf16x8_t bk = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.KBGt[16 * cb + r][kb * 32 + 8 * gq]));
            const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.VBt[16 * cb + r][kb * 32 + 8 * gq]));
            wacc[cb] = mfma_16x16x32_bf16(at, bk, wacc[cb]);
            uacc[cb] = mfma_16x16x32_bf16(at, bv, uacc[cb]);
        }
    }
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
        const int d = 16 * cb + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 16 * wave + 4 * gq + e;
            ws.W[cn * (C * D) + (size_t)i * D + d] = f32_to_bf16_rne(wacc[cb][e]);
            ws.U[cn * (C * D) + (size_t)i * D + d] = uacc[cb][e];
        }
    }
}

// ---------------------------------------------------------------------------
// Phase B
// ---------------------------------------------------------------------------
constexpr int PS = D + 8;   // padded row of S^T [col][d] bf16
constexpr int PV = C + 8;   // padded row of v_new^T [col][i] bf16

struct StateSmem {
    uint16_t ST[2][kColTile][PS];
    uint16_t VN[kColTile][PV];
};

// Per-wave MFMA operands of one chunk (all independent of S).
struct ChunkFrags {
    u32x4_t w[4];      // W rows 16w+r, k-steps 0..3 (d)
    u32x4_t qg[4];     // Q e^G rows 16w+r
    u32x4_t a[2];      // A rows 16w+r, k-steps 0..1 (chunk rows)
    u32x4_t kt[2][2];  // KgT rows d = 32w+16rb+r, k-steps 0..1
    float u[4];        // U[16w+4g+e][col]
    float gam;
};

GDN_DEV void load_frags(ChunkFrags &f, const ChunkWs &ws, size_t cn, int wave, int gq, int r,
                        int col) {
    const uint16_t *Wp = ws.W + cn * (C * D) + (size_t)(16 * wave + r) * D + 8 * gq;
    const uint16_t *Qp = ws.Qg + cn * (C * D) + (size_t)(16 * wave + r) * D + 8 * gq;
    const uint16_t *Ap = ws.A + cn * (C * C) + (size_t)(16 * wave + r) * C + 8 * gq;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        f.w[kb] = *reinterpret_cast<const u32x4_t *>(Wp + kb * 32);
        f.qg[kb] = *reinterpret_cast<const u32x4_t *>(Qp + kb * 32);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) f.a[kb] = *reinterpret_cast<const u32x4_t *>(Ap + kb * 32);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const uint16_t *Kp = ws.KgT + cn * (D * C) + (size_t)(32 * wave + 16 * rb + r) * C + 8 * gq;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) f.kt[rb][kb] = *reinterpret_cast<const u32x4_t *>(Kp + kb * 32);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) f.u[e] = ws.U[cn * (C * D) + (size_t)(16 * wave + 4 * gq + e) * D + col];
    f.gam = ws.gam[cn];
}

template <int IN_FMT, int OUT_FMT>
__global__ __launch_bounds__(256) void chunk_state_kernel(const void *S_in, void *S_out,
                                                          uint16_t *__restrict__ o, int T,
                                                          int Hv, int n0, int ncount,
                                                          int NCs, ChunkWs ws) {
    __shared__ __align__(16) StateSmem sm;
    const int ct = blockIdx.x;   // column tile
    const int h = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, r = lane & 15;
    const int col = ct * kColTile + r;
    const size_t sbase = ((size_t)b * Hv + h) * D * D;

    // state tile: wave w, row block rb -> S[d = 32w + 16rb + 4g + e][col]
    f32x4_t s[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const size_t idx = sbase + (size_t)(32 * wave + 16 * rb + 4 * gq + e) * D + col;
            if constexpr (IN_FMT == kF16) s[rb][e] = f16_to_f32(static_cast<const uint16_t *>(S_in)[idx]);
            else s[rb][e] = static_cast<const float *>(S_in)[idx];
        }

    ChunkFrags cur, nxt;
    load_frags(nxt, ws, ((size_t)b * NCs + 0) * Hv + h, wave, gq, r, col);
    int buf = 0;
    for (int nl = 0; nl < ncount; ++nl) {
        cur = nxt;
        if (nl + 1 < ncount) load_frags(nxt, ws, ((size_t)b * NCs + nl + 1) * Hv + h, wave, gq, r, col);

        // a. S (bf16) -> LDS, transposed [col][d]
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            uint2 pk;
            pk.x = pack2_bf16(s[rb][0], s[rb][1]);
            pk.y = pack2_bf16(s[rb][2], s[rb][3]);
            *reinterpret_cast<uint2 *>(&sm.ST[buf][r][32 * wave + 16 * rb + 4 * gq]) = pk;
        }
        __syncthreads();

        // c. v_new rows 16w.. = U - W S
        f32x4_t ws_acc = zero4(), o_acc = zero4();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const bf16x8_t bs = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.ST[buf][r][kb * 32 + 8 * gq]));
            ws_acc = mfma_16x16x32_bf16(as_bf16x8(cur.w[kb]), bs, ws_acc);
            o_acc = mfma_16x16x32_bf16(as_bf16x8(cur.qg[kb]), bs, o_acc);
        }
        f32x4_t vn;
#pragma unroll
        for (int e = 0; e < 4; ++e) vn[e] = cur.u[e] - ws_acc[e];
        {
            uint2 pk;
            pk.x = pack2_bf16(vn[0], vn[1]);
            pk.y = pack2_bf16(vn[2], vn[3]);
            *reinterpret_cast<uint2 *>(&sm.VN[r][16 * wave + 4 * gq]) = pk;
        }
        __syncthreads();

        // e. o rows = Q e^G S + A v_new
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.VN[r][kb * 32 + 8 * gq]));
            o_acc = mfma_16x16x32_bf16(as_bf16x8(cur.a[kb]), bv, o_acc);
        }
        const int n = n0 + nl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = n * C + 16 * wave + 4 * gq + e;
            if (t < T) o[(((size_t)b * T + t) * Hv + h) * D + col] = f32_to_bf16_rne(o_acc[e]);
        }

        // f. S = e^{G_last} S + (K e^{G_last-G})^T v_new
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
            for (int e = 0; e < 4; ++e) s[rb][e] *= cur.gam;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.VN[r][kb * 32 + 8 * gq]));
                s[rb] = mfma_16x16x32_bf16(as_bf16x8(cur.kt[rb][kb]), bv, s[rb]);
            }
        }
        buf ^= 1;
    }

#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const size_t idx = sbase + (size_t)(32 * wave + 16 * rb + 4 * gq + e) * D + col;
            if constexpr (OUT_FMT == kF16) static_cast<uint16_t *>(S_out)[idx] = f32_to_f16_rne(s[rb][e]);
            else static_cast<float *>(S_out)[idx] = s[rb][e];
        }
}

size_t seg_chunks(int T) {
    const int nchunks = (T + C - 1) / C;
    return (size_t)(nchunks < kSegChunks ? nchunks : kSegChunks);
}

}  // namespace

size_t chunk_workspace_bytes(int B, int T, int Hv) {
    const size_t ncs = seg_chunks(T);
    const size_t per = kWsW + kWsU + kWsA + kWsQ + kWsK;
    const size_t cnt = (size_t)B * ncs * Hv;
    size_t bytes = cnt * per + ((cnt * 4 + 255) / 256) * 256;
    bytes += (size_t)B * Hv * D * D * 4;  // fp32 state carried between segments
    return bytes;
}

hipError_t launch_chunk_prefill(int narrow_state, const uint16_t *q, const uint16_t *k,
                                const uint16_t *v, const float *g, const float *beta,
                                uint16_t *o, void *S, int B, int T, int Hv, int Hk,
                                float q_scale, void *workspace, hipStream_t st) {
    if (B <= 0 || T <= 0 || Hv <= 0) return hipSuccess;
    const int nchunks = (T + C - 1) / C;
    const int ncs = (int)seg_chunks(T);
    const size_t cnt = (size_t)B * ncs * Hv;
    char *p = static_cast<char *>(workspace);
    ChunkWs ws;
    ws.W = reinterpret_cast<uint16_t *>(p); p += cnt * kWsW;
    ws.U = reinterpret_cast<float *>(p);    p += cnt * kWsU;
    ws.A = reinterpret_cast<uint16_t *>(p); p += cnt * kWsA;
    ws.Qg = reinterpret_cast<uint16_t *>(p); p += cnt * kWsQ;
    ws.KgT = reinterpret_cast<uint16_t *>(p); p += cnt * kWsK;
    ws.gam = reinterpret_cast<float *>(p);  p += ((cnt * 4 + 255) / 256) * 256;
    ws.S32 = reinterpret_cast<float *>(p);

    {
        hipError_t e = hipFuncSetAttribute((const void *)chunk_prep_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)sizeof(PrepSmem));
        if (e != hipSuccess) return e;
    }

    const int nseg = (nchunks + ncs - 1) / ncs;
    for (int sgi = 0; sgi < nseg; ++sgi) {
        const int n0 = sgi * ncs;
        const int nc_here = (nchunks - n0) < ncs ? (nchunks - n0) : ncs;
        chunk_prep_kernel<<<dim3(nc_here, Hv, B), 256, sizeof(PrepSmem), st>>>(
            q, k, v, g, beta, T, Hv, Hk, n0, ncs, q_scale, ws);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // state source / destination of this segment
        const bool first = sgi == 0, last = sgi == nseg - 1;
        const void *sin = first ? S : ws.S32;
        void *sout = last ? S : ws.S32;
        const int in_fmt = first ? narrow_state : kF32;
        const int out_fmt = last ? narrow_state : kF32;
        dim3 grid(kNColTiles, Hv, B);
        // the workspace keeps the stride of a full segment (ncs) even when
        // the last segment is shorter (nc_here chunks)
        if (in_fmt == kF32 && out_fmt == kF32)
            chunk_state_kernel<kF32, kF32><<<grid, 256, 0, st>>>(sin, sout, o, T, Hv, n0, nc_here, ncs, ws);
        else if (in_fmt == kF16 && out_fmt == kF16)
            chunk_state_kernel<kF16, kF16><<<grid, 256, 0, st>>>(sin, sout, o, T, Hv, n0, nc_here, ncs, ws);
        else if (in_fmt == kF16 && out_fmt == kF32)
            chunk_state_kernel<kF16, kF32><<<grid, 256, 0, st>>>(sin, sout, o, T, Hv, n0, nc_here, ncs, ws);
        else
            chunk_state_kernel<kF32, kF16><<<grid, 256, 0, st>>>(sin, sout, o, T, Hv, n0, nc_here, ncs, ws);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace gdn

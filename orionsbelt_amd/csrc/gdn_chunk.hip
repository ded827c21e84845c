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
// Phase A (chunk_prep_kernel), parallel over (chunk, head), does everything
// that does not depend on S and leaves phase B nothing but MFMAs: K K^T and
// Q K^T on bf16 MFMA, the unit lower-triangular inverse T in fp32 (16x16
// diagonal blocks by lane-parallel forward substitution in registers, then
// three block-row levels), W = T (beta k e^G) on MFMA, and the gated,
// transposed operands.  Per (chunk, head) it writes, all bf16 and laid out so
// each MFMA fragment is one 16-byte load:
//   W [i][d]   Qg = q e^G scale [i][d]   A [i][j]   T [i][m]
//   KgT = (k e^{G_last-G})^T [d][i]      VBt = (beta v)^T [d][i]
// and e^{G_last} (fp32).  Every matrix is stored in MFMA-fragment order:
// fragment (row block rb, k-step kb) is 64 lanes x 16 B contiguous, lane
// (g, r) holding X[16 rb + r][32 kb + 8 g .. +7], so each wave-wide operand
// load is one contiguous 1 KiB request.
//
// Phase B (chunk_state_kernel) runs the recurrence.  Column j of S, U and
// v_new depends only on column j, so the 128 value columns are split into
// 32-column tiles: one workgroup per (head, column tile, sequence), 4 waves.
// Wave w owns state rows 32w..32w+31 as fp32 MFMA accumulators and chunk rows
// 16w..16w+15 of U = T VBt^T, v_new and o.  Four workgroups per head (not
// more) keep the L2 request rate of the shared per-chunk operands low.  S and v_new cross waves through
// LDS in bf16, stored transposed so every operand is one 16-byte LDS read.
// The grid's fastest dimension is the head, so all column tiles of a head fall
// on the same XCD (workgroups are dealt to the 8 XCDs round-robin) and share
// its L2.  Phase B only reads the workspace, always whole chunks (phase A
// zero-fills rows past the sequence end), so its loads are unconditional;
// the chunk loop is unrolled by two with two register buffers, so the
// operands of chunk n+1 stream in while chunk n computes.
//
// The host runs the sequence as segments of kSegChunks chunks with a
// double-buffered workspace: phase A of segment s+1 runs on a second stream
// while phase B of segment s runs on the caller's stream.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int C = kChunk;      // 64
constexpr int D = kHeadDim;    // 128
constexpr int kRec = 256;      // floats of per-row factors per (chunk, head)

// Workspace of one segment: arrays indexed by cn = (b*NCs + n)*Hv + h.
struct ChunkWs {
    uint16_t *W;    // [cn][C][D]  bf16
    uint16_t *Qg;   // [cn][C][D]  bf16  q e^G scale
    uint16_t *KgT;  // [cn][D][C]  bf16  (k e^{G_last-G})^T
    uint16_t *VBt;  // [cn][D][C]  bf16  (beta v)^T
    uint16_t *T;    // [cn][C][C]  bf16  (I + M)^-1
    uint16_t *A;    // [cn][C][C]  bf16  masked, scaled Q K^T Gamma
    float *gam;     // [cn]        e^{G_last}
};

constexpr size_t kWsBig = (size_t)C * D * 2, kWsSmall = (size_t)C * C * 2;
constexpr size_t kWsPer = 4 * kWsBig + 2 * kWsSmall + 4;

GDN_DEV uint32_t pack2_bf16(float a, float b) { return pack2_bf16_hw(a, b); }
GDN_DEV float bf_lo(uint32_t w) { return bf16_to_f32((uint16_t)(w & 0xFFFF)); }
GDN_DEV float bf_hi(uint32_t w) { return bf16_to_f32((uint16_t)(w >> 16)); }

// Element offset of fragment (rb, kb), lane l, of a matrix with `kcols`
// columns stored in MFMA-fragment order (8 bf16 per lane).
GDN_DEV constexpr size_t frag_off(int rb, int kb, int lane, int kcols) {
    return ((size_t)(rb * (kcols / 32) + kb) * 64 + lane) * 8;
}

// ---------------------------------------------------------------------------
// Phase A
// ---------------------------------------------------------------------------
constexpr int PD = D + 8;   // padded row of a [.][D] bf16 tile (272 B)
constexpr int PC = C + 8;   // padded row of a [.][C] bf16 tile (144 B)
constexpr int PF = C + 1;   // padded row of a [.][C] fp32 tile

struct PrepSmem {
    union {
        struct {
            uint16_t K[C][PD];  // raw k rows
            uint16_t Q[C][PD];  // raw q rows
        } in;
        struct {
            float M[C][PF];     // strictly lower beta K K^T Gamma
            float X[C][PF];     // T = (I + M)^-1 (lower blocks only)
        } tri;
        uint16_t VBt[D][PC];    // (beta v)^T staging, after the solve
    } u;
    union {
        uint16_t KBGt[D][PC];   // (beta k e^G)^T  [d][i]
        uint16_t Wst[C][PD];    // W staging (after its MFMAs)
    } w;
    uint16_t Ast[C][PC];        // A staging
    uint16_t Tb[C][PC];         // T in bf16, zero above the diagonal
    float P[3][16][17];         // block products of the solve
    float G[C], eG[C], eGl[C], qs[C], Bt[C], graw[C];
};

__global__ __launch_bounds__(256) void chunk_prep_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, const float *__restrict__ g,
    const float *__restrict__ beta, int T, int Hv, int Hk, int n0, int NCs, float q_scale,
    ChunkWs ws) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    PrepSmem &sm = *reinterpret_cast<PrepSmem *>(smem_raw);
    const int h = blockIdx.x;            // heads fastest: chunk (n, h) on XCD h % 8
    const int nl = blockIdx.y;           // chunk within the segment
    const int b = blockIdx.z;
    const int n = n0 + nl;               // global chunk index
    const int kh = h / (Hv / Hk);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, r = lane & 15;
    const size_t cn = ((size_t)b * NCs + nl) * Hv + h;

    // 1. gates; in-chunk cumulative sum in sequential order (as cumsum); the
    //    uniform loop adds exact zeros past row tid
    if (tid < C) {
        const int t = n * C + tid;
        const int tc = min(t, T - 1);
        const float gv = g[((size_t)b * T + tc) * Hv + h];
        const float bv = beta[((size_t)b * T + tc) * Hv + h];
        sm.graw[tid] = t < T ? gv : 0.f;
        sm.Bt[tid] = t < T ? bv : 0.f;
    }
    __syncthreads();
    if (tid < C) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < C; ++i) acc = acc + (i <= tid ? sm.graw[i] : 0.f);
        sm.G[tid] = acc;
        sm.eG[tid] = expf(acc);
    }
    __syncthreads();
    const float Glast = sm.G[C - 1];
    if (tid < C) {
        sm.eGl[tid] = expf(Glast - sm.G[tid]);
        sm.qs[tid] = q_scale * sm.eG[tid];
    }
    if (tid == 0) ws.gam[cn] = expf(Glast);

    // 2. q, k rows -> LDS; Qg -> workspace; (beta k e^G)^T -> LDS; v rows kept
    //    in registers for the (beta v)^T staging after the solve
    uint4 vrow[C * (D / 8) / 256];
#pragma unroll
    for (int j = 0; j < C * (D / 8) / 256; ++j) {
        const int it = tid + 256 * j;
        const int i = it / (D / 8);
        const int d0 = (it % (D / 8)) * 8;
        const int t = n * C + i;
        const int tc = min(t, T - 1);  // rows past the end load row T-1, then read as 0
        uint4 kv4 = *reinterpret_cast<const uint4 *>(k + (((size_t)b * T + tc) * Hk + kh) * D + d0);
        uint4 qv4 = *reinterpret_cast<const uint4 *>(q + (((size_t)b * T + tc) * Hk + kh) * D + d0);
        uint4 vv4 = *reinterpret_cast<const uint4 *>(v + (((size_t)b * T + tc) * Hv + h) * D + d0);
        if (t >= T) kv4 = qv4 = vv4 = make_uint4(0, 0, 0, 0);
        vrow[j] = vv4;
        *reinterpret_cast<uint4 *>(&sm.u.in.K[i][d0]) = kv4;
        *reinterpret_cast<uint4 *>(&sm.u.in.Q[i][d0]) = qv4;
        const float f = sm.Bt[i] * sm.eG[i];
        const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.w.KBGt[d0 + 2 * e][i] = f32_to_bf16_hw(bf_lo(kw[e]) * f);
            sm.w.KBGt[d0 + 2 * e + 1][i] = f32_to_bf16_hw(bf_hi(kw[e]) * f);
        }
    }
    __syncthreads();

    // 2a. Qg = q * scale * e^G -> workspace, fragment order (16 frags of [64][128])
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int it = tid + 256 * j;          // fragment element: frag = it / 64, lane = it % 64
        const int fr = it >> 6, l = it & 63;
        const int row = 16 * (fr >> 2) + (l & 15), col = 32 * (fr & 3) + 8 * (l >> 4);
        const uint4 qv4 = *reinterpret_cast<const uint4 *>(&sm.u.in.Q[row][col]);
        const float qs = sm.qs[row];
        const uint32_t qw[4] = {qv4.x, qv4.y, qv4.z, qv4.w};
        uint32_t qo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) qo[e] = pack2_bf16(bf_lo(qw[e]) * qs, bf_hi(qw[e]) * qs);
        *reinterpret_cast<uint4 *>(ws.Qg + cn * (C * D) + (size_t)it * 8) =
            make_uint4(qo[0], qo[1], qo[2], qo[3]);
    }

    // 2b. (k e^{G_last - G})^T [d][i] -> workspace, fragment order (16 frags of [128][64])
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int it = tid + 256 * j;
        const int fr = it >> 6, l = it & 63;
        const int d = 16 * (fr >> 1) + (l & 15), i0 = 32 * (fr & 1) + 8 * (l >> 4);
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 2 * e;
            w4[e] = pack2_bf16(bf16_to_f32(sm.u.in.K[i][d]) * sm.eGl[i],
                               bf16_to_f32(sm.u.in.K[i + 1][d]) * sm.eGl[i + 1]);
        }
        *reinterpret_cast<uint4 *>(ws.KgT + cn * (D * C) + (size_t)it * 8) =
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
    __syncthreads();  // the K/Q tiles are dead from here (tri aliases them)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int j = 16 * cb + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 16 * wave + 4 * gq + e;
            const float gam_ij = (j <= i) ? expf(sm.G[i] - sm.G[j]) : 0.f;
            sm.u.tri.M[i][j] = (j < i) ? sm.Bt[i] * kk[cb][e] * gam_ij : 0.f;
            sm.Ast[i][j] = f32_to_bf16_hw(q_scale * qk[cb][e] * gam_ij);
        }
    }
    __syncthreads();

    // A -> workspace, fragment order (8 frags of [64][64])
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int it = tid + 256 * j;
        const int fr = it >> 6, l = it & 63;
        const int row = 16 * (fr >> 1) + (l & 15), col = 32 * (fr & 1) + 8 * (l >> 4);
        *reinterpret_cast<uint4 *>(ws.A + cn * (C * C) + (size_t)it * 8) =
            *reinterpret_cast<const uint4 *>(&sm.Ast[row][col]);
    }

    // 4a. diagonal 16x16 blocks of T: wave 0, lane group g -> block g, lane r
    //     -> column r; X[i][r] = delta_ir - sum_{m<i} M[i][m] X[m][r]
    if (wave == 0) {
        const int o0 = 16 * gq;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) acc = fmaf(sm.u.tri.M[o0 + i][o0 + m], x[m], acc);
            x[i] = (i == r) ? 1.f : ((i > r) ? -acc : 0.f);
            sm.u.tri.X[o0 + i][o0 + r] = x[i];
        }
    }
    __syncthreads();
    // 4b. block rows 1..3: T_ij = -T_ii sum_{k=j}^{i-1} M_ik T_kj
    for (int bi = 1; bi < 4; ++bi) {
        for (int e = tid; e < bi * 256; e += 256) {
            const int bj = e >> 8, a = (e >> 4) & 15, c = e & 15;
            float acc = 0.f;
            for (int bk = bj; bk < bi; ++bk)
#pragma unroll
                for (int m = 0; m < 16; ++m)
                    acc = fmaf(sm.u.tri.M[16 * bi + a][16 * bk + m], sm.u.tri.X[16 * bk + m][16 * bj + c], acc);
            sm.P[bj][a][c] = acc;
        }
        __syncthreads();
        for (int e = tid; e < bi * 256; e += 256) {
            const int bj = e >> 8, a = (e >> 4) & 15, c = e & 15;
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < 16; ++m)
                acc = fmaf(sm.u.tri.X[16 * bi + a][16 * bi + m], sm.P[bj][m][c], acc);
            sm.u.tri.X[16 * bi + a][16 * bj + c] = -acc;
        }
        __syncthreads();
    }
    // 4c. bf16 copy (zero above the block diagonal) -> LDS and workspace
    for (int e = tid; e < C * C / 2; e += 256) {
        const int i = e / (C / 2), m = (e % (C / 2)) * 2;
        const float x0 = ((m >> 4) <= (i >> 4)) ? sm.u.tri.X[i][m] : 0.f;
        const float x1 = (((m + 1) >> 4) <= (i >> 4)) ? sm.u.tri.X[i][m + 1] : 0.f;
        *reinterpret_cast<uint32_t *>(&sm.Tb[i][m]) = pack2_bf16(x0, x1);
    }
    __syncthreads();  // tri is dead from here: stage (beta v)^T in its place
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // T -> workspace, fragment order
        const int it = tid + 256 * j;
        const int fr = it >> 6, l = it & 63;
        const int row = 16 * (fr >> 1) + (l & 15), col = 32 * (fr & 1) + 8 * (l >> 4);
        *reinterpret_cast<uint4 *>(ws.T + cn * (C * C) + (size_t)it * 8) =
            *reinterpret_cast<const uint4 *>(&sm.Tb[row][col]);
    }

    // 5. (beta v)^T -> LDS from the rows kept in registers
#pragma unroll
    for (int j = 0; j < C * (D / 8) / 256; ++j) {
        const int it = tid + 256 * j;
        const int i = it / (D / 8);
        const int d0 = (it % (D / 8)) * 8;
        const float bt = sm.Bt[i];
        const uint32_t vw[4] = {vrow[j].x, vrow[j].y, vrow[j].z, vrow[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sm.u.VBt[d0 + 2 * e][i] = f32_to_bf16_hw(bf_lo(vw[e]) * bt);
            sm.u.VBt[d0 + 2 * e + 1][i] = f32_to_bf16_hw(bf_hi(vw[e]) * bt);
        }
    }

    // 6. W = T (beta k e^G): wave w -> row block w, 8 column blocks
    f32x4_t wacc[8];
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) wacc[cb] = zero4();
#pragma unroll
    for (int kb = 0; kb < C / 32; ++kb) {
        const bf16x8_t at = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.Tb[16 * wave + r][kb * 32 + 8 * gq]));
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            const bf16x8_t bk = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.w.KBGt[16 * cb + r][kb * 32 + 8 * gq]));
            wacc[cb] = mfma_16x16x32_bf16(at, bk, wacc[cb]);
        }
    }
    __syncthreads();  // every wave is done with KBGt: stage W in its place
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            sm.w.Wst[16 * wave + 4 * gq + e][16 * cb + r] = f32_to_bf16_hw(wacc[cb][e]);
    __syncthreads();  // W and (beta v)^T staged
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int it = tid + 256 * j;
        const int fr = it >> 6, l = it & 63;
        // W [64][128]: 16 frags
        const int wrow = 16 * (fr >> 2) + (l & 15), wcol = 32 * (fr & 3) + 8 * (l >> 4);
        *reinterpret_cast<uint4 *>(ws.W + cn * (C * D) + (size_t)it * 8) =
            *reinterpret_cast<const uint4 *>(&sm.w.Wst[wrow][wcol]);
        // (beta v)^T [128][64]: 16 frags
        const int vrow_ = 16 * (fr >> 1) + (l & 15), vcol = 32 * (fr & 1) + 8 * (l >> 4);
        *reinterpret_cast<uint4 *>(ws.VBt + cn * (D * C) + (size_t)it * 8) =
            *reinterpret_cast<const uint4 *>(&sm.u.VBt[vrow_][vcol]);
    }
}

// ---------------------------------------------------------------------------
// Phase B
// ---------------------------------------------------------------------------
constexpr int kColTile = 32;            // value columns per workgroup
constexpr int kNcb = kColTile / 16;     // 16-column MFMA blocks per workgroup

struct StateSmem {
    uint16_t ST[2][kColTile][PD];   // S^T (bf16) [col][d], double buffered
    uint16_t VN[kColTile][PC];      // v_new^T (bf16) [col][i]
};

// One thread's MFMA operands for one chunk, all from the workspace.
struct ChunkOps {
    u32x4_t w[4];          // W fragments (row block w, k-steps 0..3)
    u32x4_t qg[4];         // Qg fragments (row block w)
    u32x4_t a[2];          // A fragments (row block w, k-steps 0..1)
    u32x4_t t[2];          // T fragments (row block w)
    u32x4_t kt[2][2];      // KgT fragments (row blocks 2w, 2w+1)
    u32x4_t vb[kNcb][2];   // VBt fragments (column blocks of this tile)
    float gam;
};

struct OpPtrs {
    const uint16_t *W, *Qg, *A, *T, *KgT, *VBt;
    const float *gam;
};

// Per-lane pointers into chunk 0 of this (b, h); chunk nl adds nl*Hv chunks.
GDN_DEV OpPtrs op_ptrs(const ChunkWs &ws, size_t cn0, int wave, int lane, int ct) {
    OpPtrs p;
    p.W = ws.W + cn0 * (C * D) + frag_off(wave, 0, lane, D);
    p.Qg = ws.Qg + cn0 * (C * D) + frag_off(wave, 0, lane, D);
    p.A = ws.A + cn0 * (C * C) + frag_off(wave, 0, lane, C);
    p.T = ws.T + cn0 * (C * C) + frag_off(wave, 0, lane, C);
    p.KgT = ws.KgT + cn0 * (D * C) + frag_off(2 * wave, 0, lane, C);
    p.VBt = ws.VBt + cn0 * (D * C) + frag_off(kNcb * ct, 0, lane, C);
    p.gam = ws.gam + cn0;
    return p;
}

GDN_DEV void load_ops(ChunkOps &f, const OpPtrs &p, size_t nl, int Hv) {
    const size_t big = nl * Hv * (size_t)(C * D), small = nl * Hv * (size_t)(C * C);
    constexpr int F = 64 * 8;  // elements per fragment
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        f.w[kb] = *reinterpret_cast<const u32x4_t *>(p.W + big + kb * F);
        f.qg[kb] = *reinterpret_cast<const u32x4_t *>(p.Qg + big + kb * F);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        f.a[kb] = *reinterpret_cast<const u32x4_t *>(p.A + small + kb * F);
        f.t[kb] = *reinterpret_cast<const u32x4_t *>(p.T + small + kb * F);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
            f.kt[rb][kb] = *reinterpret_cast<const u32x4_t *>(p.KgT + big + (size_t)(rb * 2 + kb) * F);
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb)
            f.vb[cb][kb] = *reinterpret_cast<const u32x4_t *>(p.VBt + big + (size_t)(cb * 2 + kb) * F);
    }
    f.gam = p.gam[nl * Hv];
}

// One chunk of the recurrence (buf selects the S^T buffer).  State tile
// s[rb][cb]: S[d = 32w + 16rb + 4g + e][col0 + 16cb + r].
GDN_DEV void state_step(StateSmem &sm, f32x4_t (&s)[2][kNcb], const ChunkOps &f, int buf,
                        int wave, int gq, int r, uint16_t *__restrict__ o, size_t orow0, int t0,
                        int T, size_t ostride) {
    // a. S (bf16) -> LDS, transposed [col][d]
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb) {
            u32x2_t pk;
            pk[0] = pack2_bf16(s[rb][cb][0], s[rb][cb][1]);
            pk[1] = pack2_bf16(s[rb][cb][2], s[rb][cb][3]);
            *reinterpret_cast<u32x2_t *>(&sm.ST[buf][16 * cb + r][32 * wave + 16 * rb + 4 * gq]) = pk;
        }
    // U = T (beta v) does not depend on S: issue it before the barrier
    f32x4_t uacc[kNcb];
#pragma unroll
    for (int cb = 0; cb < kNcb; ++cb) {
        uacc[cb] = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
            uacc[cb] = mfma_16x16x32_bf16(as_bf16x8(f.t[kb]), as_bf16x8(f.vb[cb][kb]), uacc[cb]);
    }
    __syncthreads();
    // b. v_new = U - W S ;  o = Qg S
    f32x4_t oacc[kNcb];
#pragma unroll
    for (int cb = 0; cb < kNcb; ++cb) {
        f32x4_t w0 = zero4(), w1 = zero4();
        oacc[cb] = zero4();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const bf16x8_t bs = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.ST[buf][16 * cb + r][kb * 32 + 8 * gq]));
            if (kb & 1) w1 = mfma_16x16x32_bf16(as_bf16x8(f.w[kb]), bs, w1);
            else w0 = mfma_16x16x32_bf16(as_bf16x8(f.w[kb]), bs, w0);
            oacc[cb] = mfma_16x16x32_bf16(as_bf16x8(f.qg[kb]), bs, oacc[cb]);
        }
        f32x4_t vn;
#pragma unroll
        for (int e = 0; e < 4; ++e) vn[e] = uacc[cb][e] - (w0[e] + w1[e]);
        u32x2_t pk;
        pk[0] = pack2_bf16(vn[0], vn[1]);
        pk[1] = pack2_bf16(vn[2], vn[3]);
        *reinterpret_cast<u32x2_t *>(&sm.VN[16 * cb + r][16 * wave + 4 * gq]) = pk;
    }
    __syncthreads();
    // c. S = e^{G_last} S + KgT v_new ;  o += A v_new
#pragma unroll
    for (int cb = 0; cb < kNcb; ++cb) {
        bf16x8_t bv[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
            bv[kb] = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.VN[16 * cb + r][kb * 32 + 8 * gq]));
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
            for (int e = 0; e < 4; ++e) s[rb][cb][e] *= f.gam;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                s[rb][cb] = mfma_16x16x32_bf16(as_bf16x8(f.kt[rb][kb]), bv[kb], s[rb][cb]);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) oacc[cb] = mfma_16x16x32_bf16(as_bf16x8(f.a[kb]), bv[kb], oacc[cb]);
    }
    if (t0 + C <= T) {  // whole chunk (uniform branch): unpredicated stores
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[orow0 + (size_t)(16 * wave + 4 * gq + e) * ostride + 16 * cb] = f32_to_bf16_hw(oacc[cb][e]);
    } else {
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = t0 + 16 * wave + 4 * gq + e;
                if (t < T) o[orow0 + (size_t)(16 * wave + 4 * gq + e) * ostride + 16 * cb] = f32_to_bf16_hw(oacc[cb][e]);
            }
    }
}

template <int IN_FMT, int OUT_FMT>
__global__ __launch_bounds__(256) void chunk_state_kernel(const void *S_in, void *S_out,
                                                          uint16_t *__restrict__ o, int T,
                                                          int Hv, int n0, int ncount, int NCs,
                                                          ChunkWs ws) {
    __shared__ __align__(16) StateSmem sm;
    const int h = blockIdx.x;    // heads fastest: all column tiles of a head share an XCD
    const int ct = blockIdx.y;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, r = lane & 15;
    const int col0 = ct * kColTile;
    const size_t sbase = ((size_t)b * Hv + h) * D * D;

    f32x4_t s[2][kNcb];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const size_t idx = sbase + (size_t)(32 * wave + 16 * rb + 4 * gq + e) * D + col0 + 16 * cb + r;
                if constexpr (IN_FMT == kF16) s[rb][cb][e] = f16_to_f32(static_cast<const uint16_t *>(S_in)[idx]);
                else s[rb][cb][e] = static_cast<const float *>(S_in)[idx];
            }

    const OpPtrs p = op_ptrs(ws, ((size_t)b * NCs) * Hv + h, wave, lane, ct);
    const size_t ostride = (size_t)Hv * D;              // one token
    const size_t obase = ((size_t)b * T * Hv + h) * D + col0 + r;
    // Prefetches are unconditional (the index is clamped; a clamped load is
    // simply not used) so the compiler's wait counts stay exact.
    ChunkOps f0, f1;
    load_ops(f0, p, 0, Hv);
    int nl = 0;
    for (; nl + 1 < ncount; nl += 2) {
        load_ops(f1, p, nl + 1, Hv);
        const int t0 = (n0 + nl) * C;
        state_step(sm, s, f0, 0, wave, gq, r, o, obase + (size_t)t0 * ostride, t0, T, ostride);
        load_ops(f0, p, min(nl + 2, ncount - 1), Hv);
        state_step(sm, s, f1, 1, wave, gq, r, o, obase + (size_t)(t0 + C) * ostride, t0 + C, T,
                   ostride);
    }
    if (nl < ncount) {
        const int t0 = (n0 + nl) * C;
        state_step(sm, s, f0, 0, wave, gq, r, o, obase + (size_t)t0 * ostride, t0, T, ostride);
    }

#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < kNcb; ++cb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const size_t idx = sbase + (size_t)(32 * wave + 16 * rb + 4 * gq + e) * D + col0 + 16 * cb + r;
                if constexpr (OUT_FMT == kF16) static_cast<uint16_t *>(S_out)[idx] = f32_to_f16_rne(s[rb][cb][e]);
                else static_cast<float *>(S_out)[idx] = s[rb][cb][e];
            }
}

constexpr int kSegChunks = 32;  // chunks per segment

size_t seg_chunks(int T) {
    const int nchunks = (T + C - 1) / C;
    return (size_t)(nchunks < kSegChunks ? nchunks : kSegChunks);
}

void carve(char *p, size_t cnt, ChunkWs &ws) {
    ws.W = reinterpret_cast<uint16_t *>(p); p += cnt * kWsBig;
    ws.Qg = reinterpret_cast<uint16_t *>(p); p += cnt * kWsBig;
    ws.KgT = reinterpret_cast<uint16_t *>(p); p += cnt * kWsBig;
    ws.VBt = reinterpret_cast<uint16_t *>(p); p += cnt * kWsBig;
    ws.T = reinterpret_cast<uint16_t *>(p); p += cnt * kWsSmall;
    ws.A = reinterpret_cast<uint16_t *>(p); p += cnt * kWsSmall;
    ws.gam = reinterpret_cast<float *>(p);
}

void launch_state(int in_fmt, int out_fmt, const void *sin, void *sout, uint16_t *o, int B,
                  int T, int Hv, int n0, int nc_here, int ncs, const ChunkWs &ws,
                  hipStream_t st) {
    dim3 grid(Hv, D / kColTile, B);
#define GDN_ST(I, O)                                                                         \
    if (in_fmt == I && out_fmt == O) {                                                       \
        chunk_state_kernel<I, O><<<grid, 256, 0, st>>>(sin, sout, o, T, Hv, n0, nc_here, ncs, \
                                                      ws);                                   \
        return;                                                                              \
    }
    GDN_ST(kF32, kF32)
    GDN_ST(kF16, kF16)
    GDN_ST(kF16, kF32)
    GDN_ST(kF32, kF16)
#undef GDN_ST
}

}  // namespace

size_t chunk_workspace_bytes(int B, int T, int Hv) {
    const size_t cnt = (size_t)B * seg_chunks(T) * Hv;
    const int nchunks = (T + C - 1) / C;
    const int nbuf = nchunks > kSegChunks ? 2 : 1;
    return nbuf * cnt * kWsPer + (size_t)B * Hv * D * D * 4;  // + fp32 state carry
}

hipError_t launch_chunk_prefill(int narrow_state, const uint16_t *q, const uint16_t *k,
                                const uint16_t *v, const float *g, const float *beta,
                                uint16_t *o, void *S, int B, int T, int Hv, int Hk,
                                float q_scale, void *workspace, const PrefillStreams &ps,
                                hipStream_t st) {
    if (B <= 0 || T <= 0 || Hv <= 0) return hipSuccess;
    const int nchunks = (T + C - 1) / C;
    const int ncs = (int)seg_chunks(T);
    const int nseg = (nchunks + ncs - 1) / ncs;
    const size_t cnt = (size_t)B * ncs * Hv;
    ChunkWs ws[2];
    char *p = static_cast<char *>(workspace);
    carve(p, cnt, ws[0]);
    const int nbuf = nseg > 1 ? 2 : 1;
    if (nbuf == 2) carve(p + cnt * kWsPer, cnt, ws[1]);
    float *S32 = reinterpret_cast<float *>(p + nbuf * cnt * kWsPer);

    hipError_t e = hipFuncSetAttribute((const void *)chunk_prep_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)sizeof(PrepSmem));
    if (e != hipSuccess) return e;

    // Phase A runs on ps.aux once the caller's prior work is done, and phase
    // B on the caller's stream; events order the double-buffered workspace.
    const bool overlap = nseg > 1 && ps.aux != nullptr;
    hipStream_t sa = overlap ? ps.aux : st;
    if (overlap) {
        if ((e = hipEventRecord(ps.ready, st)) != hipSuccess) return e;
        if ((e = hipStreamWaitEvent(sa, ps.ready, 0)) != hipSuccess) return e;
    }
    for (int sgi = 0; sgi < nseg; ++sgi) {
        const int bi = sgi % nbuf;
        const int n0 = sgi * ncs;
        const int nc_here = (nchunks - n0) < ncs ? (nchunks - n0) : ncs;
        if (overlap && sgi >= 2 && (e = hipStreamWaitEvent(sa, ps.b_done[bi], 0)) != hipSuccess)
            return e;
        chunk_prep_kernel<<<dim3(Hv, nc_here, B), 256, sizeof(PrepSmem), sa>>>(
            q, k, v, g, beta, T, Hv, Hk, n0, ncs, q_scale, ws[bi]);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (overlap) {
            if ((e = hipEventRecord(ps.a_done[bi], sa)) != hipSuccess) return e;
            if ((e = hipStreamWaitEvent(st, ps.a_done[bi], 0)) != hipSuccess) return e;
        }
        const bool first = sgi == 0, last = sgi == nseg - 1;
        const void *sin = first ? S : S32;
        void *sout = last ? S : S32;
        const int in_fmt = first ? narrow_state : kF32;
        const int out_fmt = last ? narrow_state : kF32;
        launch_state(in_fmt, out_fmt, sin, sout, o, B, T, Hv, n0, nc_here, ncs, ws[bi], st);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (overlap && (e = hipEventRecord(ps.b_done[bi], st)) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace gdn

// gdn_prefill.hip -- chunkwise (WY) gated delta rule prefill for gfx950,
// parallel over the sequence.
//
// Algorithm: HF torch_chunk_gated_delta_rule (transformers
// modeling_qwen3_5.py:248-328), chunk size 64, head dims 128.  Per (sequence
// b, value head h, chunk n) with G = cumsum(g) inside the chunk and
// Gamma_ij = exp(G_i - G_j) (i >= j):
//   M = tril(beta_i (k_i . k_j) Gamma_ij, -1)       T = (I + M)^-1
//   U = T diag(beta) V        W = T diag(beta e^G) K
//   A = tril(Gamma_ij (q_i . k_j)) * scale
// and, sequentially over chunks, with S the [128 x 128] state:
//   v_new = U - W S ;  o = e^G scale (q S) + A v_new ;
//   S' = e^{G_last} S + K^T diag(e^{G_last - G}) v_new
//
// Parallel over the sequence.  The step is affine in S:
//   S' = Phi_n S + C_n,  Phi_n = e^{G_last} I - K^T diag(e^{G_last-G}) W,
//   C_n = K^T diag(e^{G_last-G}) U,
// so the chunks are cut into P segments and
//   pass 1: segment 0 runs the recurrence from the initial state (with o);
//           every middle segment p runs it from S = 0 and, alongside, on
//           128 more state columns started at I with U = 0, which yields its
//           local result C_p and its transition Phi_p;
//   pass 2: segment p = 1 .. P-1 first composes its start state,
//           S_start(q+1) = Phi_q S_start(q) + C_q from S_start(1) = the end of
//           segment 0, then reruns the recurrence from it, with o.
// The work is twice that of one sequential pass, spread over (P-1) x heads
// workgroups instead of heads.
//
// Each workgroup (8 waves, two per SIMD, so that one wave's LDS and MFMA
// latencies overlap the other's work) owns one (sequence, head, segment)
// and walks its chunks.  Per chunk, stage A loads the chunk's k, q, v rows
// into LDS, forms K K^T and Q K^T on bf16 MFMA, inverts (I + M) by 16 x 16
// blocks and solves for W and U.  Stage B (each wave, its own 16 state
// columns) runs the recurrence: the state and v_new never leave registers.
//
// Fragment orders.  The 32 k-indices of one 16x16x32 MFMA may be assigned
// to lanes in any order as long as both operands use the same order.
//  - k = t (a chunk row): lane group g holds t = {4g..4g+3, 16+4g..16+4g+3}
//    of a 32-block, which is the accumulator layout of two stacked 16 x 16
//    tiles (lane group g holds rows 4g..4g+3 of each), so v_new feeds the
//    next products straight from registers.
//  - k = d (a state row): lane group g holds d = 8g..8g+7 of a 32-block, the
//    natural order, so q and Phi rows are read with one 16-byte LDS read per
//    lane.  For that, state tile 2j + u holds, in lane group g, the state
//    rows 32j + 8g + 4u + e (e = 0..3): the state's rows are permuted among
//    the tiles (srow below), which the products that write the state follow
//    by reading their A operand rows in the same order.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int C = kChunk;     // 64
constexpr int D = kHeadDim;   // 128
constexpr int NW = 8;         // waves per workgroup
constexpr int NT = 64 * NW;   // threads per workgroup
constexpr int PC = C + 8;     // bf16 row pitch of the [.][C] tiles Wt and Ot (144 B)
constexpr int PA = C + 16;    // bf16 row pitch of At (160 B: conflict-free transposing reads)

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

// State row held by element e of lane group g in state tile rt.
GDN_DEV int srow(int rt, int g, int e) { return 32 * (rt >> 1) + 8 * g + 4 * (rt & 1) + e; }

GDN_DEV u32x4_t join(u32x2_t a, u32x2_t b) {
    u32x4_t v;
    v[0] = a[0];
    v[1] = a[1];
    v[2] = b[0];
    v[3] = b[1];
    return v;
}

// Transposing LDS read: within each group of 16 lanes, output lane 4m+e gets
// element e of the 8-byte rows addressed by lanes m, m+4, m+8, m+12.
GDN_DEV u32x2_t lds_tr(const uint16_t *p) {
    const v4s_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(p));
    u32x2_t u;
    u[0] = (uint32_t)(uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16);
    u[1] = (uint32_t)(uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16);
    return u;
}

// B operand from two stacked accumulator tiles (k-slots 0..3 from lo, 4..7
// from hi), optionally scaled per row.
GDN_DEV bf16x8_t frag_acc(const f32x4_t &lo, const f32x4_t &hi) {
    u32x4_t u;
    u[0] = pack2_bf16_hw(lo[0], lo[1]);
    u[1] = pack2_bf16_hw(lo[2], lo[3]);
    u[2] = pack2_bf16_hw(hi[0], hi[1]);
    u[3] = pack2_bf16_hw(hi[2], hi[3]);
    return as_bf16x8(u);
}
GDN_DEV bf16x8_t frag_acc_scaled(const f32x4_t &lo, const f32x4_t &hi, const f32x4_t &slo,
                                 const f32x4_t &shi) {
    u32x4_t u;
    u[0] = pack2_bf16_hw(lo[0] * slo[0], lo[1] * slo[1]);
    u[1] = pack2_bf16_hw(lo[2] * slo[2], lo[3] * slo[3]);
    u[2] = pack2_bf16_hw(hi[0] * shi[0], hi[1] * shi[1]);
    u[3] = pack2_bf16_hw(hi[2] * shi[2], hi[3] * shi[3]);
    return as_bf16x8(u);
}

// ---------------------------------------------------------------------------
// 16x16x16 MFMA helpers.  Layout: A lane (g, r) = A[r][4g..4g+3],
// B lane (g, r) = B[4g..4g+3][r], C lane (g, r) = C[4g..4g+3][r].  So the
// accumulator of a 16x16 tile is the B operand of the next product, and the
// accumulator of X^T is the A operand of X: X Y = mfma(C(X^T), C(Y)).
// ---------------------------------------------------------------------------

GDN_DEV f32x4_t mfma16(s4_t a, s4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
GDN_DEV u32x2_t bf4u(const f32x4_t &x) {
    u32x2_t u;
    u[0] = pack2_bf16_hw(x[0], x[1]);
    u[1] = pack2_bf16_hw(x[2], x[3]);
    return u;
}
GDN_DEV s4_t bf4(const f32x4_t &x) { return __builtin_bit_cast(s4_t, bf4u(x)); }

// x = hi + lo with hi = bf16(x) and lo = bf16(x - hi): 16 significant bits.
GDN_DEV void split_bf(const f32x4_t &x, u32x2_t &hi, u32x2_t &lo) {
    hi = bf4u(x);
    f32x4_t r;
    r[0] = x[0] - __uint_as_float(hi[0] << 16);
    r[1] = x[1] - __uint_as_float(hi[0] & 0xFFFF0000u);
    r[2] = x[2] - __uint_as_float(hi[1] << 16);
    r[3] = x[3] - __uint_as_float(hi[1] & 0xFFFF0000u);
    lo = bf4u(r);
}

// c + X Y in fp32 for 16x16 tiles given as accumulators xt = C(X^T) and
// y = C(Y): four mfma_f32_16x16x4_f32 steps, step s taking k = 4g + s in lane
// group g, which is element s of both accumulator tiles.  The block inverse
// needs the full fp32 significand: its partial products (I + Z)(I + Z^2)...
// can exceed the final entries by several orders of magnitude (repeated
// keys, beta near 1) and cancel.
GDN_DEV f32x4_t mfma_f32x16(const f32x4_t &xt, const f32x4_t &y, f32x4_t c) {
#pragma unroll
    for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(xt[s], y[s], c, 0, 0, 0);
    return c;
}

// Inclusive prefix sum over the 64 lanes of a wavefront with DPP: shifts
// within rows of 16 lanes, then the last lane of row 0 (row_bcast:15) and of
// row 1 (row_bcast:31) carried into the rows after them.  Lanes whose source
// is outside the row, or whose row is masked off, add 0.
template <int CTRL, int ROW_MASK> GDN_DEV float dpp_src(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                   ROW_MASK, 0xF, false));
}
GDN_DEV float wave_incl_scan(float x) {
    x += dpp_src<0x111, 0xF>(x);  // row_shr:1
    x += dpp_src<0x112, 0xF>(x);  // row_shr:2
    x += dpp_src<0x114, 0xF>(x);  // row_shr:4
    x += dpp_src<0x118, 0xF>(x);  // row_shr:8
    x += dpp_src<0x142, 0xA>(x);  // row_bcast:15 into rows 1, 3
    x += dpp_src<0x143, 0xC>(x);  // row_bcast:31 into rows 2, 3
    return x;
}

// ---------------------------------------------------------------------------
// Shared memory and stage A
// ---------------------------------------------------------------------------

// Chunk tiles (k, q, v rows: [64][128] bf16) are written by direct
// global -> LDS loads, 1 KiB (4 rows) per wave instruction, unpadded.  The
// 16-byte piece c of row i is stored in slot c ^ fsw(i), with fsw swapping
// the two 2-bit halves of i mod 16: sixteen consecutive rows then hit
// sixteen different slots (row reads), and so do four consecutive rows x
// four pieces (the transposing reads of k^T).
GDN_DEV int fsw(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
GDN_DEV int sw(int row, int col) { return row * D + ((((col >> 3) ^ fsw(row)) << 3) | (col & 7)); }

struct Smem {
    uint16_t Kb[2][C * D];   // k rows, two buffers (chunk n and n+1)
    uint16_t Qb[2][C * D];   // q rows (output passes)
    uint16_t Vb[2][C * D];   // v rows
    float grb[2][C], btb[2][C];  // log-gates, beta
    uint16_t Wt[D][PC];   // -W^T  [d][i]
    uint16_t At[C][PA];   // A^T   [j][i]
    uint16_t Ot[D][PC];   // o^T of the chunk, staged for row stores
    u32x2_t Mf[6][64];    // A fragments of -M_ab (a > b), 16x16x16 layout
    u32x2_t Lf[4][64];    // A fragments of T_aa - I
    float G2[C], eG[C], eGl[C], bt[C], bg[C];  // G2 = G log2(e)
};

// The rows of one chunk in LDS.
struct ChunkView {
    const uint16_t *K, *Q, *V;
    const float *gr, *bt;
};
GDN_DEV ChunkView chunk_view(const Smem &sm, int buf) {
    return ChunkView{sm.Kb[buf], sm.Qb[buf], sm.Vb[buf], sm.grb[buf], sm.btb[buf]};
}

GDN_DEV int mf_index(int a, int b) { return a * (a - 1) / 2 + b; }  // a > b

// Per-lane element offsets of the direct loads within one chunk (fixed for a
// segment).  Wave w fills rows 8w .. 8w+7 of each tile, 4 rows per
// instruction: lane L of instruction j takes row i = 8w + 4j + L/16 and LDS
// slot L%16, i.e. piece c = (L%16) ^ fsw(i) of the row in HBM.
struct LoadPlan {
    int kq[2], v[2];  // row offset * row stride + 8c, for k/q and for v
    int row[2];       // i
};
GDN_DEV LoadPlan load_plan(int Hv, int Hk, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    LoadPlan lp;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = 8 * wave + 4 * j + (lane >> 4);
        const int c = (lane & 15) ^ fsw(i);
        lp.row[j] = i;
        lp.kq[j] = i * Hk * D + 8 * c;
        lp.v[j] = i * Hv * D + 8 * c;
    }
    return lp;
}

// Issue the direct loads of chunk n into buffer `buf` (completion: vmcnt).
// Rows past the sequence end read row T-1 and are zeroed later.  Waves 0 and
// 1 also load the 64 log-gates and betas (4 bytes per lane).
template <bool WITH_Q>
GDN_DEV void load_chunk(Smem &sm, int buf, const LoadPlan &lp, const uint16_t *q,
                        const uint16_t *k, const uint16_t *v, const float *g, const float *beta,
                        int b, int h, int kh, int n, int T, int Hv, int Hk, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const size_t t0 = (size_t)b * T + (size_t)n * C;   // first row of the chunk
    const uint16_t *kb = k + (t0 * Hk + kh) * D;
    const uint16_t *qb = q + (t0 * Hk + kh) * D;
    const uint16_t *vb = v + (t0 * Hv + h) * D;
    const bool tail = n * C + C > T;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i0 = 8 * wave + 4 * j;
        int okq = lp.kq[j], ov = lp.v[j];
        if (tail) {
            const int last = T - 1 - n * C;  // last row inside the sequence
            const int dr = min(lp.row[j], last) - lp.row[j];
            okq += dr * Hk * D;
            ov += dr * Hv * D;
        }
        __builtin_amdgcn_global_load_lds(kb + okq, (lds_void_t *)&sm.Kb[buf][i0 * D], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vb + ov, (lds_void_t *)&sm.Vb[buf][i0 * D], 16, 0, 0);
        if constexpr (WITH_Q)
            __builtin_amdgcn_global_load_lds(qb + okq, (lds_void_t *)&sm.Qb[buf][i0 * D], 16, 0, 0);
    }
    if (wave < 2) {
        const int tc = min(n * C + lane, T - 1);
        const float *src = (wave == 0 ? g : beta) + ((size_t)b * T + tc) * Hv + h;
        __builtin_amdgcn_global_load_lds(src, (lds_void_t *)(wave == 0 ? sm.grb[buf] : sm.btb[buf]),
                                         4, 0, 0);
    }
}

// Wait for this thread's outstanding global loads and stores (including the
// direct LDS loads).
GDN_DEV void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Workgroup barrier for LDS traffic only.  __syncthreads() is also a release
// fence for global memory, which would wait for the next chunk's direct loads
// at every barrier; here the waves only exchange data through LDS, so the
// barrier waits for this wave's LDS operations and nothing else.  Global
// visibility of the direct loads is established by wait_vmem() before the
// barrier that ends a chunk.
GDN_DEV void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Rows of chunk n past the sequence end read as zero (HF pads with zeros).
// Call between barriers, after the chunk's loads have landed.
template <bool WITH_Q>
GDN_DEV void zero_tail(Smem &sm, int buf, int n, int T, int tid) {
    const int valid = T - n * C;  // 1 .. 63
    for (int e = tid; e < (C - valid) * (D / 8); e += NT) {
        const int i = valid + e / (D / 8), c = e % (D / 8);
        const uint4 z = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4 *>(&sm.Kb[buf][i * D + 8 * c]) = z;
        *reinterpret_cast<uint4 *>(&sm.Vb[buf][i * D + 8 * c]) = z;
        if constexpr (WITH_Q) *reinterpret_cast<uint4 *>(&sm.Qb[buf][i * D + 8 * c]) = z;
    }
    if (tid >= valid && tid < C) {
        sm.grb[buf][tid] = 0.f;
        sm.btb[buf][tid] = 0.f;
    }
}

// Row-order operand of a swizzled chunk tile: element k = 8g + s of row
// row0 + r (one 16-byte read).
GDN_DEV bf16x8_t sfrag_nat(const uint16_t *base, int row0, int k0, int g, int r) {
    return as_bf16x8(*reinterpret_cast<const u32x4_t *>(base + sw(row0 + r, k0 + 8 * g)));
}

// A operand of K^T for the state update, k = t in the t order above and rows
// in state tile order: lane (g, r) gets K[k0 + {4g..4g+3, 16+4g..16+4g+3}]
// [d], d = the state row of tile rt held at row r (two transposing reads:
// source lane m + 4j addresses row k0 + 4g + j, columns 8m + .. of the
// tile's 32-block, so output lane 4m + e gets column 32 (rt>>1) + 8m +
// 4 (rt&1) + e).
GDN_DEV bf16x8_t kfrag_t(const uint16_t *base, int k0, int rt, int g, int r) {
    const int row = k0 + 4 * g + (r >> 2);
    const int col = 32 * (rt >> 1) + 8 * (r & 3) + 4 * (rt & 1);
    return as_bf16x8(join(lds_tr(base + sw(row, col)), lds_tr(base + sw(row + 16, col))));
}

// A operand of W for v = U - W S (rows t = 16 rt + r, k = d natural) from
// -W^T [d][t]: source lane m + 4j addresses row 32 kb + 8g + j (+4).
GDN_DEV bf16x8_t wfrag(const uint16_t (&Wt)[D][PC], int kb, int rt, int g, int r) {
    const uint16_t *p = &Wt[32 * kb + 8 * g + (r >> 2)][16 * rt + 4 * (r & 3)];
    return as_bf16x8(join(lds_tr(p), lds_tr(p + 4 * PC)));
}

// A operand of A for o += A v (rows i = 16 rt + r, k = j in t order) from
// A^T [j][i].
GDN_DEV bf16x8_t afrag(const uint16_t (&At)[C][PA], int kb, int rt, int g, int r) {
    const uint16_t *p = &At[32 * kb + 4 * g + (r >> 2)][16 * rt + 4 * (r & 3)];
    return as_bf16x8(join(lds_tr(p), lds_tr(p + 16 * PA)));
}

// Accumulator tile (rows row0 .. row0+15, columns col .. col+15) of a chunk
// tile, scaled per row by sc (rows row0 + 4g .. +3): one transposing read.
GDN_DEV f32x4_t rhs_tile(const uint16_t *base, int row0, int col, const f32x4_t &sc, int g, int r) {
    const u32x2_t w = lds_tr(base + sw(row0 + 4 * g + (r >> 2), col + 4 * (r & 3)));
    f32x4_t x;
    x[0] = __uint_as_float(w[0] << 16) * sc[0];
    x[1] = __uint_as_float(w[0] & 0xFFFF0000u) * sc[1];
    x[2] = __uint_as_float(w[1] << 16) * sc[2];
    x[3] = __uint_as_float(w[1] & 0xFFFF0000u) * sc[3];
    return x;
}

GDN_DEV f32x4_t lds_f4(const float *p) { return *reinterpret_cast<const f32x4_t *>(p); }

// Stage A for the chunk in view cv (landed and visible to all threads).
//  - wave 0 derives the gates: G = cumsum(g) (kept as G log2(e)), e^G,
//    e^{G_last - G}, beta, beta e^G;
//  - waves 0..3: row tile w of K K^T; waves 4..7 (output passes): row tile
//    w-4 of Q K^T;
//  - waves 0..3: K K^T is symmetric, so the upper tiles of its row tile give
//    the A operands of the lower blocks of M directly and the diagonal tile
//    gives both Z = -M_ww and Z^T.  The wave inverts its diagonal block,
//    T_ww = (I + Z)(I + Z^2)(I + Z^4)(I + Z^8) (Z is nilpotent), on fp32
//    MFMA.  Waves 4..7 write A^T;
//  - each wave solves (I + M) X = R by block rows for its right-hand sides:
//    W columns 16w .. 16w+15 (R = diag(beta e^G) K) and U columns
//    ucol0 .. ucol0 + 16 NUT - 1 (R = diag(beta) V), kept in registers;
//  - -W^T goes to LDS.
template <bool WITH_Q, int NUT, bool DO_U>
GDN_DEV void stage_a(Smem &sm, const ChunkView &cv, float q_scale, int tid, int ucol0,
                     f32x4_t (&U)[4][NUT]) {
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int rw = wave & 3;  // row tile of this wave's Gram product
    const bool gram = wave < 4 || WITH_Q;
    const bool kk_wave = wave < 4;

    if (wave == 0) {
        const float x = wave_incl_scan(cv.gr[lane]);
        const float glast = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
        const float eg = expf(x);
        sm.G2[lane] = x * 1.4426950408889634f;
        sm.eG[lane] = eg;
        sm.eGl[lane] = expf(glast - x);
        const float bv = cv.bt[lane];
        sm.bt[lane] = bv;
        sm.bg[lane] = bv * eg;
    }
    lds_barrier();
    f32x4_t acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = zero4();
    if (gram) {
        const uint16_t *X = kk_wave ? cv.K : cv.Q;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            const bf16x8_t ax = sfrag_nat(X, 16 * rw, 32 * kb, g, r);
            // all four column tiles: branch-free code lets the LDS reads run
            // ahead of the MFMAs (tiles outside the triangle are discarded)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
                acc[ct] = mfma_16x16x32_bf16(ax, sfrag_nat(cv.K, 16 * ct, 32 * kb, g, r), acc[ct]);
        }
    }

    if (gram) {
        // Gates of this lane's rows (16 rw + 4g + e) and columns (16 ct + r).
        // Every element below uses exactly one Gamma factor: exp(G_i - G_j)
        // where row i >= column j (A, Z) and exp(G_j - G_i) where j > i (the
        // transposed entries of M); masked elements take the other direction
        // and are discarded by the select.
        const f32x4_t Gw = lds_f4(&sm.G2[16 * rw + 4 * g]);
        float Gc[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) Gc[ct] = sm.G2[16 * ct + r];
        f32x4_t ga[4];  // ga[ct][e] = Gamma for row 16 rw + 4g + e, column 16 ct + r
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool lower = 16 * ct + r <= 16 * rw + 4 * g + e;
                ga[ct][e] = __builtin_amdgcn_exp2f(lower ? Gw[e] - Gc[ct] : Gc[ct] - Gw[e]);
            }
        if (!kk_wave) {
            // A^T [j][i] = scale Gamma_ij (q_i . k_j), j <= i; zero above
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                const int j = 16 * ct + r;
                f32x4_t av;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 16 * rw + 4 * g + e;
                    av[e] = (j <= i) ? q_scale * acc[ct][e] * ga[ct][e] : 0.f;
                }
                *reinterpret_cast<u32x2_t *>(&sm.At[j][16 * rw + 4 * g]) = bf4u(av);
            }
        } else {
            const f32x4_t Bw = lds_f4(&sm.bt[16 * rw + 4 * g]);
            float Bc[4];
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) Bc[ct] = sm.bt[16 * ct + r];
            // A fragments of -M_{a,rw}, a > rw: element e of lane (g, r) is
            // -M[16a + r][16 rw + 4g + e] = -beta Gamma (k.k) from tile (rw, a)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                if (ct > rw) {
                    f32x4_t m;
#pragma unroll
                    for (int e = 0; e < 4; ++e) m[e] = -Bc[ct] * ga[ct][e] * acc[ct][e];
                    sm.Mf[mf_index(ct, rw)][lane] = bf4u(m);
                }
            }
            // diagonal block: Z = -M_ww and Z^T as accumulator tiles (tile
            // ct = rw, selected without indexing registers by a runtime value)
            f32x4_t Z = zero4(), Zt = zero4(), I4;
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                if (ct == rw) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = 4 * g + e, j = r;
                        Z[e] = (i > j) ? -Bw[e] * ga[ct][e] * acc[ct][e] : 0.f;
                        Zt[e] = (j > i) ? -Bc[ct] * ga[ct][e] * acc[ct][e] : 0.f;
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) I4[e] = (4 * g + e == r) ? 1.f : 0.f;
            const f32x4_t Z2 = mfma_f32x16(Zt, Z, zero4());
            const f32x4_t Z2t = mfma_f32x16(Z, Zt, zero4());
            const f32x4_t Z4 = mfma_f32x16(Z2t, Z2, zero4());
            const f32x4_t Z4t = mfma_f32x16(Z2, Z2t, zero4());
            const f32x4_t Z8 = mfma_f32x16(Z4t, Z4, zero4());
            // T^T = (I + Z^8)^T (I + Z^4)^T (I + Z^2)^T (I + Z)^T, built up as
            // P^T <- P^T + (Z^k)^T P^T = P^T + mfma(C(Z^k), C(P^T))
            f32x4_t Pt = I4 + Zt;
            Pt = mfma_f32x16(Z2, Pt, Pt);
            Pt = mfma_f32x16(Z4, Pt, Pt);
            Pt = mfma_f32x16(Z8, Pt, Pt);
            sm.Lf[rw][lane] = bf4u(Pt - I4);  // A fragment of T - I
        }
    }
    lds_barrier();

    // block forward substitution: X_a = T_aa (R_a - sum_{b<a} M_ab X_b)
    f32x4_t Wx[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        Wx[a] = rhs_tile(cv.K, 16 * a, 16 * wave, lds_f4(&sm.bg[16 * a + 4 * g]), g, r);  // beta e^G
        if constexpr (DO_U) {
            const f32x4_t su = lds_f4(&sm.bt[16 * a + 4 * g]);  // beta
#pragma unroll
            for (int t = 0; t < NUT; ++t) U[a][t] = rhs_tile(cv.V, 16 * a, ucol0 + 16 * t, su, g, r);
        }
#pragma unroll
        for (int b = 0; b < a; ++b) {
            const s4_t am = __builtin_bit_cast(s4_t, sm.Mf[mf_index(a, b)][lane]);
            Wx[a] = mfma16(am, bf4(Wx[b]), Wx[a]);
            if constexpr (DO_U) {
#pragma unroll
                for (int t = 0; t < NUT; ++t) U[a][t] = mfma16(am, bf4(U[b][t]), U[a][t]);
            }
        }
        const s4_t al = __builtin_bit_cast(s4_t, sm.Lf[a][lane]);
        Wx[a] = mfma16(al, bf4(Wx[a]), Wx[a]);
        if constexpr (DO_U) {
#pragma unroll
            for (int t = 0; t < NUT; ++t) U[a][t] = mfma16(al, bf4(U[a][t]), U[a][t]);
        }
    }
    // -W^T [d][i]
#pragma unroll
    for (int a = 0; a < 4; ++a)
        *reinterpret_cast<u32x2_t *>(&sm.Wt[16 * wave + r][16 * a + 4 * g]) = bf4u(-Wx[a]);
    lds_barrier();
}

// ---------------------------------------------------------------------------
// State I/O
// ---------------------------------------------------------------------------

template <int FMT> GDN_DEV float state_ld(const void *S, size_t i) {
    if constexpr (FMT == kF16) return f16_to_f32(static_cast<const uint16_t *>(S)[i]);
    else return static_cast<const float *>(S)[i];
}
template <int FMT> GDN_DEV void state_st(void *S, size_t i, float x) {
    if constexpr (FMT == kF16) static_cast<uint16_t *>(S)[i] = f32_to_f16_rne(x);
    else static_cast<float *>(S)[i] = x;
}

// State tiles of a [128][NCT*16] column block of a row-major [128][128]
// matrix at column c0: tile (rt, ct), lane (g, r), element e is row
// srow(rt, g, e), column c0 + 16 ct + r.
template <int FMT, int NCT>
GDN_DEV void tiles_load(f32x4_t (&S)[8][NCT], const void *src, int c0, int g, int r) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                S[rt][ct][e] = state_ld<FMT>(src, (size_t)srow(rt, g, e) * D + c0 + 16 * ct + r);
}
template <int FMT, int NCT>
GDN_DEV void tiles_store(const f32x4_t (&S)[8][NCT], void *dst, int c0, int g, int r) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                state_st<FMT>(dst, (size_t)srow(rt, g, e) * D + c0 + 16 * ct + r, S[rt][ct][e]);
}

// Per (sequence, head): slot p of the carry buffer holds, for segment p,
// S_start (p >= 1), Phi and C (1 <= p <= P-2), each [128][128] fp32.
GDN_DEV float *carry_slot(float *carry, int b, int h, int Hv, int P, int p, int which) {
    return carry + ((((size_t)b * Hv + h) * P + p) * 3 + which) * (size_t)(D * D);
}
GDN_DEV const float *carry_slot(const float *carry, int b, int h, int Hv, int P, int p, int which) {
    return carry + ((((size_t)b * Hv + h) * P + p) * 3 + which) * (size_t)(D * D);
}
constexpr int kSst = 0, kPhi = 1, kCst = 2;

// ---------------------------------------------------------------------------
// Segment kernels
// ---------------------------------------------------------------------------

struct SegArgs {
    const uint16_t *q, *k, *v;
    const float *g, *beta;
    uint16_t *o;
    void *S;          // initial state in, final state out
    float *carry;
    int T, Hv, Hk, NC, L, P;
    float q_scale;
};

// The recurrence with output over chunks [n0, n1) of one (b, h), from the
// state `S` in registers (wave w owns columns 16w .. 16w+15).
GDN_DEV void run_output_segment(Smem &sm, f32x4_t (&S)[8][1], const SegArgs &a, int b, int h,
                                int n0, int n1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int kh = h / (a.Hv / a.Hk);
    const int c0 = 16 * wave;
    const LoadPlan lp = load_plan(a.Hv, a.Hk, tid);
    load_chunk<true>(sm, 0, lp, a.q, a.k, a.v, a.g, a.beta, b, h, kh, n0, a.T, a.Hv, a.Hk, tid);
    wait_vmem();
    lds_barrier();
    for (int n = n0; n < n1; ++n) {
        const int buf = (n - n0) & 1;
        if (n * C + C > a.T) {  // last, partial chunk
            zero_tail<true>(sm, buf, n, a.T, tid);
            lds_barrier();
        }
        if (n + 1 < n1)  // the next chunk's rows stream into the other buffer
            load_chunk<true>(sm, buf ^ 1, lp, a.q, a.k, a.v, a.g, a.beta, b, h, kh, n + 1, a.T, a.Hv,
                             a.Hk, tid);
        const ChunkView cv = chunk_view(sm, buf);
        // v starts as U = T diag(beta) V (this wave's columns), o as 0
        f32x4_t vacc[4][1], oacc[4];
        stage_a<true, 1, true>(sm, cv, a.q_scale, tid, c0, vacc);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) oacc[rt] = zero4();
        // v -= W S ;  o = q S
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            const bf16x8_t sb = frag_acc(S[2 * kb][0], S[2 * kb + 1][0]);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                vacc[rt][0] = mfma_16x16x32_bf16(wfrag(sm.Wt, kb, rt, g, r), sb, vacc[rt][0]);
                oacc[rt] = mfma_16x16x32_bf16(sfrag_nat(cv.Q, 16 * rt, 32 * kb, g, r), sb, oacc[rt]);
            }
        }
        // o = e^G scale (q S) + A v
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const f32x4_t eg = lds_f4(&sm.eG[16 * rt + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) oacc[rt][e] *= a.q_scale * eg[e];
        }
#pragma unroll
        for (int kb = 0; kb < C / 32; ++kb) {
            const bf16x8_t vb = frag_acc(vacc[2 * kb][0], vacc[2 * kb + 1][0]);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
                oacc[rt] = mfma_16x16x32_bf16(afrag(sm.At, kb, rt, g, r), vb, oacc[rt]);
        }
        // o -> HBM through LDS: each wave writes its columns of o^T (4 rows of
        // one column per 8-byte write), reads them back transposed (row t,
        // 8 consecutive columns per lane) and stores 16 B per lane.  Only this
        // wave touches its columns, so no barrier is needed.
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
            *reinterpret_cast<u32x2_t *>(&sm.Ot[c0 + r][16 * rt + 4 * g]) = bf4u(oacc[rt]);
        {
            const int t = n * C + 16 * g + r;   // lane (g, r) stores row 16g + r
            uint16_t *orow = a.o + (((size_t)b * a.T + t) * a.Hv + h) * D + c0;
#pragma unroll
            for (int qd = 0; qd < 2; ++qd) {
                const uint16_t *src = &sm.Ot[c0 + 8 * qd + (r >> 2)][16 * g + 4 * (r & 3)];
                const u32x4_t w = join(lds_tr(src), lds_tr(src + 4 * PC));
                if (t < a.T) *reinterpret_cast<u32x4_t *>(orow + 8 * qd) = w;
            }
        }
        // S = e^{G_last} S + K^T diag(e^{G_last - G}) v
        {
            const float gam = sm.eG[C - 1];
#pragma unroll
            for (int rt = 0; rt < 8; ++rt)
#pragma unroll
                for (int e = 0; e < 4; ++e) S[rt][0][e] *= gam;
#pragma unroll
            for (int kb = 0; kb < C / 32; ++kb) {
                const bf16x8_t vg = frag_acc_scaled(vacc[2 * kb][0], vacc[2 * kb + 1][0],
                                                    lds_f4(&sm.eGl[32 * kb + 4 * g]),
                                                    lds_f4(&sm.eGl[32 * kb + 16 + 4 * g]));
#pragma unroll
                for (int rt = 0; rt < 8; ++rt)
                    S[rt][0] = mfma_16x16x32_bf16(kfrag_t(cv.K, 32 * kb, rt, g, r), vg, S[rt][0]);
            }
        }
        wait_vmem();      // the next chunk's rows have landed
        lds_barrier();    // and this chunk's buffer may be refilled
    }
}

// Middle segment of pass 1: the recurrence from S = 0 on state columns
// 0..127 (waves 0..3) and from Phi = I with U = 0 on 128 more columns
// (waves 4..7), without output.  Wave w owns columns 32 (w & 3) .. +31 of
// its block.
GDN_DEV void run_transition_segment(Smem &sm, const SegArgs &a, int b, int h, int p, int n0,
                                    int n1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int kh = h / (a.Hv / a.Hk);
    const LoadPlan lp = load_plan(a.Hv, a.Hk, tid);
    const bool is_phi = wave >= 4;
    const int c0 = 32 * (wave & 3);   // column of the S or Phi block
    f32x4_t X[8][2];
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                X[rt][ct][e] = (is_phi && srow(rt, g, e) == c0 + 16 * ct + r) ? 1.f : 0.f;

    load_chunk<false>(sm, 0, lp, a.q, a.k, a.v, a.g, a.beta, b, h, kh, n0, a.T, a.Hv, a.Hk, tid);
    wait_vmem();
    lds_barrier();
    for (int n = n0; n < n1; ++n) {
        const int buf = (n - n0) & 1;
        if (n * C + C > a.T) {
            zero_tail<false>(sm, buf, n, a.T, tid);
            lds_barrier();
        }
        if (n + 1 < n1)
            load_chunk<false>(sm, buf ^ 1, lp, a.q, a.k, a.v, a.g, a.beta, b, h, kh, n + 1, a.T, a.Hv,
                              a.Hk, tid);
        const ChunkView cv = chunk_view(sm, buf);
        // v starts as U (state waves) or 0 (transition waves)
        f32x4_t vacc[4][2];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) vacc[rt][ct] = zero4();
        if (is_phi)
            stage_a<false, 2, false>(sm, cv, a.q_scale, tid, c0, vacc);
        else
            stage_a<false, 2, true>(sm, cv, a.q_scale, tid, c0, vacc);
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t xb[2];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) xb[ct] = frag_acc(X[2 * kb][ct], X[2 * kb + 1][ct]);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const bf16x8_t aw = wfrag(sm.Wt, kb, rt, g, r);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) vacc[rt][ct] = mfma_16x16x32_bf16(aw, xb[ct], vacc[rt][ct]);
            }
        }
        {
            const float gam = sm.eG[C - 1];
#pragma unroll
            for (int rt = 0; rt < 8; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int e = 0; e < 4; ++e) X[rt][ct][e] *= gam;
#pragma unroll
            for (int kb = 0; kb < C / 32; ++kb) {
                const f32x4_t slo = lds_f4(&sm.eGl[32 * kb + 4 * g]);
                const f32x4_t shi = lds_f4(&sm.eGl[32 * kb + 16 + 4 * g]);
                bf16x8_t vg[2];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    vg[ct] = frag_acc_scaled(vacc[2 * kb][ct], vacc[2 * kb + 1][ct], slo, shi);
#pragma unroll
                for (int rt = 0; rt < 8; ++rt) {
                    const bf16x8_t ak = kfrag_t(cv.K, 32 * kb, rt, g, r);
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) X[rt][ct] = mfma_16x16x32_bf16(ak, vg[ct], X[rt][ct]);
                }
            }
        }
        wait_vmem();
        lds_barrier();
    }
    tiles_store<kF32, 2>(X, carry_slot(a.carry, b, h, a.Hv, a.P, p, is_phi ? kPhi : kCst), c0, g, r);
}

// Start state of segment p >= 1 of pass 2, composed by the workgroup itself:
// S_start(1) = the end state of segment 0 (in the carry); for q = 1 .. p-1,
// S_start(q+1) = Phi_q S_start(q) + C_q.  Phi_{q+1} streams from the carry
// into an fp32 LDS buffer by direct loads (and C_{q+1} into registers) while
// step q computes; at the start of a step the threads split the staged Phi
// into bf16 hi and lo halves, so every wave reads MFMA-ready A fragments; the
// product is hi*hi + hi*lo + lo*hi (near-fp32 accuracy).  Wave w keeps
// columns 16w .. 16w+15, as the output pass does.  The halves are unpadded
// [128][128] tiles with the 16-byte piece c of row i in slot c ^ csw(i):
// the sixteen rows of one state tile land in sixteen different slots.
struct CombSmem {
    float raw[D * D];       // Phi as loaded, row-major fp32
    uint16_t hi[D * D];
    uint16_t lo[D * D];
};
GDN_DEV int csw(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
GDN_DEV int cidx(int row, int col) { return row * D + ((((col >> 3) ^ csw(row)) << 3) | (col & 7)); }

// Direct loads of one 64 KiB Phi: wave w moves kilobytes 8w .. 8w+7.
GDN_DEV void comb_fetch(CombSmem &sm, const float *phi, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int blk = 8 * wave + j;  // 1 KiB = 256 floats
        __builtin_amdgcn_global_load_lds(phi + blk * 256 + 4 * lane, (lds_void_t *)&sm.raw[blk * 256],
                                         16, 0, 0);
    }
}

GDN_DEV void combine_prefix(CombSmem &sm, f32x4_t (&S)[8][1], const float *carry, int b, int h,
                            int Hv, int P, int p, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int c0 = 16 * wave;
    tiles_load<kF32, 1>(S, carry_slot(carry, b, h, Hv, P, 1, kSst), c0, g, r);
    if (p < 2) return;
    f32x4_t cn[8][1];
    tiles_load<kF32, 1>(cn, carry_slot(carry, b, h, Hv, P, 1, kCst), c0, g, r);
    comb_fetch(sm, carry_slot(carry, b, h, Hv, P, 1, kPhi), tid);
    wait_vmem();
    lds_barrier();
    for (int q = 1; q < p; ++q) {
#pragma unroll 4
        for (int j = 0; j < (D * D) / (4 * NT); ++j) {
            const int it = tid + NT * j;
            const int row = it >> 5, col = (it & 31) * 4;
            const f32x4_t x = *reinterpret_cast<const f32x4_t *>(&sm.raw[row * D + col]);
            u32x2_t xh, xl;
            split_bf(x, xh, xl);
            *reinterpret_cast<u32x2_t *>(&sm.hi[cidx(row, col)]) = xh;
            *reinterpret_cast<u32x2_t *>(&sm.lo[cidx(row, col)]) = xl;
        }
        lds_barrier();  // halves ready, raw buffer free
        f32x4_t acc[8];
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) acc[rt] = cn[rt][0];
        if (q + 1 < p) {  // next step's operands stream in during this one
            comb_fetch(sm, carry_slot(carry, b, h, Hv, P, q + 1, kPhi), tid);
            tiles_load<kF32, 1>(cn, carry_slot(carry, b, h, Hv, P, q + 1, kCst), c0, g, r);
        }
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            u32x2_t h0, l0, h1, l1;
            split_bf(S[2 * kb][0], h0, l0);
            split_bf(S[2 * kb + 1][0], h1, l1);
            const bf16x8_t sbh = as_bf16x8(join(h0, h1)), sbl = as_bf16x8(join(l0, l1));
#pragma unroll
            for (int rt = 0; rt < 8; ++rt) {
                // output row r of tile rt is state row srow(rt, r >> 2, r & 3)
                const int row = srow(rt, r >> 2, r & 3);
                const bf16x8_t ah = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.hi[cidx(row, 32 * kb + 8 * g)]));
                const bf16x8_t al = as_bf16x8(*reinterpret_cast<const u32x4_t *>(&sm.lo[cidx(row, 32 * kb + 8 * g)]));
                acc[rt] = mfma_16x16x32_bf16(ah, sbh, acc[rt]);
                acc[rt] = mfma_16x16x32_bf16(ah, sbl, acc[rt]);
                acc[rt] = mfma_16x16x32_bf16(al, sbh, acc[rt]);
            }
        }
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) S[rt][0] = acc[rt];
        wait_vmem();    // the next Phi has landed
        lds_barrier();  // and every wave is done with the halves
    }
}

// Pass 1: slot p = blockIdx.y < P-1.  Segment 0 runs the output recurrence
// from the initial state; segments 1 .. P-2 their transition.
template <int IN_FMT, int OUT_FMT>
__global__ __launch_bounds__(NT) void prefill_pass1_kernel(SegArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
    const int h = blockIdx.x, p = blockIdx.y, b = blockIdx.z;
    const int n0 = p * a.L, n1 = min(a.NC, n0 + a.L);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    if (p == 0) {
        f32x4_t S[8][1];
        void *Sg = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (IN_FMT == kF16 ? 2 : 4);
        tiles_load<IN_FMT, 1>(S, Sg, 16 * wave, g, r);
        run_output_segment(sm, S, a, b, h, n0, n1);
        if (a.P == 1) {
            void *So = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (OUT_FMT == kF16 ? 2 : 4);
            tiles_store<OUT_FMT, 1>(S, So, 16 * wave, g, r);
        } else {
            tiles_store<kF32, 1>(S, carry_slot(a.carry, b, h, a.Hv, a.P, 1, kSst), 16 * wave, g, r);
        }
    } else {
        run_transition_segment(sm, a, b, h, p, n0, n1);
    }
}

// Pass 2: slot blockIdx.y -> segment p = blockIdx.y + 1, from S_start(p),
// which the workgroup first composes from the pass-1 results.
template <int OUT_FMT>
__global__ __launch_bounds__(NT) void prefill_pass2_kernel(SegArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
    const int h = blockIdx.x, p = blockIdx.y + 1, b = blockIdx.z;
    const int n0 = p * a.L, n1 = min(a.NC, n0 + a.L);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r = lane & 15;
    f32x4_t S[8][1];
    combine_prefix(*reinterpret_cast<CombSmem *>(smem_raw), S, a.carry, b, h, a.Hv, a.P, p,
                   threadIdx.x);
    run_output_segment(sm, S, a, b, h, n0, n1);
    if (p == a.P - 1) {
        void *So = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (OUT_FMT == kF16 ? 2 : 4);
        tiles_store<OUT_FMT, 1>(S, So, 16 * wave, g, r);
    }
}

// Segments: enough middle segments that a pass fills the device (about 256
// workgroups), at least kMinSegChunks chunks each; P = 2 would only
// serialise, so it falls back to 1.
constexpr int kMinSegChunks = 8;
constexpr int kTargetWgs = 256;

void plan_segments(int B, int Hv, int NC, int &P, int &L) {
    const int bh = B * Hv;
    int want = 1 + (kTargetWgs + bh - 1) / bh;
    const int cap = NC / kMinSegChunks;
    if (want > cap) want = cap;
    if (want < 3) want = 1;
    P = want;
    L = (NC + P - 1) / P;
    P = (NC + L - 1) / L;  // drop empty trailing segments
    if (P < 3) {
        P = 1;
        L = NC;
    }
}

}  // namespace

size_t prefill_carry_bytes(int B, int T, int Hv) {
    const int NC = (T + C - 1) / C;
    int P, L;
    plan_segments(B, Hv, NC, P, L);
    return P > 1 ? (size_t)B * Hv * P * 3 * D * D * sizeof(float) : 0;
}

hipError_t launch_prefill_seq(int narrow_state, const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, const float *g, const float *beta, uint16_t *o,
                              void *S, int B, int T, int Hv, int Hk, float q_scale, void *carry,
                              hipStream_t st) {
    if (B <= 0 || T <= 0) return hipSuccess;
    if (Hv <= 0 || Hk <= 0 || Hv % Hk) return hipErrorInvalidValue;
    const int NC = (T + C - 1) / C;
    SegArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.g = g;
    a.beta = beta;
    a.o = o;
    a.S = S;
    a.carry = static_cast<float *>(carry);
    a.T = T;
    a.Hv = Hv;
    a.Hk = Hk;
    a.NC = NC;
    a.q_scale = q_scale;
    plan_segments(B, Hv, NC, a.P, a.L);
    if (a.P > 1 && !carry) return hipErrorInvalidValue;
    static_assert(sizeof(CombSmem) <= sizeof(Smem), "the start-state staging reuses the chunk LDS");
    const size_t smem = sizeof(Smem);
    auto pass1 = narrow_state == kF16 ? prefill_pass1_kernel<kF16, kF16> : prefill_pass1_kernel<kF32, kF32>;
    auto pass2 = narrow_state == kF16 ? prefill_pass2_kernel<kF16> : prefill_pass2_kernel<kF32>;
    static bool attr_set = false;  // idempotent; races only repeat the same call
    if (!attr_set) {
        hipError_t e;
        for (auto f : {prefill_pass1_kernel<kF32, kF32>, prefill_pass1_kernel<kF16, kF16>})
            if ((e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)smem)) != hipSuccess)
                return e;
        for (auto f : {prefill_pass2_kernel<kF32>, prefill_pass2_kernel<kF16>})
            if ((e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)smem)) != hipSuccess)
                return e;
        attr_set = true;
    }
    const int slots = a.P > 1 ? a.P - 1 : 1;
    pass1<<<dim3(Hv, slots, B), NT, smem, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.P == 1) return e;
    pass2<<<dim3(Hv, a.P - 1, B), NT, smem, st>>>(a);
    return hipGetLastError();
}

}  // namespace gdn

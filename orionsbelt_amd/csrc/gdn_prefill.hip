// gdn_prefill.hip -- chunkwise (WY) gated delta rule prefill for gfx950,
// parallel over the sequence.
//
// Algorithm: HF torch_chunk_gated_delta_rule (transformers
// modeling_qwen3_5.py:248-328), chunk size 64, head dims 128.  Per (sequence
// b, value head h, chunk n) with G = cumsum(g) inside the chunk and
// Gamma_ij = exp(G_i - G_j) (i >= j):
//   M = tril(beta_i (k_i . k_j) Gamma_ij, -1)       T = (I + M)^-1
//   A = tril(Gamma_ij (q_i . k_j)) * scale
// and, sequentially over chunks, with S the [128 x 128] state:
//   v_new = U - W S = T diag(beta) (V - diag(e^G) K S)
//   o = scale e^G (q S) + A v_new
//   S' = e^{G_last} S + K^T diag(e^{G_last - G}) v_new
// HF forms U = T diag(beta) V and W = T diag(beta e^G) K first
// (modeling_qwen3_5.py:299-300); the product is regrouped here so that the
// chunk's 64x64 T multiplies one right-hand side, after the K S product.
//
// Parallel over the sequence.  The step is affine in S:
//   S' = Phi_n S + C_n,  Phi_n = e^{G_last} I - K^T diag(e^{G_last-G}) W,
//   C_n = K^T diag(e^{G_last-G}) U,
// so the chunks are cut into P segments and
//   pass 1: segment 0 runs the recurrence from the initial state (with o);
//           every middle segment p runs it from S = 0 and, alongside, on
//           128 more state columns started at I with V = 0, which yields its
//           local result C_p and its transition Phi_p;
//   pass 2: segment p = 1 .. P-1 first composes its start state,
//           S_start(q+1) = Phi_q S_start(q) + C_q from S_start(1) = the end of
//           segment 0, then reruns the recurrence from it, with o.
// Where the gates let the state forget within a few chunks (checked on the
// device per sequence and head, before pass 1), a head instead runs its
// segments independently in pass 1, each from S = 0 a short window before
// its first output chunk ("windowed segments", below).
//
// Workgroup: 8 waves in two roles, one of each role per SIMD.
//  - State waves 0..3 own 32 state columns each (48 of the 256 in a
//    transition segment, where helpers 1 and 2 own the last 32 columns of
//    C and of Phi) in VGPRs and run the S-dependent products of chunk n:
//    P = K S and O = Q S (phase 1), then v = T diag(beta)(V - e^G P),
//    o^T = e^G scale O^T + v^T A^T and the state update (phase 2).
//  - Helper waves 4..7 prepare the S-independent operands one chunk ahead
//    and stream the chunk tiles.  While the state waves are in phase 1 of
//    chunk n, helper 0 finishes T of chunk n (the off-diagonal 16x16 blocks
//    on MFMA), helpers 1 and 2 form K K^T of chunk n+1 and write M, and
//    helper 3 issues tile loads.  In phase 2, helper 0 starts T of chunk
//    n+1 (forward substitution of the diagonal blocks of M on the VALU),
//    helpers 1 and 3 form K Q^T of chunk n+1 (the A fragments), and helper 2
//    issues tile loads.
//  Two LDS barriers per chunk separate the phases, so the MFMA-heavy state
//  work of one role overlaps the latency-bound work of the other.
//
// Loads: helpers 2 and 3 move chunk tiles straight from HBM into LDS
// (global_load_lds_dwordx4, 1 KiB per wave instruction): the k and q rows,
// gates and betas of chunk n+2 and the v rows of chunk n+1, each at least
// one phase before the barrier that publishes it (helper 3 alone in a
// transition segment).
// Rows past the sequence end read its last row (their values are
// multiplied by beta = 0 or never stored).
//
// Fragment orders.  The 32 k-indices of one 16x16x32 MFMA may be assigned
// to lanes in any order as long as both operands use the same order.
//  - k = t (a chunk row): lane group g holds t = {4g..4g+3, 16+4g..16+4g+3}
//    of a 32-block ("t order"), which is the accumulator layout of two
//    stacked 16 x 16 tiles (lane group g holds rows 4g..4g+3 of each), so an
//    accumulator feeds the next products straight from registers, as the
//    B operand and, for its transpose, as the A operand.
//  - k = d (a state row): lane group g holds d = 8g..8g+7 of a 32-block, the
//    natural order, so q and k rows are read with one 16-byte LDS read per
//    lane.  For that, state tile 2j + u holds, in lane group g, the state
//    rows 32j + 8g + 4u + e (e = 0..3): the state's rows are permuted among
//    the tiles (srow below), which the products that write the state follow
//    by reading their A operand rows in the same order.

#include <algorithm>

#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int C = kChunk;     // 64
constexpr int D = kHeadDim;   // 128
constexpr int NW = 8;         // waves per workgroup
constexpr int NT = 64 * NW;   // threads per workgroup
constexpr int NSW = 4;        // state waves (the first four)
constexpr int kMaxSegs = 64;  // segments of one sequence
constexpr float kLog2e = 1.4426950408889634f;

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
// accumulator of X^T is the A operand of X.
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

// B operand pair (hi, lo) of two stacked accumulator tiles: hi + lo carries
// 16 significant bits of each element.
GDN_DEV void frag_acc_split(const f32x4_t &lo_tile, const f32x4_t &hi_tile, bf16x8_t &hi, bf16x8_t &lo) {
    u32x2_t ah, al, bh, bl;
    split_bf(lo_tile, ah, al);
    split_bf(hi_tile, bh, bl);
    hi = as_bf16x8(join(ah, bh));
    lo = as_bf16x8(join(al, bl));
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

// Index of this wave in the workgroup, as a wave-uniform (scalar) value, so
// that branches on a wave's role compile to scalar branches.
GDN_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// 4 x 4 transpose of (16-lane row, register): afterwards x[b] row g holds
// what x[g] row b held.  v_permlane32_swap exchanges the upper two rows of
// its first operand with the lower two of its second, v_permlane16_swap the
// odd rows of the first with the even rows of the second.
GDN_DEV void row_transpose4(u32x4_t &x) {
    auto s02 = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
    auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    x[0] = s01[0];
    x[1] = s01[1];
    x[2] = s23[0];
    x[3] = s23[1];
}

// Wait for this wave's outstanding LDS operations and order the compiler's
// LDS accesses around the wait (a wave reads back what it wrote itself).
GDN_DEV void lds_fence() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier for LDS traffic only.  __syncthreads() is also a release
// fence for global memory, which would wait for outstanding direct loads at
// every barrier; here the waves exchange data only through LDS, so the
// barrier waits for this wave's LDS operations and nothing else.  Direct
// loads become visible to other waves once their issuing wave has waited
// for them (vmcnt) before a barrier.
GDN_DEV void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// vmcnt(n): at most n of this wave's vector memory operations outstanding.
GDN_DEV void wait_vmem0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---------------------------------------------------------------------------
// Shared memory
// ---------------------------------------------------------------------------

// Chunk tiles (k, q, v rows: [64][128] bf16) are written by direct
// global -> LDS loads, 1 KiB (4 rows) per wave instruction, unpadded.  The
// 16-byte piece c of row i is stored in slot c ^ fsw(i), with fsw swapping
// the two 2-bit halves of i mod 16: sixteen consecutive rows then hit
// sixteen different slots (row reads), and so do four consecutive rows x
// four pieces (the transposing reads of k^T).
GDN_DEV int fsw(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
GDN_DEV int sw(int row, int col) { return row * D + ((((col >> 3) ^ fsw(row)) << 3) | (col & 7)); }

// Per-chunk gates for the state waves.
struct Gates {
    float bt[C];    // beta (0 past the sequence end)
    float eg[C];    // e^{G}
    float egl[C];   // e^{G_last - G}
    float seg[C];   // scale e^{G}
    float gam;      // e^{G_last}
    float mnorm;    // largest column sum of |M| (the matrix 1-norm), NaN if M is not finite
    float pad[2];
};

// Fragments of the lower block triangle of a 64x64 matrix X for 16x16x32
// MFMA with k in t order: fragment (rt, kb) (rt = 0..3, kb <= rt/2), lane
// (g, r), slots 4h + e hold X[16 rt + r][32 kb + 16 h + 4 g + e], i.e. half
// h of the fragment is the 16x16x16 A layout of block (rt, 2 kb + h).  The
// upper blocks (0, 1) and (2, 3) are zero and are never written after set-up.
GDN_DEV constexpr int fidx(int rt, int kb) { return rt < 2 ? rt : 2 * rt - 2 + kb; }
// M blocks (a >= b), fp32 row-major 16x16.
GDN_DEV constexpr int mbi(int a, int b) { return a * (a + 1) / 2 + b; }

// Floats per column of an M block in LDS: 16 rows + 4 pad, so that the
// 16-byte accesses of lanes that walk the columns (a 16-float stride would
// put every second column on the same four banks) cover the 32 banks once
// per 8 lanes.
constexpr int kMbPitch = 20;

struct Smem {
    uint16_t Kb[3][C * D];   // k rows of chunks n, n+1, n+2
    uint16_t Qb[2][C * D];   // q rows (output segments)
    uint16_t Vb[2][C * D];   // v rows
    float graw[2][C], braw[2][C];  // log-gates and betas as loaded
    Gates gt[2];
    u32x4_t Af[2][6][64];    // A fragments (output segments), two chunks
    u32x4_t Tf[2][6][64];    // (T - I) fragments, two chunks
    float Mb[10][16 * kMbPitch];  // M blocks of the next chunk, fp32 column-major:
                                  // Mb[.][kMbPitch j + i] = M[i][j]
    float hg[4][2][C];       // per helper wave: G log2(e) and beta of its chunk
};

// ---------------------------------------------------------------------------
// Loads
// ---------------------------------------------------------------------------

// Row 0 of chunk ci of head `head` of a [B][T][H][128] tensor.
GDN_DEV const uint16_t *chunk_rows(const uint16_t *x, int H, int head, int b, int ci, int T) {
    return x + (((size_t)b * T + (size_t)ci * C) * H + head) * D;
}
// Log-gates (helpers 0, 1) or betas (2, 3), 32 tokens each.
GDN_DEV void load_gates(Smem &sm, int slot, const float *g, const float *beta, int b, int h, int Hv,
                        int ci, int T, int hw, int lane) {
    if (lane < 32) {
        const int t = 32 * (hw & 1) + lane;
        const int tc = min(ci * C + t, T - 1);
        const float *src = (hw < 2 ? g : beta) + ((size_t)b * T + tc) * Hv + h;
        float *dst = (hw < 2 ? sm.graw[slot] : sm.braw[slot]) + 32 * (hw & 1);
        __builtin_amdgcn_global_load_lds(src, (lds_void_t *)dst, 4, 0, 0);
    }
}

// All 64 log-gates (which = 0) or betas (which = 1) of chunk ci: one
// instruction.
GDN_DEV void load_gates_all(Smem &sm, int slot, const float *x, int b, int h, int Hv, int ci, int T,
                            int which, int lane) {
    const int tc = min(ci * C + lane, T - 1);
    __builtin_amdgcn_global_load_lds(x + ((size_t)b * T + tc) * Hv + h,
                                     (lds_void_t *)(which == 0 ? sm.graw[slot] : sm.braw[slot]), 4, 0, 0);
}

// Rows r0 .. r0 + 4 NJ - 1 of chunk ci of one head of a [B][T][H][128]
// tensor into its swizzled LDS tile (NJ instructions; offsets computed here:
// the wave that issues these loads has the time).
template <int NJ>
GDN_DEV void load_rows_n(uint16_t *tile, const uint16_t *x, int H, int head, int b, int ci, int T, int r0,
                         int lane) {
    const int valid = min(C, T - ci * C);
    const uint16_t *rows = chunk_rows(x, H, head, b, ci, T);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int i = r0 + 4 * j + (lane >> 4);
        const int c = (lane & 15) ^ fsw(i);
        const int ii = min(i, valid - 1);
        __builtin_amdgcn_global_load_lds(rows + (size_t)ii * H * D + 8 * c,
                                         (lds_void_t *)&tile[(r0 + 4 * j) * D], 16, 0, 0);
    }
}

// ---------------------------------------------------------------------------
// Operand readers
// ---------------------------------------------------------------------------

// The lane index, opaque to the optimiser: offsets derived from it inside a
// loop are recomputed there (a few VALU operations) instead of being kept
// live in VGPRs across the loop.
GDN_DEV int opaque_lane(int lane) {
    __asm__ volatile("" : "+v"(lane));
    return lane;
}

// Per-lane element offsets into a swizzled [64][128] chunk tile.  The
// swizzle permutes the 16-byte pieces of a row by a function of the row's
// low 4 bits only, so moving by 16 rows or by 32 columns adds a constant:
// each operand below is one of four per-lane offsets plus an immediate.
struct TileOffs {
    int nat[4];  // row r, columns 32 kb + 8 g .. +7
    int tr[4];   // row 4 g + r/4, 8-byte piece at column 32 q + 8 (r & 3)
};
GDN_DEV TileOffs tile_offs(int g, int r) {
    TileOffs o;
    const int row = 4 * g + (r >> 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        o.nat[j] = sw(r, 32 * j + 8 * g);
        o.tr[j] = row * D + 8 * ((4 * j + (r & 3)) ^ fsw(row));
    }
    return o;
}

// Row-order operand: lane (g, r) gets row 16 rt + r, elements 32 kb + 8 g ..
// +7 (one 16-byte read).
GDN_DEV bf16x8_t nat_frag(const uint16_t *tile, const TileOffs &o, int rt, int kb) {
    return as_bf16x8(*reinterpret_cast<const u32x4_t *>(tile + 16 * rt * D + o.nat[kb]));
}

// A operand of K^T for the state update, k = t in t order and rows in state
// tile order: lane (g, r) gets K[32 kb + {4g..4g+3, 16+4g..16+4g+3}][d], d =
// the state row of tile rt held at row r (two transposing reads: source lane
// m + 4j addresses row 32 kb + 4g + j, columns 8m + .. of the tile's
// 32-block, so output lane 4m + e gets column 32 (rt>>1) + 8m + 4 (rt&1) + e).
GDN_DEV bf16x8_t kt_frag(const uint16_t *tile, const TileOffs &o, int rt, int kb) {
    const uint16_t *p = tile + 32 * kb * D + o.tr[rt >> 1] + 4 * (rt & 1);
    return as_bf16x8(join(lds_tr(p), lds_tr(p + 16 * D)));
}

// Offset of the accumulator tile (rows 4g + e, column 16 cb + r) of column
// block cb of a chunk tile, for acc_tile.
GDN_DEV int acc_off(int cb, int g, int r) {
    const int row = 4 * g + (r >> 2);
    return row * D + 8 * ((2 * cb + ((r >> 1) & 1)) ^ fsw(row)) + 4 * (r & 1);
}
// Accumulator tile (rows 16 rt + 4g + e, column 16 cb + r): one transposing
// read at the offset acc_off(cb).
GDN_DEV f32x4_t acc_tile(const uint16_t *tile, int off, int rt) {
    const u32x2_t w = lds_tr(tile + 16 * rt * D + off);
    f32x4_t x;
    x[0] = __uint_as_float(w[0] << 16);
    x[1] = __uint_as_float(w[0] & 0xFFFF0000u);
    x[2] = __uint_as_float(w[1] << 16);
    x[3] = __uint_as_float(w[1] & 0xFFFF0000u);
    return x;
}

GDN_DEV f32x4_t lds_f4(const float *p) { return *reinterpret_cast<const f32x4_t *>(p); }
GDN_DEV bf16x8_t frag_ld(const u32x4_t &p) { return as_bf16x8(p); }

// ---------------------------------------------------------------------------
// Helper work
// ---------------------------------------------------------------------------

// Gates of chunk c for this lane's token (lane = row of the chunk), both
// zeroed past the sequence end (HF pads the last chunk with zeros): G log2(e)
// and beta go to the helper's own copy hg[hw] (read back by this wave only);
// `write` selects which of the state waves' per-chunk gates the wave also
// stores: bit 0 beta and e^G, bit 1 e^{G_last - G}, scale e^G and e^{G_last}
// (the two helpers that form M each store half).
GDN_DEV void chunk_gates(Smem &sm, int slot, int c, int T, float q_scale, int hw, int lane, int write) {
    // no fused multiply-adds: every inlined copy (prologue, loop, each
    // helper) must round the gates identically
#pragma clang fp contract(off)
    const int valid = min(C, T - c * C);
    const float x = lane < valid ? sm.graw[slot][lane] : 0.f;
    const float bv = lane < valid ? sm.braw[slot][lane] : 0.f;
    const float G = wave_incl_scan(x);
    const float G2 = G * kLog2e;
    sm.hg[hw][0][lane] = G2;
    sm.hg[hw][1][lane] = bv;
    if (write) {
        Gates &gt = sm.gt[slot];
        const float eg = __builtin_amdgcn_exp2f(G2);
        if (write & 1) {
            gt.bt[lane] = bv;
            gt.eg[lane] = eg;
        }
        if (write & 2) {
            const float Gl2 =
                __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, G2), 63));
            gt.egl[lane] = __builtin_amdgcn_exp2f(Gl2 - G2);
            gt.seg[lane] = q_scale * eg;
            if (lane == 0) gt.gam = __builtin_amdgcn_exp2f(Gl2);
        }
    }
    lds_fence();
}

// K K^T tiles of row blocks A0 < A1 (all column blocks b <= a), then
// M_ab = beta_i Gamma_ij (k_i . k_j) for i > j into Mb (fp32 row-major).
template <int A> GDN_DEV void write_m(Smem &sm, const f32x4_t (&acc)[A + 1], const float *G2, const float *Bt,
                                      int g, int r) {
    const f32x4_t Gi = lds_f4(&G2[16 * A + 4 * g]);
    const f32x4_t Bi = lds_f4(&Bt[16 * A + 4 * g]);
#pragma unroll
    for (int b = 0; b <= A; ++b) {
        const float Gj = G2[16 * b + r];
        f32x4_t m;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool lower = (b < A) || (4 * g + e > r);
            const float gm = __builtin_amdgcn_exp2f(lower ? Gi[e] - Gj : 0.f);
            m[e] = lower ? Bi[e] * gm * acc[b][e] : 0.f;
        }
        // column-major: lane (g, r) holds rows 4g .. 4g+3 of column r
        *reinterpret_cast<f32x4_t *>(&sm.Mb[mbi(A, b)][kMbPitch * r + 4 * g]) = m;
    }
}
// K Q^T tiles (b, a) for q row blocks A0 < A1 and b <= a: lane (g, r),
// element e holds k_{t'} . q_t with t' = 16 b + 4 g + e, t = 16 a + r, which
// is the A-fragment slot layout, so each tile is one 8-byte store of
// A[t][t'] = scale Gamma_{t t'} (q_t . k_t'), t' <= t.
template <int A> GDN_DEV void write_a(u32x4_t (&af)[6][64], const f32x4_t (&acc)[A + 1], const float *G2,
                                      float q_scale, int lane, int g, int r) {
    const float Gt = G2[16 * A + r];
#pragma unroll
    for (int b = 0; b <= A; ++b) {
        const f32x4_t Gp = lds_f4(&G2[16 * b + 4 * g]);
        f32x4_t x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool lower = (b < A) || (4 * g + e <= r);
            const float gm = __builtin_amdgcn_exp2f(lower ? Gt - Gp[e] : 0.f);
            x[e] = lower ? q_scale * gm * acc[b][e] : 0.f;
        }
        *reinterpret_cast<u32x2_t *>(reinterpret_cast<char *>(&af[fidx(A, b >> 1)][lane]) + 8 * (b & 1)) =
            bf4u(x);
    }
}
// The Gram tiles of chunk rows A0 < A1 (every column block b <= a): with
// WITH_K, K K^T tiles (a, b) -> M blocks; with WITH_Q, K Q^T tiles (b, a) ->
// A fragments.
template <int A0, int A1, bool WITH_K, bool WITH_Q>
GDN_DEV void gram_rows(Smem &sm, u32x4_t (&af)[6][64], const uint16_t *K, const uint16_t *Q,
                       const float *G2, const float *Bt, float q_scale, int lane, int g, int r) {
    const TileOffs to = tile_offs(g, r);
    f32x4_t kk0[A0 + 1], kk1[A1 + 1], qk0[A0 + 1], qk1[A1 + 1];
#pragma unroll
    for (int b = 0; b <= A0; ++b) kk0[b] = qk0[b] = zero4();
#pragma unroll
    for (int b = 0; b <= A1; ++b) kk1[b] = qk1[b] = zero4();
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        bf16x8_t kf[A1 + 1];
#pragma unroll
        for (int b = 0; b <= A1; ++b) kf[b] = nat_frag(K, to, b, kb);
        if constexpr (WITH_K) {
#pragma unroll
            for (int b = 0; b <= A0; ++b) kk0[b] = mfma_16x16x32_bf16(kf[A0], kf[b], kk0[b]);
#pragma unroll
            for (int b = 0; b <= A1; ++b) kk1[b] = mfma_16x16x32_bf16(kf[A1], kf[b], kk1[b]);
        }
        if constexpr (WITH_Q) {
            const bf16x8_t q0 = nat_frag(Q, to, A0, kb);
            const bf16x8_t q1 = nat_frag(Q, to, A1, kb);
#pragma unroll
            for (int b = 0; b <= A0; ++b) qk0[b] = mfma_16x16x32_bf16(kf[b], q0, qk0[b]);
#pragma unroll
            for (int b = 0; b <= A1; ++b) qk1[b] = mfma_16x16x32_bf16(kf[b], q1, qk1[b]);
        }
    }
    if constexpr (WITH_K) {
        write_m<A0>(sm, kk0, G2, Bt, g, r);
        write_m<A1>(sm, kk1, G2, Bt, g, r);
    }
    if constexpr (WITH_Q) {
        write_a<A0>(af, qk0, G2, q_scale, lane, g, r);
        write_a<A1>(af, qk1, G2, q_scale, lane, g, r);
    }
}

// T = (I + M)^-1 of a chunk whose M is in Mb, as (T - I) fragments in Tf,
// in two steps one phase apart (one helper wave, its values kept in
// registers in between):
//  t_subst: the diagonal blocks by substitution in fp32 on the VALU (the row
//     recurrence of HF, modeling_qwen3_5.py:294-297, on each 16x16 block,
//     solved for the rows of T_aa): lane (a, j) computes row j of T_aa; the
//     rows go to the diagonal fragment halves, and the step keeps them and
//     the accumulator tiles of the off-diagonal M blocks in registers;
//  t_chain: the off-diagonal blocks T_ab = -T_aa sum_{c=b}^{a-1} M_ac T_cb
//     on bf16 MFMA, with T_aa = I + L_aa so that the identity parts stay
//     exact: Y = M_ab + M_ab L_bb + sum_{c>b} M_ac T_cb,  T_ab = -(Y + L_aa Y).
struct TRegs {
    u32x4_t w01, w23;  // bf16 pairs of L = T_aa - I: row j, columns 4q .. 4q+3 (vectors:
                       // kept in registers across the phases)
    f32x4_t MC[6];            // accumulator tiles of M_ab: (1,0) (2,1) (3,2) (2,0) (3,1) (3,0)
};

// Row j of T_aa = (I + M_aa)^-1 in lane (a, j), from T (I + M) = I:
// T[j][i] = delta_ji - sum_{k>i} T[j][k] M[k][i], for i = 15 down to 0,
// right-looking: once x[k] = T[j][k] is final, row k of M updates every
// earlier column.  mcol holds column j of M_aa (mcol[q][e] = M[4q+e][j]);
// M[k][i] is element k of lane (a, i)'s column, broadcast within the 16-lane
// row of block a (DPP row_newbcast).  Each step is one inline-asm block
// with a single hazard wait (gdn_subst_steps.inc); acc starts at -delta so
// that a step's x is one subtraction.
#include "gdn_subst_steps.inc"
GDN_DEV void row_subst(float (&x)[16], const f32x4_t (&mcol)[4], int j) {
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = (i == j) ? -1.f : 0.f;
    subst_step_15(acc, x[15], mcol[3][3]);
    subst_step_14(acc, x[14], mcol[3][2]);
    subst_step_13(acc, x[13], mcol[3][1]);
    subst_step_12(acc, x[12], mcol[3][0]);
    subst_step_11(acc, x[11], mcol[2][3]);
    subst_step_10(acc, x[10], mcol[2][2]);
    subst_step_9(acc, x[9], mcol[2][1]);
    subst_step_8(acc, x[8], mcol[2][0]);
    subst_step_7(acc, x[7], mcol[1][3]);
    subst_step_6(acc, x[6], mcol[1][2]);
    subst_step_5(acc, x[5], mcol[1][1]);
    subst_step_4(acc, x[4], mcol[1][0]);
    subst_step_3(acc, x[3], mcol[0][3]);
    subst_step_2(acc, x[2], mcol[0][2]);
    subst_step_1(acc, x[1], mcol[0][1]);
    x[0] = -acc[0];
}

// The 1-norm of M (largest column sum of |M|) from the values t_subst holds:
// lane (a, j) column j of M_aa, every lane (g, r) rows 4g .. 4g+3 of column
// r of each off-diagonal block.  Sums of |x| propagate NaN; the max keeps it.
GDN_DEV float m_one_norm(const f32x4_t (&mcol)[4], const f32x4_t (&MC)[6]) {
    constexpr int off_b[6] = {0, 1, 2, 0, 1, 0};
    // per lane: column r of each column block b < 3, over the rows it holds
    u32x4_t cb;
    float c[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) c[off_b[i]] += fabsf(MC[i][e]);
#pragma unroll
    for (int b = 0; b < 4; ++b) cb[b] = __builtin_bit_cast(uint32_t, c[b]);
    // afterwards cb[q] row g holds c[g] of row group q: their sum is the
    // off-diagonal part of column 16 g + r
    row_transpose4(cb);
    float col = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) col += __builtin_bit_cast(float, cb[q]);
    // the diagonal block's part: lane (a, j) holds column j of block a,
    // the same column
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) col += fabsf(mcol[q][e]);
    // largest over the wave: rows by DPP, then the four rows' last lanes
    auto mx = [](float x, float y) { return (x > y || x != x) ? x : y; };
    col = mx(col, dpp_src<0x111, 0xF>(col));  // row_shr:1
    col = mx(col, dpp_src<0x112, 0xF>(col));  // row_shr:2
    col = mx(col, dpp_src<0x114, 0xF>(col));  // row_shr:4
    col = mx(col, dpp_src<0x118, 0xF>(col));  // row_shr:8
    const int ci = __builtin_bit_cast(int, col);
    float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(ci, 15));
    m = mx(m, __builtin_bit_cast(float, __builtin_amdgcn_readlane(ci, 31)));
    m = mx(m, __builtin_bit_cast(float, __builtin_amdgcn_readlane(ci, 47)));
    return mx(m, __builtin_bit_cast(float, __builtin_amdgcn_readlane(ci, 63)));
}

GDN_DEV void t_subst(Smem &sm, u32x4_t (&Tf)[6][64], TRegs &tr, float *mnorm, int lane) {
    const int g = lane >> 4, r = lane & 15;
    // one LDS round trip for every input: lane (a, j) reads column j of M_aa,
    // every lane the accumulator tiles of the six off-diagonal blocks
    const int a = lane >> 4, j = lane & 15;
    f32x4_t mcol[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) mcol[q] = lds_f4(&sm.Mb[mbi(a, a)][kMbPitch * j + 4 * q]);
    constexpr int off_a[6] = {1, 2, 3, 2, 3, 3}, off_b[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
    for (int i = 0; i < 6; ++i) tr.MC[i] = lds_f4(&sm.Mb[mbi(off_a[i], off_b[i])][kMbPitch * r + 4 * g]);
    {
        const float mn = m_one_norm(mcol, tr.MC);
        if (lane == 0) *mnorm = mn;
    }
    // lane (a, j) computes row j of T_aa
    {
        float x[16];
        row_subst(x, mcol, j);
        // x[j] is exactly 1 (x[k] = 0 for k > j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            tr.w01[q] = pack2_bf16_hw(4 * q == j ? 0.f : x[4 * q], 4 * q + 1 == j ? 0.f : x[4 * q + 1]);
            tr.w23[q] = pack2_bf16_hw(4 * q + 2 == j ? 0.f : x[4 * q + 2], 4 * q + 3 == j ? 0.f : x[4 * q + 3]);
        }
    }
    // the diagonal fragment halves for the state waves: row j, columns
    // 4q .. 4q+3 of block (a, a) -> fragment fidx(a, a/2), lane 16 q + j,
    // slots 4 (a&1) .. +3
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        u32x2_t w;
        w[0] = tr.w01[q];
        w[1] = tr.w23[q];
        reinterpret_cast<u32x2_t *>(&Tf[fidx(a, a >> 1)][16 * q + j])[a & 1] = w;
    }
}

GDN_DEV void t_chain(u32x4_t (&Tf)[6][64], TRegs &tr, int lane) {
    const int g = lane >> 4, r = lane & 15;
    // identity, accumulator layout (bf16): transposes by one MFMA
    s4_t I4;
    {
        f32x4_t id;
#pragma unroll
        for (int e = 0; e < 4; ++e) id[e] = (4 * g + e == r) ? 1.f : 0.f;
        I4 = bf4(id);
    }
    // L_bb in the 16x16x16 A layout: lane (g, r) holds row r, columns
    // 4g .. 4g+3 of block b, i.e. what lane (b, r) holds in its words for
    // q = g: a transpose of (16-lane row, q).
    row_transpose4(tr.w01);
    row_transpose4(tr.w23);
    // L_bb in the accumulator layout (A layout of L times I) and M_ab in the
    // A layout (accumulator of M_ab read as an A operand is M_ab^T; times I
    // gives M_ab^T in the accumulator layout = M_ab in the A layout).  The
    // transposes are exact: bf16 values times 1.
    s4_t LA[4], LB[3], MA[6];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        u32x2_t w;
        w[0] = tr.w01[b];
        w[1] = tr.w23[b];
        LA[b] = __builtin_bit_cast(s4_t, w);
    }
#pragma unroll
    for (int b = 0; b < 3; ++b) LB[b] = bf4(mfma16(LA[b], I4, zero4()));
#pragma unroll
    for (int i = 0; i < 6; ++i) MA[i] = bf4(mfma16(bf4(tr.MC[i]), I4, zero4()));
    const f32x4_t (&MC)[6] = tr.MC;
    auto fin = [&](int a2, const f32x4_t &y) { return -mfma16(LA[a2], bf4(y), y); };
    f32x4_t y;
    y = mfma16(MA[0], LB[0], MC[0]);
    const f32x4_t T10 = fin(1, y);
    y = mfma16(MA[1], LB[1], MC[1]);
    const f32x4_t T21 = fin(2, y);
    y = mfma16(MA[2], LB[2], MC[2]);
    const f32x4_t T32 = fin(3, y);
    y = mfma16(MA[3], LB[0], MC[3]);
    y = mfma16(MA[1], bf4(T10), y);
    const f32x4_t T20 = fin(2, y);
    y = mfma16(MA[4], LB[1], MC[4]);
    y = mfma16(MA[2], bf4(T21), y);
    const f32x4_t T31 = fin(3, y);
    y = mfma16(MA[5], LB[0], MC[5]);
    y = mfma16(MA[4], bf4(T10), y);
    y = mfma16(MA[2], bf4(T20), y);
    const f32x4_t T30 = fin(3, y);
    // block (a2, b) into its fragment half (A layout, by the same transpose):
    // one 8-byte store
    auto put = [&](int a2, int b, const f32x4_t &x) {
        const f32x4_t xa = mfma16(bf4(x), I4, zero4());
        reinterpret_cast<u32x2_t *>(&Tf[fidx(a2, b >> 1)][lane])[b & 1] = bf4u(xa);
    };
    put(1, 0, T10);
    put(2, 0, T20);
    put(2, 1, T21);
    put(3, 0, T30);
    put(3, 1, T31);
    put(3, 2, T32);
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
// Segment loops
// ---------------------------------------------------------------------------

struct SegArgs {
    const uint16_t *q, *k, *v;
    const float *g, *beta;
    uint16_t *o;
    void *S;          // initial state in, final state out
    float *carry;
    int T, Hv, Hk, NC, P;
    int bnd[kMaxSegs + 1];  // segment p covers chunks [bnd[p], bnd[p+1])
    float q_scale;
    // Windowed segments (0 when the call has none): segment p outputs chunks
    // [wbnd[p], wbnd[p+1]) and starts its recurrence at the chunk its head's
    // window word names.
    int Pw;
    int wbnd[kMaxSegs + 1];
    int Wmax;  // longest window checked, in chunks (kWinMin .. kWinCap)
};

// Ring slots of chunk n in a segment starting at n0.
GDN_DEV int kslot(int n, int n0) { return (n - n0) % 3; }
GDN_DEV int pslot(int n, int n0) { return (n - n0) & 1; }

// Zero the two upper blocks of the fragment layouts (constant).
GDN_DEV void zero_upper_halves(Smem &sm, int tid) {
    if (tid < 64 * 8) {
        const int which = tid >> 6, lane = tid & 63;
        u32x4_t(*f)[64] = which < 4 ? sm.Tf[which >> 1] : sm.Af[(which - 4) >> 1];
        const int frag = (which & 1) ? fidx(2, 1) : fidx(0, 0);
        reinterpret_cast<u32x2_t *>(&f[frag][lane])[1] = u32x2_t{0u, 0u};
    }
}

// A transition chunk for column tiles c0 .. c0 + 16 NCT - 1 of the
// 256-column state [C | Phi] (C from 0 driven by V, Phi from I with V = 0),
// no output.  Phase 1: P = K X.
template <int NCT>
GDN_DEV void trans_phase1(Smem &sm, const f32x4_t (&X)[8][NCT], f32x4_t (&P)[4][NCT], int n, int n0, int lane) {
    TileOffs to;
    {
        const int ln = opaque_lane(lane);
        to = tile_offs(ln >> 4, ln & 15);
    }
    const uint16_t *K = sm.Kb[kslot(n, n0)];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) P[i][ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        bf16x8_t xf[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) xf[ct] = frag_acc(X[2 * kb][ct], X[2 * kb + 1][ct]);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const bf16x8_t kf = nat_frag(K, to, rt, kb);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) P[rt][ct] = mfma_16x16x32_bf16(kf, xf[ct], P[rt][ct]);
        }
        // one k-block of bf16 state fragments live at a time (registers)
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Phase 2: R = beta (V - e^G P), v = R + (T - I) R, and the state update.
template <int NCT>
GDN_DEV void trans_phase2(Smem &sm, f32x4_t (&X)[8][NCT], f32x4_t (&P)[4][NCT], int n, int n0, int c0, bool is_phi,
                          int lane) {
    const int g = lane >> 4;
    TileOffs to;
    {
        const int ln = opaque_lane(lane);
        to = tile_offs(ln >> 4, ln & 15);
    }
    const uint16_t *K = sm.Kb[kslot(n, n0)];
    const uint16_t *V = sm.Vb[pslot(n, n0)];
    const Gates &gt = sm.gt[pslot(n, n0)];
    // R = beta (V - e^G P)  (Phi columns: V = 0)
    if (is_phi) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const f32x4_t bt = lds_f4(&gt.bt[16 * rt + 4 * g]);
            const f32x4_t eg = lds_f4(&gt.eg[16 * rt + 4 * g]);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                for (int e = 0; e < 4; ++e) P[rt][ct][e] = -bt[e] * eg[e] * P[rt][ct][e];
        }
    } else {
        int voff[NCT];
        {
            const int ln = opaque_lane(lane);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) voff[ct] = acc_off(c0 / 16 + ct, ln >> 4, ln & 15);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const f32x4_t bt = lds_f4(&gt.bt[16 * rt + 4 * g]);
            const f32x4_t eg = lds_f4(&gt.eg[16 * rt + 4 * g]);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const f32x4_t vv = acc_tile(V, voff[ct], rt);
#pragma unroll
                for (int e = 0; e < 4; ++e) P[rt][ct][e] = bt[e] * (vv[e] - eg[e] * P[rt][ct][e]);
            }
        }
    }
    // v = R + (T - I) R (R as a hi + lo pair), one column tile at a time
    // (registers)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        bf16x8_t rh[2], rl[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) frag_acc_split(P[2 * kb][ct], P[2 * kb + 1][ct], rh[kb], rl[kb]);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int kb = 0; kb <= (rt >> 1); ++kb) {
                const bf16x8_t tf = frag_ld(sm.Tf[pslot(n, n0)][fidx(rt, kb)][lane]);
                P[rt][ct] = mfma_16x16x32_bf16(tf, rh[kb], P[rt][ct]);
                P[rt][ct] = mfma_16x16x32_bf16(tf, rl[kb], P[rt][ct]);
            }
    }
    {
        const float gam = gt.gam;
#pragma unroll
        for (int rt = 0; rt < 8; ++rt)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                for (int e = 0; e < 4; ++e) X[rt][ct][e] *= gam;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const f32x4_t slo = lds_f4(&gt.egl[32 * kb + 4 * g]);
            const f32x4_t shi = lds_f4(&gt.egl[32 * kb + 16 + 4 * g]);
            bf16x8_t vg[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) vg[ct] = frag_acc_scaled(P[2 * kb][ct], P[2 * kb + 1][ct], slo, shi);
#pragma unroll
            for (int rt = 0; rt < 8; ++rt) {
                const bf16x8_t kt = kt_frag(K, to, rt, kb);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) X[rt][ct] = mfma_16x16x32_bf16(kt, vg[ct], X[rt][ct]);
            }
        }
    }
}

// The state's columns in a transition segment: the state waves 0 .. 3 hold
// 48 columns each (waves 0, 1: C columns 0 .. 95; waves 2, 3: Phi columns
// 0 .. 95), helpers 1 and 2 the last 32 columns of C and of Phi, in the
// phases where their helper work leaves room (no q in such a segment).
constexpr int kTransCols = 48;
constexpr int kTransHelperCols = D - 2 * kTransCols;

// Initial transition state for column tiles from c0: 0 (C) or I (Phi).
template <int NCT>
GDN_DEV void trans_init(f32x4_t (&X)[8][NCT], int c0, bool is_phi, int g, int r) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) X[rt][ct][e] = (is_phi && srow(rt, g, e) == c0 + 16 * ct + r) ? 1.f : 0.f;
}

// State waves of a transition segment.
template <int NCT>
GDN_DEV void state_loop_trans(Smem &sm, f32x4_t (&X)[8][NCT], int n0, int n1, int c0, bool is_phi, int lane) {
    lds_barrier();
    lds_barrier();
    lds_barrier();
    for (int n = n0; n < n1; ++n) {
        f32x4_t P[4][NCT];
        trans_phase1<NCT>(sm, X, P, n, n0, lane);
        lds_barrier();  // X
        trans_phase2<NCT>(sm, X, P, n, n0, c0, is_phi, lane);
        lds_barrier();  // Y
    }
}

// Helper waves (hw = wave - 4) of a segment over chunks [n0, n1).  WITH_Q:
// output segment (q rows, K Q^T and the A fragments).  The barrier sequence
// matches the state loops'.  In iteration n (the state waves on chunk n):
//   phase 1: hw0 finishes T of chunk n (t_chain); hw1, hw2 form M of chunk
//            n+1 (K K^T rows {0, 3} and {1, 2}, gates: hw1 stores them for
//            the state waves); hw3 issues the loads of the k rows and gates
//            of chunk n+2 and the v rows of chunk n+1;
//   phase 2: hw0 starts T of chunk n+1 (t_subst); hw3 and hw1 form the A
//            fragments of chunk n+1 (rows {0, 3} and {1, 2}), and hw3 waits
//            for its loads; hw2 issues the loads of the q rows of chunk n+2,
//            which it waits for at the end of the next phase 1.
// In a transition segment (no q) hw3 loads chunk n+1's v rows in phase 2
// instead of in phase 1, and waits for them before the phase ends.
// Every load thus has at least a whole phase to land.
// SNCT > 0 (a transition segment): helpers 1 and 2, which issue no loads
// there, also run SNCT column tiles of the state from column c0 (C for
// helper 1, Phi for helper 2).
template <bool WITH_Q, int SNCT = 0>
GDN_DEV void helper_loop(Smem &sm, const SegArgs &a, int b, int h, int n0, int n1, int hw, int lane,
                         f32x4_t (&X)[8][SNCT > 0 ? SNCT : 1], int c0 = 0) {
    // with SNCT > 0 only helpers 1 and 2 run this instance: helper 0's role
    // and helper 2's loads are dead code in it, so that their registers (T's
    // rows kept across the phases) and the state's are never live together
    const bool with_state = SNCT > 0;
    const bool h0 = SNCT == 0 && hw == 0, h2 = SNCT == 0 && hw == 2;
    const int g = lane >> 4, r = lane & 15;
    const int kh = h / (a.Hv / a.Hk);
    const int NC = a.NC;
    TRegs tr;
    auto kk = [&](int c, bool rows03) {
        const int ps = pslot(c, n0);
        chunk_gates(sm, ps, c, a.T, a.q_scale, hw, lane, rows03 ? 1 : 2);
        const float *G2 = sm.hg[hw][0], *Bt = sm.hg[hw][1];
        const uint16_t *K = sm.Kb[kslot(c, n0)];
        if (rows03) gram_rows<0, 3, true, false>(sm, sm.Af[ps], K, K, G2, Bt, a.q_scale, lane, g, r);
        else gram_rows<1, 2, true, false>(sm, sm.Af[ps], K, K, G2, Bt, a.q_scale, lane, g, r);
    };
    auto qk = [&](int c, bool rows03) {
        const int ps = pslot(c, n0);
        chunk_gates(sm, ps, c, a.T, a.q_scale, hw, lane, 0);
        const float *G2 = sm.hg[hw][0], *Bt = sm.hg[hw][1];
        const uint16_t *K = sm.Kb[kslot(c, n0)];
        const uint16_t *Q = sm.Qb[ps];
        if (rows03) gram_rows<0, 3, false, true>(sm, sm.Af[ps], K, Q, G2, Bt, a.q_scale, lane, g, r);
        else gram_rows<1, 2, false, true>(sm, sm.Af[ps], K, Q, G2, Bt, a.q_scale, lane, g, r);
    };
    // prologue: chunk n0 (all tiles) and n0+1 (k, q, gates), a quarter of
    // the rows per helper
    {
        const int c1 = min(n0 + 1, NC - 1);
        load_rows_n<4>(sm.Kb[0], a.k, a.Hk, kh, b, n0, a.T, 16 * hw, lane);
        load_rows_n<4>(sm.Vb[0], a.v, a.Hv, h, b, n0, a.T, 16 * hw, lane);
        load_gates(sm, 0, a.g, a.beta, b, h, a.Hv, n0, a.T, hw, lane);
        load_rows_n<4>(sm.Kb[1], a.k, a.Hk, kh, b, c1, a.T, 16 * hw, lane);
        load_gates(sm, 1, a.g, a.beta, b, h, a.Hv, c1, a.T, hw, lane);
        if (WITH_Q) {
            load_rows_n<4>(sm.Qb[0], a.q, a.Hk, kh, b, n0, a.T, 16 * hw, lane);
            load_rows_n<4>(sm.Qb[1], a.q, a.Hk, kh, b, c1, a.T, 16 * hw, lane);
        }
        wait_vmem0();
    }
    lds_barrier();
    if (hw == 1) kk(n0, true);
    else if (hw == 2) kk(n0, false);
    else if (WITH_Q && hw == 3) qk(n0, true);
    else if (WITH_Q && h0) qk(n0, false);
    lds_barrier();
    if (h0) t_subst(sm, sm.Tf[pslot(n0, n0)], tr, &sm.gt[pslot(n0, n0)].mnorm, lane);
    lds_barrier();
    for (int n = n0; n < n1; ++n) {
        const bool more = n + 1 < n1;
        const int c2 = min(n + 2, NC - 1), c1 = min(n + 1, NC - 1);
        if (h0) {
            __builtin_amdgcn_s_setprio(3);
            t_chain(sm.Tf[pslot(n, n0)], tr, lane);
            __builtin_amdgcn_s_setprio(0);
        } else if (hw == 3) {
            // into slots whose last readers finished in the previous chunk
            load_rows_n<16>(sm.Kb[kslot(n + 2, n0)], a.k, a.Hk, kh, b, c2, a.T, 0, lane);
            load_gates_all(sm, pslot(n + 2, n0), a.g, b, h, a.Hv, c2, a.T, 0, lane);
            load_gates_all(sm, pslot(n + 2, n0), a.beta, b, h, a.Hv, c2, a.T, 1, lane);
            if (WITH_Q) load_rows_n<16>(sm.Vb[pslot(n + 1, n0)], a.v, a.Hv, h, b, c1, a.T, 0, lane);
        } else if (more) {
            __builtin_amdgcn_s_setprio(2);
            kk(n + 1, hw == 1);
            __builtin_amdgcn_s_setprio(0);
        }
        [[maybe_unused]] f32x4_t P[4][SNCT > 0 ? SNCT : 1];
        if constexpr (SNCT > 0)
            if (with_state) trans_phase1<SNCT>(sm, X, P, n, n0, lane);
        if (h2) wait_vmem0();  // q rows of chunk n+1
        lds_barrier();              // X
        if (h0) {
            if (more) t_subst(sm, sm.Tf[pslot(n + 1, n0)], tr, &sm.gt[pslot(n + 1, n0)].mnorm, lane);
        } else if (WITH_Q && h2) {
            // into the slot chunk n's q leaves (read in phase 1 only)
            load_rows_n<16>(sm.Qb[pslot(n + 2, n0)], a.q, a.Hk, kh, b, c2, a.T, 0, lane);
        } else {
            // transition segments: the v rows of chunk n+1 (whose slot chunk
            // n-1 left), here rather than with the phase-1 loads, which bound
            // that phase; phase 2 outlasts them.  Only helper 3 issues loads
            // there: a wave that reads LDS after its own DMA waits for that
            // DMA first
            if (!WITH_Q && hw == 3) load_rows_n<16>(sm.Vb[pslot(n + 1, n0)], a.v, a.Hv, h, b, c1, a.T, 0, lane);
            if (WITH_Q && more) qk(n + 1, hw == 3);
            if constexpr (SNCT > 0)
                if (with_state) trans_phase2<SNCT>(sm, X, P, n, n0, c0, hw == 2, lane);
            if (hw == 3) wait_vmem0();  // k rows, gates of chunk n+2, v rows of n+1
        }
        lds_barrier();  // Y
    }
    wait_vmem0();
}

// State waves of an output segment: columns c0 .. c0 + 31 (two tiles).
// o^T tiles: lane (g, r) of tile (ct, tt) holds o[t = 16 tt + r][c0 + 16 ct
// + 4g .. +3].  Chunks before n_out (a windowed segment's warm-up) update
// the state only: no o products, no stores.
GDN_DEV void state_loop_out(Smem &sm, f32x4_t (&S)[8][2], const SegArgs &a, int b, int h, int n0,
                            int n1, int n_out, int c0, int lane) {
    const int g = lane >> 4, r = lane & 15;
    const TileOffs to = tile_offs(g, r);
    const int voff[2] = {acc_off(c0 / 16, g, r), acc_off(c0 / 16 + 1, g, r)};
    lds_barrier();  // prologue loads landed
    lds_barrier();  // chunk n0's gates and M written
    lds_barrier();  // chunk n0's T and A fragments written
    for (int n = n0; n < n1; ++n) {
        const uint16_t *K = sm.Kb[kslot(n, n0)];
        const uint16_t *Q = sm.Qb[pslot(n, n0)];
        const uint16_t *V = sm.Vb[pslot(n, n0)];
        const Gates &gt = sm.gt[pslot(n, n0)];
        // phase 1: P = K S, O^T = S^T Q^T
        f32x4_t P[4][2], O[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                P[i][ct] = zero4();
                O[ct][i] = zero4();
            }
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t sf[2];
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) sf[ct] = frag_acc(S[2 * kb][ct], S[2 * kb + 1][ct]);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const bf16x8_t kf = nat_frag(K, to, rt, kb);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) P[rt][ct] = mfma_16x16x32_bf16(kf, sf[ct], P[rt][ct]);
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const bf16x8_t qf = nat_frag(Q, to, tt, kb);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) O[ct][tt] = mfma_16x16x32_bf16(sf[ct], qf, O[ct][tt]);
            }
        }
        lds_barrier();  // X: T of chunk n is ready
        // this phase bounds the chunk: its waves issue ahead of the helpers'
        __builtin_amdgcn_s_setprio(2);
        // R = beta (V - e^G P)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
            const f32x4_t bt = lds_f4(&gt.bt[16 * rt + 4 * g]);
            const f32x4_t eg = lds_f4(&gt.eg[16 * rt + 4 * g]);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const f32x4_t vv = acc_tile(V, voff[ct], rt);
#pragma unroll
                for (int e = 0; e < 4; ++e) P[rt][ct][e] = bt[e] * (vv[e] - eg[e] * P[rt][ct][e]);
            }
        }
        // v = R + (T - I) R.  Consecutive rows of R can nearly cancel in T R
        // (repeated keys), so R goes in as a hi + lo pair of bf16 fragments,
        // unless the chunk's M has 1-norm s < 1/2: then |T - I|_1 <= s/(1-s)
        // and |R|_1 <= (1+s)|v|_1 bound the error of one bf16 rounding of R
        // by 1.5 bf16 roundings of v, which the products below apply to v
        // anyway.
        {
            const float mn = __builtin_bit_cast(
                float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, gt.mnorm)));
            if (mn < 0.5f) {
                bf16x8_t rh[2][2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) rh[kb][ct] = frag_acc(P[2 * kb][ct], P[2 * kb + 1][ct]);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                    for (int kb = 0; kb <= (rt >> 1); ++kb) {
                        const bf16x8_t tf = frag_ld(sm.Tf[pslot(n, n0)][fidx(rt, kb)][lane]);
#pragma unroll
                        for (int ct = 0; ct < 2; ++ct) P[rt][ct] = mfma_16x16x32_bf16(tf, rh[kb][ct], P[rt][ct]);
                    }
            } else {
                bf16x8_t rh[2][2], rl[2][2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        frag_acc_split(P[2 * kb][ct], P[2 * kb + 1][ct], rh[kb][ct], rl[kb][ct]);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                    for (int kb = 0; kb <= (rt >> 1); ++kb) {
                        const bf16x8_t tf = frag_ld(sm.Tf[pslot(n, n0)][fidx(rt, kb)][lane]);
#pragma unroll
                        for (int ct = 0; ct < 2; ++ct) {
                            P[rt][ct] = mfma_16x16x32_bf16(tf, rh[kb][ct], P[rt][ct]);
                            P[rt][ct] = mfma_16x16x32_bf16(tf, rl[kb][ct], P[rt][ct]);
                        }
                    }
            }
        }
        // o^T = scale e^G O^T + v^T A^T (a warm-up chunk stores no outputs)
        if (n >= n_out) {
            const int ps = pslot(n, n0);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const float s = gt.seg[16 * tt + r];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int e = 0; e < 4; ++e) O[ct][tt][e] *= s;
            }
            bf16x8_t vf[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) vf[kb][ct] = frag_acc(P[2 * kb][ct], P[2 * kb + 1][ct]);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                for (int kb = 0; kb <= (tt >> 1); ++kb) {
                    const bf16x8_t af = frag_ld(sm.Af[ps][fidx(tt, kb)][lane]);
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) O[ct][tt] = mfma_16x16x32_bf16(vf[kb][ct], af, O[ct][tt]);
                }
            // one 16-byte store per row tile: a swap between neighbouring
            // 16-lane rows gives lane (g, r) the eight consecutive columns
            // 16 (g & 1) + 8 (g >> 1) .. +7 (rows 0, 2 of tile 0 keep theirs
            // and take rows 0, 2 of tile 1's; rows 1, 3 the reverse)
            const int valid = min(C, a.T - n * C);
            uint16_t *ob = a.o + (((size_t)b * a.T + (size_t)n * C) * a.Hv + h) * D + c0 + 16 * (g & 1) +
                           8 * (g >> 1);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const u32x2_t w0 = bf4u(O[0][tt]), w1 = bf4u(O[1][tt]);
                const auto s0 = __builtin_amdgcn_permlane16_swap(w0[0], w1[0], false, false);
                const auto s1 = __builtin_amdgcn_permlane16_swap(w0[1], w1[1], false, false);
                u32x4_t w;
                w[0] = s0[0];
                w[1] = s1[0];
                w[2] = s0[1];
                w[3] = s1[1];
                const int t = 16 * tt + r;
                if (t < valid) *reinterpret_cast<u32x4_t *>(ob + (size_t)t * a.Hv * D) = w;
            }
        }
        // S = e^{G_last} S + K^T diag(e^{G_last - G}) v
        {
            const float gam = gt.gam;
#pragma unroll
            for (int rt = 0; rt < 8; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int e = 0; e < 4; ++e) S[rt][ct][e] *= gam;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const f32x4_t slo = lds_f4(&gt.egl[32 * kb + 4 * g]);
                const f32x4_t shi = lds_f4(&gt.egl[32 * kb + 16 + 4 * g]);
                bf16x8_t vg[2];
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) vg[ct] = frag_acc_scaled(P[2 * kb][ct], P[2 * kb + 1][ct], slo, shi);
#pragma unroll
                for (int rt = 0; rt < 8; ++rt) {
                    const bf16x8_t kt = kt_frag(K, to, rt, kb);
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) S[rt][ct] = mfma_16x16x32_bf16(kt, vg[ct], S[rt][ct]);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();  // Y
    }
}

// Start state of segment p >= 1 of pass 2, composed by the workgroup itself:
// S_start(1) = the end state of segment 0 (in the carry); for q = 1 .. p-1,
// S_start(q+1) = Phi_q S_start(q) + C_q.  Phi_{q+1} streams from the carry
// into an fp32 LDS buffer by direct loads (and C_{q+1} into registers) while
// step q computes; at the start of a step the threads split the staged Phi
// into bf16 hi and lo halves, so every wave reads MFMA-ready A fragments; the
// product is hi*hi + hi*lo + lo*hi (near-fp32 accuracy).  Wave w keeps
// columns 16w .. 16w+15.  The halves are unpadded [128][128] tiles with the
// 16-byte piece c of row i in slot c ^ csw(i): the sixteen rows of one state
// tile land in sixteen different slots.
struct CombSmem {
    float raw[D * D];       // Phi as loaded, row-major fp32
    uint16_t hi[D * D];
    uint16_t lo[D * D];
};
GDN_DEV int csw(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
GDN_DEV int cidx(int row, int col) { return row * D + ((((col >> 3) ^ csw(row)) << 3) | (col & 7)); }

// Direct loads of one 64 KiB Phi: wave w moves kilobytes 8w .. 8w+7.
GDN_DEV void comb_fetch(CombSmem &sm, const float *phi, int tid) {
    const int lane = tid & 63, wave = wave_id();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int blk = 8 * wave + j;  // 1 KiB = 256 floats
        __builtin_amdgcn_global_load_lds(phi + blk * 256 + 4 * lane, (lds_void_t *)&sm.raw[blk * 256],
                                         16, 0, 0);
    }
}

GDN_DEV void combine_prefix(CombSmem &sm, f32x4_t (&S)[8][1], const float *carry, int b, int h,
                            int Hv, int P, int p, int tid) {
    const int lane = tid & 63, wave = wave_id();
    const int g = lane >> 4, r = lane & 15;
    const int c0 = 16 * wave;
    tiles_load<kF32, 1>(S, carry_slot(carry, b, h, Hv, P, 1, kSst), c0, g, r);
    if (p < 2) return;
    f32x4_t cn[8][1];
    tiles_load<kF32, 1>(cn, carry_slot(carry, b, h, Hv, P, 1, kCst), c0, g, r);
    comb_fetch(sm, carry_slot(carry, b, h, Hv, P, 1, kPhi), tid);
    wait_vmem0();
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
        wait_vmem0();   // the next Phi has landed
        lds_barrier();  // and every wave is done with the halves
    }
}

// Value head of workgroup column x.  Workgroups go to the 8 XCDs round-robin
// by linear id, and gridDim.x = Hv, so x % 8 names the XCD: heads are laid
// out so that each XCD holds Hv/8 consecutive heads, which keeps the value
// heads of one key head (and their shared k and q rows) in one L2.
GDN_DEV int head_of(int x, int Hv) { return (Hv % 8 == 0) ? (Hv / 8) * (x % 8) + x / 8 : x; }

// Output segment over chunks [n0, n1) from S (state waves' registers),
// outputs stored from chunk n_out on.
GDN_DEV void run_output(Smem &sm, f32x4_t (&S)[8][2], const SegArgs &a, int b, int h, int n0, int n1,
                        int n_out) {
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    zero_upper_halves(sm, tid);
    if (wave < NSW) state_loop_out(sm, S, a, b, h, n0, n1, n_out, 32 * wave, lane);
    else {
        f32x4_t none[8][1];
        helper_loop<true>(sm, a, b, h, n0, n1, wave - NSW, lane, none);
    }
}

// ---------------------------------------------------------------------------
// Windowed segments
// ---------------------------------------------------------------------------
//
// One token maps the state as S -> A_t S + beta_t k_t v_t^T with
// A_t = gamma_t (I - beta_t k_t k_t^T), gamma_t = e^{g_t}; I - b k k^T has the
// eigenvalues 1 and 1 - b |k|^2, so ||A_t||_2 = gamma_t max(1, |1 - beta_t
// |k_t|^2|).  Over a window of chunks the state that entered it is carried
// by a map of norm at most the product of these.  When that product is at
// most 2^-24 (one fp32 rounding of the state it multiplies), a segment can
// start its recurrence from S = 0 at the window's first chunk instead of
// from the true state: what it drops is below that state's own fp32
// resolution.  A head whose every segment boundary has such a window of at
// most Wmax chunks (checked on the device for each call) runs its
// segments independently in one pass: segment p runs chunks [start_p,
// wbnd[p+1]) and stores the outputs of [wbnd[p], wbnd[p+1]).  Other heads run
// the two-pass algorithm, which is exact for any gates.
//
// Per (sequence, head), slot 0 of the carry (which the two-pass path does not
// use) holds the window words in its Phi area (word p >= 1: start_p, or -1
// when boundary p has no window; the head runs windowed when none is -1)
// and, in its S area, the final state as fp32: the last segment writes it
// there and pass 2 moves it to the caller's state, so that no segment that
// reads the initial state races the one that ends the sequence.
// Wmax: the planned segment length, at least kWinMin and at most kWinCap
// chunks.  A window as long as the segment doubles that segment's chunk
// steps, about what the two-pass path costs.
constexpr int kWinMin = 4, kWinCap = 32;
constexpr int kCheckWaves = 16;
constexpr float kWinLog2Bound = -24.f;

GDN_DEV int *win_words(float *carry, int b, int h, int Hv, int P) {
    return reinterpret_cast<int *>(carry_slot(carry, b, h, Hv, P, 0, kPhi));
}

// One workgroup per (head, boundary p >= 1, sequence): the bound's log2 over
// up to Wmax chunks before wbnd[p] (chunk j: wbnd[p] - 1 - j), then the
// shortest window that meets the bound: word p = its first chunk, or -1 when
// none does.  A window that reaches chunk 0 starts from the initial state
// and is exact.  The key factors are at least 1 (log2 >= 0), so no window
// shorter than the first whose gates alone meet the bound can meet it: the
// k rows (16 coalesced 1 KiB row groups per chunk; a row's |k|^2 sums over
// its 16 lanes) are read only for that window's chunks, and for the longer
// windows only when it fails.  A head whose gates never reach the bound
// reads no k rows.  The windows' sums are prefix sums over the chunks (one
// wave, lane j = chunk j), and the shortest window is the first lane whose
// sum meets the bound; the gates' and the key factors' sums take the same
// order, so a chunk whose key factors are all 1 sums exactly as its gates.
__global__ __launch_bounds__(64 * kCheckWaves) void prefill_window_check_kernel(SegArgs a) {
    const int h = blockIdx.x, p = blockIdx.y + 1, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kh = h / (a.Hv / a.Hk);
    const int W = a.Wmax;
    __shared__ float gsum[kWinCap], lam[kWinCap];
    __shared__ float kkrow[kCheckWaves][C];  // |k_t|^2 of the chunk a wave is on
    __shared__ int win[2];                   // L1, then the window's start (or -2: read more)
    auto chunk_of = [&](int j) { return a.wbnd[p] - 1 - j; };
    auto gate_at = [&](const float *x, int c) {
        return x[((size_t)b * a.T + min(c * C + lane, a.T - 1)) * a.Hv + h];
    };
    // the first lane j < n whose prefix sum of v meets the bound or whose
    // chunk is before chunk 0, as j + 1 (0: none); wave 0, every lane
    auto first_window = [&](const float *v, int n) {
        const bool in = lane < n;
        const float x = in && chunk_of(lane) >= 0 ? v[lane] : 0.f;
        const float pre = wave_incl_scan(x);
        const bool hit = in && (chunk_of(lane) < 0 || pre <= kWinLog2Bound);  // false for NaN
        const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
        return m ? (int)__builtin_ctzll(m) + 1 : 0;
    };
    // gsum[j] for chunks j in [j0, j1): log2 of the gates alone, chunk
    // j0 + wave + 16 i to this wave, its loads issued together
    auto gate_sums = [&](int j0, int j1) {
        constexpr int kPer = kWinCap / kCheckWaves;
        float x[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = j0 + wave + kCheckWaves * i, c = chunk_of(j);
            x[i] = j < j1 && c >= 0 && c * C + lane < a.T ? gate_at(a.g, c) * kLog2e : 0.f;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int j = j0 + wave + kCheckWaves * i;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) x[i] += __shfl_xor(x[i], off);
            if (lane == 0 && j < j1) gsum[j] = x[i];
        }
    };
    // the gates in two rounds: the nearest four chunks, then the rest only
    // when those do not meet the bound (a lane's gate shares its L2 line
    // with the other heads', so each chunk costs 64 lines)
    const int W1 = min(4, W);
    gate_sums(0, W1);
    __syncthreads();
    if (wave == 0) {
        const int L = first_window(gsum, W1);
        if (lane == 0) win[0] = L;
    }
    __syncthreads();
    if (win[0] == 0 && W1 < W) {
        gate_sums(W1, W);
        __syncthreads();
        if (wave == 0) {
            const int L = first_window(gsum, W);
            if (lane == 0) win[0] = L;
        }
        __syncthreads();
    }
    const int L1 = win[0];
    // lam[j] = log2 of the bound over chunk j
    auto chunk_bound = [&](int j) {
        const int c = chunk_of(j);
        const int sub = lane >> 4, piece = lane & 15;
        u32x4_t w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = min(c * C + 4 * i + sub, a.T - 1);
            w[i] = *reinterpret_cast<const u32x4_t *>(a.k + (((size_t)b * a.T + t) * a.Hk + kh) * D + 8 * piece);
        }
        const float gv = gate_at(a.g, c), bv = gate_at(a.beta, c);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float kk = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = __uint_as_float(w[i][e] << 16), hi = __uint_as_float(w[i][e] & 0xFFFF0000u);
                kk += lo * lo + hi * hi;
            }
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) kk += __shfl_xor(kk, off);
            if (piece == 0) kkrow[wave][4 * i + sub] = kk;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float x = 0.f;
        if (c * C + lane < a.T) x = gv * kLog2e + __log2f(fmaxf(1.f, fabsf(1.f - bv * kkrow[wave][lane])));
        __builtin_amdgcn_wave_barrier();  // every lane has read kkrow before the next chunk writes it
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
        if (lane == 0) lam[j] = x;
    };
    // the window's first chunk (0 when it reaches the start), -1 for none
    auto start_of = [&](int L) { return L == 0 ? -1 : max(chunk_of(L - 1), 0); };
    if (L1 > 0) {
        for (int j = wave; j < L1 && chunk_of(j) >= 0; j += kCheckWaves) chunk_bound(j);
        __syncthreads();
        if (wave == 0) {
            const int L = first_window(lam, L1);
            if (lane == 0) win[1] = L > 0 ? start_of(L) : (L1 < W ? -2 : -1);
        }
        __syncthreads();
        if (win[1] == -2) {  // the first window failed on its key factors: the longer ones
            for (int j = L1 + wave; j < W && chunk_of(j) >= 0; j += kCheckWaves) chunk_bound(j);
            __syncthreads();
            if (wave == 0) {
                const int L = first_window(lam, W);
                if (lane == 0) win[1] = start_of(L);
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        int start = L1 > 0 ? win[1] : -1;
        if (start < 0 && a.wbnd[p] <= W) start = 0;
        win_words(a.carry, b, h, a.Hv, a.P)[p] = start;
    }
}

// Segment p of a windowed head.
template <int IN_FMT>
GDN_DEV void run_window(Smem &sm, const SegArgs &a, int b, int h, int p, const int *w) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int g = lane >> 4, r = lane & 15;
    const int n_out = a.wbnd[p], n1 = a.wbnd[p + 1];
    const int n0 = p == 0 ? 0 : __builtin_amdgcn_readfirstlane(w[p]);
    f32x4_t S[8][2];
    if (wave < NSW) {
        if (n0 == 0) {
            const void *Sg = static_cast<const char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (IN_FMT == kF16 ? 2 : 4);
            tiles_load<IN_FMT, 2>(S, Sg, 32 * wave, g, r);
        } else {
#pragma unroll
            for (int rt = 0; rt < 8; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) S[rt][ct] = zero4();
        }
    }
    run_output(sm, S, a, b, h, n0, n1, n_out);
    if (wave < NSW && p == a.Pw - 1)  // pass 2 moves it to the caller's state
        tiles_store<kF32, 2>(S, carry_slot(a.carry, b, h, a.Hv, a.P, 0, kSst), 32 * wave, g, r);
}

// True when head h of sequence b runs windowed in this call: every
// boundary has a window (words 1 .. Pw-1 >= 0), read by one lane each.
GDN_DEV bool head_windowed(const SegArgs &a, int b, int h) {
    if (a.Pw == 0) return false;
    const int lane = threadIdx.x & 63;
    const int *w = win_words(a.carry, b, h, a.Hv, a.P);
    const int x = lane + 1 < a.Pw ? w[lane + 1] : 0;
    return __builtin_amdgcn_ballot_w64(x < 0) == 0;
}

// Pass 1: slot p = blockIdx.y < P-1.  Segment 0 runs the output recurrence
// from the initial state; segments 1 .. P-2 their transition.  A windowed
// head's workgroups instead run its segments p < Pw (the grid covers the
// longer of the two plans).
template <int IN_FMT, int OUT_FMT>
__global__ __launch_bounds__(NT) void prefill_pass1_kernel(SegArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
    const int h = head_of(blockIdx.x, a.Hv), p = blockIdx.y, b = blockIdx.z;
    if (a.Pw > 0) {
        if (head_windowed(a, b, h)) {
            if (p < a.Pw) run_window<IN_FMT>(sm, a, b, h, p, win_words(a.carry, b, h, a.Hv, a.P));
            return;
        }
        if (p >= a.P - 1) return;
    }
    const int n0 = a.bnd[p], n1 = a.bnd[p + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int g = lane >> 4, r = lane & 15;
    if (p == 0) {
        f32x4_t S[8][2];
        const void *Sg = static_cast<const char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (IN_FMT == kF16 ? 2 : 4);
        if (wave < NSW) tiles_load<IN_FMT, 2>(S, Sg, 32 * wave, g, r);
        run_output(sm, S, a, b, h, n0, n1, n0);
        if (wave < NSW) {
            if (a.P == 1) {
                void *So = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (OUT_FMT == kF16 ? 2 : 4);
                tiles_store<OUT_FMT, 2>(S, So, 32 * wave, g, r);
            } else {
                tiles_store<kF32, 2>(S, carry_slot(a.carry, b, h, a.Hv, a.P, 1, kSst), 32 * wave, g, r);
            }
        }
    } else {
        zero_upper_halves(sm, tid);
        if (wave < NSW) {
            constexpr int NCT = kTransCols / 16;
            const bool is_phi = wave >= 2;
            const int c0 = kTransCols * (wave & 1);
            f32x4_t X[8][NCT];
            trans_init<NCT>(X, c0, is_phi, g, r);
            state_loop_trans<NCT>(sm, X, n0, n1, c0, is_phi, lane);
            tiles_store<kF32, NCT>(X, carry_slot(a.carry, b, h, a.Hv, a.P, p, is_phi ? kPhi : kCst), c0, g, r);
        } else if (wave == NSW + 1 || wave == NSW + 2) {
            constexpr int NCT = kTransHelperCols / 16;
            const int hw = wave - NSW;
            const bool is_phi = hw == 2;
            const int c0 = 2 * kTransCols;
            f32x4_t X[8][NCT];
            trans_init<NCT>(X, c0, is_phi, g, r);
            helper_loop<false, NCT>(sm, a, b, h, n0, n1, hw, lane, X, c0);
            tiles_store<kF32, NCT>(X, carry_slot(a.carry, b, h, a.Hv, a.P, p, is_phi ? kPhi : kCst), c0, g, r);
        } else {
            f32x4_t none[8][1];
            helper_loop<false>(sm, a, b, h, n0, n1, wave - NSW, lane, none);
        }
    }
}

// Pass 2: slot blockIdx.y -> segment p = blockIdx.y + 1, from S_start(p),
// which the workgroup first composes from the pass-1 results (all eight
// waves, 16 columns each) and hands to the state waves through LDS.
template <int OUT_FMT>
__global__ __launch_bounds__(NT) void prefill_pass2_kernel(SegArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem &sm = *reinterpret_cast<Smem *>(smem_raw);
    const int h = head_of(blockIdx.x, a.Hv), p = blockIdx.y + 1, b = blockIdx.z;
    if (head_windowed(a, b, h)) {
        // pass 1 ran it: its final state into the caller's, in 16-byte
        // pieces spread over all of this head's workgroups
        const float *src = carry_slot(a.carry, b, h, a.Hv, a.P, 0, kSst);
        void *So = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (OUT_FMT == kF16 ? 2 : 4);
        for (int i = blockIdx.y * NT + threadIdx.x; i < D * D / 4; i += gridDim.y * NT) {
            const f32x4_t x = *reinterpret_cast<const f32x4_t *>(src + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) state_st<OUT_FMT>(So, 4 * i + e, x[e]);
        }
        return;
    }
    const int n0 = a.bnd[p], n1 = a.bnd[p + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int g = lane >> 4, r = lane & 15;
    f32x4_t S[8][2];
    {
        f32x4_t S16[8][1];
        combine_prefix(*reinterpret_cast<CombSmem *>(smem_raw), S16, a.carry, b, h, a.Hv, a.P, p, tid);
        float *Sl = reinterpret_cast<float *>(smem_raw);  // [128][128] fp32 hand-off
        lds_barrier();
        tiles_store<kF32, 1>(S16, Sl, 16 * wave, g, r);
        lds_barrier();
        if (wave < NSW) tiles_load<kF32, 2>(S, Sl, 32 * wave, g, r);
        lds_barrier();
    }
    run_output(sm, S, a, b, h, n0, n1, n0);
    if (wave < NSW && p == a.P - 1) {
        void *So = static_cast<char *>(a.S) + ((size_t)b * a.Hv + h) * (D * D) * (OUT_FMT == kF16 ? 2 : 4);
        tiles_store<OUT_FMT, 2>(S, So, 32 * wave, g, r);
    }
}

// Segments.  P: at most what fills the device in one pass (about 256
// workgroups), at least kMinSegChunks chunks per segment on average, at most
// kMaxSegs, and the count whose best plan has the lowest modelled time
// (plan_segments); P = 2 would only serialise, so it is never chosen, and
// one segment (the plain recurrence) is kept when no plan beats it.
// Lengths: segment 0
// runs with outputs in pass 1 only; segments 1 .. P-2 run their transition
// in pass 1 (kCostTrans per chunk, relative to a chunk with outputs) and
// rerun with outputs in pass 2 after composing their start state
// (kCostPrologue + kCostStep per transition composed); segment P-1 runs in
// pass 2 only.  The lengths minimise the modelled pass 1 + pass 2 time:
// transitions share one cap M, segment 0 takes kCostTrans * M, and the
// pass-2 segments shrink with their composition cost.  The costs come from
// the kernels' per-chunk times (shader-clock counters: an output chunk 7.4K
// cycles, a composition step 9.3K) and, for the transition chunk since six
// waves share its state, from timing plans of different costs: at T = 16K,
// 32 heads, 1.10 measured 231.1 us against 234.4 (1.20), 232.4 (1.00) and
// 238.5 (1.28, the cost when four waves held the state).
// 4 chunks per segment at least: against 8, short sequences gain more from
// the parallel segments than they lose to transitions (T = 1K: 53.3 against
// 56.6 us, 2K: 68.7 against 77.9 us, 4K: 93.1 against 94.5 us; 3 is as good
// at 1K and worse at 2K)
constexpr int kMinSegChunks = 4;
constexpr int kTargetWgs = 256;
constexpr double kCostTrans = 1.10, kCostStep = 1.26, kCostPrologue = 1.0;

struct SegPlan {
    int P;
    int bnd[kMaxSegs + 1];
};

// Lengths of pass-2 segments p = 1 .. P-1 under the pass-2 bound X, the
// transitions capped at M: len[p] = clamp(floor(X - prologue(p)), 1, M).
int pass2_lengths(int P, int M, double X, int *len) {
    int sum = 0;
    for (int p = 1; p < P; ++p) {
        int l = (int)floor(X - kCostPrologue - kCostStep * (p - 1));
        if (p < P - 1 && l > M) l = M;
        if (l < 1) l = 1;
        len[p] = l;
        sum += l;
    }
    return sum;
}

double plan_cost(int P, const int *len) {
    double t1 = len[0], t2 = 0.0;
    for (int p = 1; p < P; ++p) {
        if (p < P - 1) t1 = fmax(t1, kCostTrans * len[p]);
        t2 = fmax(t2, kCostPrologue + kCostStep * (p - 1) + len[p]);
    }
    return t1 + t2;
}

// The lengths of the cheapest plan with P segments (P >= 3); its modelled
// cost, or +inf when no plan exists.
double plan_lengths(int P, int NC, int *best) {
    int len[kMaxSegs];
    double best_cost = 1e30;
    const int m_max = min(NC, 2 * NC / (P - 1) + 1);  // the cap is near NC / (P - 1)
    for (int M = 1; M <= m_max; ++M) {
        len[0] = min(NC - (P - 1), (int)floor(kCostTrans * M));
        const int rem = NC - len[0];
        if (rem < P - 1 || pass2_lengths(P, M, 1e9, len) < rem) continue;
        double lo = 0.0, hi = NC + kCostPrologue + kCostStep * P;  // pass-2 bound X
        for (int it = 0; it < 40; ++it) {
            const double mid = 0.5 * (lo + hi);
            (pass2_lengths(P, M, mid, len) >= rem ? hi : lo) = mid;
        }
        int sum = pass2_lengths(P, M, hi, len);
        for (int p = P - 1; p >= 1 && sum > rem; --p) {  // trim the excess from the end
            const int cut = min(sum - rem, len[p] - 1);
            len[p] -= cut;
            sum -= cut;
        }
        if (sum != rem) continue;
        const double cost = plan_cost(P, len);
        if (cost < best_cost) {
            best_cost = cost;
            for (int p = 0; p < P; ++p) best[p] = len[p];
        }
    }
    return best_cost;
}

// P is searched up to the number that fills the device once (each pass
// launches (P - 1) x B x Hv workgroups): the composition chain grows with
// P, so with few heads fewer segments than that plan faster (at Hv = 4,
// T = 16K: 23 segments at a modelled 47 chunk times, against 86 for 64).
void plan_segments(int B, int Hv, int NC, SegPlan &pl) {
    const int bh = B * Hv;
    int pmax = 1 + (kTargetWgs + bh - 1) / bh;
    pmax = min(pmax, NC / kMinSegChunks);
    pmax = min(pmax, kMaxSegs);
    int best[kMaxSegs], len[kMaxSegs];
    double best_cost = (double)NC;  // one segment: the plain recurrence
    int best_p = 1;
    for (int P = 3; P <= pmax; ++P) {
        const double cost = plan_lengths(P, NC, len);
        if (cost < best_cost) {
            best_cost = cost;
            best_p = P;
            for (int p = 0; p < P; ++p) best[p] = len[p];
        }
    }
    pl.P = best_p;
    pl.bnd[0] = 0;
    if (best_p == 1) {
        pl.bnd[1] = NC;
        return;
    }
    for (int p = 0; p < best_p; ++p) pl.bnd[p + 1] = pl.bnd[p] + best[p];
}

// The plan of the last shape asked for on this thread (a layer calls the
// prefill with one shape over and over).
const SegPlan &cached_plan(int B, int Hv, int NC) {
    thread_local int key_bh = -1, key_nc = -1;
    thread_local SegPlan plan;
    if (key_bh != B * Hv || key_nc != NC) {
        plan_segments(B, Hv, NC, plan);
        key_bh = B * Hv;
        key_nc = NC;
    }
    return plan;
}

// Windowed plan: P segments whose longest fills the device in the fewest
// rounds of kTargetWgs workgroups.  Segments p >= 1 also run a warm-up
// window (kWinTyp chunks assumed for planning; the device picks 1 ..
// Wmax), so segment 0, which has none, takes kWinTyp more output
// chunks.  Modelled time: rounds x the longest segment's chunks.
constexpr int kWinTyp = 2;

void plan_window(int B, int Hv, int NC, SegPlan &pl) {
    const int bh = B * Hv;
    int best_p = 1;
    long best_cost = NC;
    for (int P = 2; P <= kMaxSegs && P <= NC - kWinTyp; ++P) {
        const long rounds = ((long)bh * P + kTargetWgs - 1) / kTargetWgs;
        const long len = (NC + (long)(P - 1) * kWinTyp + P - 1) / P;
        if (rounds * len < best_cost) {
            best_cost = rounds * len;
            best_p = P;
        }
    }
    pl.P = best_p;
    pl.bnd[0] = 0;
    if (best_p == 1) {
        pl.bnd[1] = NC;
        return;
    }
    // segment 0: L + kWinTyp chunks; the remainder goes to the last segments
    const int L = (NC - kWinTyp) / best_p, rem = (NC - kWinTyp) - L * best_p;
    pl.bnd[1] = L + kWinTyp;
    for (int q = 1; q < best_p; ++q) pl.bnd[q + 1] = pl.bnd[q] + L + (q >= best_p - rem ? 1 : 0);
}

const SegPlan &cached_window_plan(int B, int Hv, int NC) {
    thread_local int key_bh = -1, key_nc = -1;
    thread_local SegPlan plan;
    if (key_bh != B * Hv || key_nc != NC) {
        plan_window(B, Hv, NC, plan);
        key_bh = B * Hv;
        key_nc = NC;
    }
    return plan;
}

// The shape and plan of the last call on each device that could run
// windowed, for prefill_windowed_heads (calls on one device are serialised
// by the caller, which holds that device's lock).
struct LastWindowCall {
    const float *carry = nullptr;
    int B = 0, Hv = 0, P = 0, Pw = 0;
};
constexpr int kMaxDevices = 64;
LastWindowCall g_last_window[kMaxDevices];
LastWindowCall *last_window_slot() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    return &g_last_window[dev];
}

}  // namespace

size_t prefill_carry_bytes(int B, int T, int Hv) {
    const int NC = (T + C - 1) / C;
    const int P = cached_plan(B, Hv, NC).P;
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
    {
        const SegPlan &pl = cached_plan(B, Hv, NC);
        a.P = pl.P;
        for (int p = 0; p <= pl.P; ++p) a.bnd[p] = pl.bnd[p];
    }
    if (a.P > 1 && !carry) return hipErrorInvalidValue;
    static_assert(sizeof(CombSmem) <= sizeof(Smem), "the start-state staging reuses the chunk LDS");
    static_assert(sizeof(Smem) <= 160 * 1024, "LDS budget");
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
    // windowed segments: only where the two-pass path would segment (it
    // provides the carry); the device decides per head which path runs
    if (a.P > 1) {
        const SegPlan &wp = cached_window_plan(B, Hv, NC);
        if (wp.P > 1) {
            a.Pw = wp.P;
            for (int p = 0; p <= wp.P; ++p) a.wbnd[p] = wp.bnd[p];
            a.Wmax = std::min(kWinCap, std::max(kWinMin, NC / wp.P));
        }
    }
    hipError_t e;
    if (a.Pw > 0) {
        prefill_window_check_kernel<<<dim3(Hv, a.Pw - 1, B), 64 * kCheckWaves, 0, st>>>(a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (LastWindowCall *lw = last_window_slot()) *lw = LastWindowCall{a.carry, B, Hv, a.P, a.Pw};
    } else if (LastWindowCall *lw = last_window_slot()) {
        *lw = LastWindowCall{};
    }
    const int slots = a.P > 1 ? a.P - 1 : 1;
    pass1<<<dim3(Hv, a.Pw > slots ? a.Pw : slots, B), NT, smem, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess || a.P == 1) return e;
    pass2<<<dim3(Hv, a.P - 1, B), NT, smem, st>>>(a);
    return hipGetLastError();
}

int prefill_windowed_heads() {
    const LastWindowCall *lw = last_window_slot();
    if (!lw) return -1;
    const LastWindowCall w = *lw;
    if (!w.carry) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    int n = 0;
    for (int b = 0; b < w.B; ++b)
        for (int h = 0; h < w.Hv; ++h) {
            const size_t slot = (((size_t)b * w.Hv + h) * w.P + 0) * 3 + kPhi;
            int words[kMaxSegs];
            if (hipMemcpy(words, w.carry + slot * (size_t)(D * D), sizeof(int) * w.Pw, hipMemcpyDeviceToHost) !=
                hipSuccess)
                return -1;
            bool ok = true;
            for (int p = 1; p < w.Pw; ++p) ok = ok && words[p] >= 0;
            n += ok;
        }
    return n;
}

}  // namespace gdn

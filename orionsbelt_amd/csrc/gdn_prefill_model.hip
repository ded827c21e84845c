// gdn_prefill_model.hip -- the many-row matmul and the causal attention of
// the hybrid model's prefill (include/kai_gdn_hybrid.h) for gfx950.
//
// Prefill GEMM: y[m][n] = scale[n] sum_k x[m][k] Wq[n][k] for M rows (a
// whole prompt), on the same pre-tiled int8 weights as the decode GEMM
// (gdn_model.hip, w8f_tile_kernel) -- the M > 1 counterpart of the
// reference e2e loop's gemm_int8_neon (gdn_e2e_decode.c:606-612).  Block
// tile 128 rows x 128 channels, k in steps of 64, 4 waves as 2 x 2 (64 x 64
// each, four 32x32x16 fp16 MFMA tiles: the larger MFMA shape delivers about
// 1.5 times the 16x16x32 rate on gfx950).  Per step a thread stages 4 x 16
// bytes of activations and 2 x 16 bytes of weights in registers while the
// waves multiply the previous step from LDS; the weights are widened to
// fp16 (exactly) on their way into LDS, so every MFMA operand is one
// 16-byte LDS read.  LDS rows are 64 k + 8 pad halves (144 bytes): the
// 16-byte reads of 8 consecutive rows then cover the 32 banks once.  The
// weight is the A operand, so a lane's accumulators hold runs of 4
// consecutive channels of one row (16-byte stores), and the interleaved
// gate/up rows put each gate channel and its up channel in the same lane.
//
// Prefill attention: Qwen3_5Attention's causal softmax(q k^T / 16) v with
// the sigmoid output gate (modeling_qwen3_5.py:629-701), GQA, head dim 256,
// on the model's fp16 KV cache.  Block (64 positions, kv head), 8 waves: wave
// w takes query head kv * rep + (w % 4) at positions +32 (w / 4) .. +31, as
// two 16-query tiles, and walks the keys in blocks of 64 shared through LDS
// (K and a transposed copy of V, both moved by DMA).  Scores on fp16 MFMA
// 16x16x32 as S^T = K q^T (A = the 16-key x 32-dim fragment, which is one
// contiguous 1 KB of the tiled K cache; B = the tile's queries), online
// softmax in exp2 per query column, then O^T = V^T P^T with P taken from the
// score registers as the B operand (the 8 keys a lane holds, 4g .. 4g+3 and
// 16 + 4g .. 16 + 4g+3, permute the k index of both operands alike).  Each K
// and V fragment read from LDS feeds both query tiles.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int kPBM = 128;    // activation rows per block
constexpr int kPBN = 128;    // channels per block (two 64-channel groups of the tiled weights)
constexpr int kPPitch = 72;  // halves per LDS row: 64 k + 8

struct W8pStage {
    uint16_t x[kPBM * kPPitch];
    uint16_t w[kPBN * kPPitch];
};

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Epilogue of one 32x32 accumulator tile (channels nt .. nt+31, one row per
// lane): lane l holds, for q = 0..3, channels nt + 8 q + 4 (l / 32) .. +3 of
// its row (C element 4 q + e).
GDN_DEV void w8p_store_tile(const f32x16_t &acc, int row, int nt, int h2, const float *__restrict__ scale, int N,
                            const W8Out &out) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = nt + 8 * q + 4 * h2;
        const f32x4_t sc = *reinterpret_cast<const f32x4_t *>(scale + n);
        f32x4_t y = f32x4_t{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]} * sc;
        if (out.mode == kW8SwiGLU) {
            // 16-channel groups: 8 gate channels (q even), then their 8 up channels (q + 1)
            if (q & 1) continue;
            const f32x4_t su = *reinterpret_cast<const f32x4_t *>(scale + n + 8);
            const f32x4_t up = f32x4_t{acc[4 * q + 4], acc[4 * q + 5], acc[4 * q + 6], acc[4 * q + 7]} * su;
            uint32_t hv[2];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float a = y[e] / (1.0f + expf(-y[e])) * up[e];
                const float b = y[e + 1] / (1.0f + expf(-y[e + 1])) * up[e + 1];
                hv[e / 2] = (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
            }
            const int cc = (nt + 16 * (q >> 1)) / 2 + 4 * h2;
            *reinterpret_cast<uint2 *>(out.x16 + (size_t)row * (N / 2) + cc) = make_uint2(hv[0], hv[1]);
        } else if (n < out.seg[out.nseg - 1].n_end) {  // channels past the last segment: padding
            int sgi = 0, nb = 0;
#pragma unroll
            for (int qq = 0; qq < kW8MaxSegs - 1; ++qq)
                if (qq < out.nseg - 1 && n >= out.seg[qq].n_end) {
                    sgi = qq + 1;
                    nb = out.seg[qq].n_end;
                }
            float *dst = out.seg[0].dst;
            int ld = out.seg[0].ld;
#pragma unroll
            for (int qq = 1; qq < kW8MaxSegs; ++qq)
                if (qq == sgi) {
                    dst = out.seg[qq].dst;
                    ld = out.seg[qq].ld;
                }
            // the residual add (one segment): may be in place, each element
            // is read and written by this lane only
            if (out.add_in) y = *reinterpret_cast<const f32x4_t *>(out.add_in + (size_t)row * out.add_ld + n) + y;
            *reinterpret_cast<f32x4_t *>(dst + (size_t)row * ld + (n - nb)) = y;
        }
    }
}

__global__ __launch_bounds__(256, 2) void w8p_kernel(const uint16_t *__restrict__ X, int ldx,
                                                     const int8_t *__restrict__ W, const float *__restrict__ scale,
                                                     int M, int N, int K, W8Out out) {
    __shared__ __align__(16) W8pStage st[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;  // rows 64 wm .., channels 64 wn .. of the block
    const int n0 = blockIdx.x * kPBN, m0 = blockIdx.y * kPBM;
    const int steps = K / 64;
    const bool two = n0 + 64 < N;        // the block's second channel group exists
    const bool active = wn == 0 || two;  // this wave's channels exist (wave-uniform)

    // staging: activation chunk c = tid + 256 i is row c / 8, k 8 (c % 8) .. +7
    // (rows past M read row M - 1, never stored); weight chunk tid of each
    // group's 4 KB step block (tile tid / 64, tiled lane tid % 64)
    const uint16_t *xp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        xp[i] = X + (size_t)min(m0 + (c >> 3), M - 1) * ldx + (c & 7) * 8;
    }
    const int8_t *wp0 = W + (size_t)(n0 / 64) * steps * 4096 + tid * 16;
    const int8_t *wp1 = two ? wp0 + (size_t)steps * 4096 : wp0;
    // Two register stages: the loads of step s + 2 are issued before the
    // waves multiply step s, so each load has two steps' compute to land.
    struct Stage {
        u32x4_t x[4], w[2];
    };
    auto gload = [&](int s, Stage &r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r.x[i] = *reinterpret_cast<const u32x4_t *>(xp[i] + s * 64);
        r.w[0] = *reinterpret_cast<const u32x4_t *>(wp0 + (size_t)s * 4096);
        r.w[1] = *reinterpret_cast<const u32x4_t *>(wp1 + (size_t)s * 4096);
    };
    const int wq = tid & 63, wrow = 16 * (tid >> 6) + (wq & 15), wk = 16 * (wq >> 4);
    auto lstore = [&](int b, const Stage &r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<u32x4_t *>(&st[b].x[(c >> 3) * kPPitch + (c & 7) * 8]) = r.x[i];
        }
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            f16x8_t lo, hi;
            i8x16_to_f16(r.w[gi], lo, hi);
            uint16_t *d = &st[b].w[(64 * gi + wrow) * kPPitch + wk];
            *reinterpret_cast<f16x8_t *>(d) = lo;
            *reinterpret_cast<f16x8_t *>(d + 8) = hi;
        }
    };

    // 32x32x16 fp16 MFMA: A lane l = W row (channel) l % 32, k 8 (l / 32)
    // .. +7; B lane l = x row l % 32, the same k; C element e of lane l =
    // channel 8 (e / 4) + 4 (l / 32) + e % 4, row l % 32
    f32x16_t acc[2][2];  // [channel tile jt][row tile it], 32 x 32 each
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[jt][it][e] = 0.f;
    const int l32 = lane & 31, h2 = lane >> 5;
    auto compute = [&](int b) {
        if (!active) return;
#pragma unroll
        for (int kk = 0; kk < 64; kk += 16) {
            f16x8_t a[2], bx[2];
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
                a[jt] = *reinterpret_cast<const f16x8_t *>(
                    &st[b].w[(64 * wn + 32 * jt + l32) * kPPitch + kk + 8 * h2]);
#pragma unroll
            for (int it = 0; it < 2; ++it)
                bx[it] = *reinterpret_cast<const f16x8_t *>(
                    &st[b].x[(64 * wm + 32 * it + l32) * kPPitch + kk + 8 * h2]);
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
#pragma unroll
                for (int it = 0; it < 2; ++it)
                    acc[jt][it] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[jt], bx[it], acc[jt][it], 0, 0, 0);
        }
    };

    // step s: registers R[s % 2], LDS buffer s % 2; the loop is unrolled by
    // two so that every register stage is a fixed set of registers
    // Loads are issued on every turn (past the last step they re-read it:
    // in bounds, never stored), so that every path has the same loads in
    // flight and the compiler waits only for the older stage.
    Stage R0, R1;
    const int last = steps - 1;
    gload(0, R0);
    gload(min(1, last), R1);
    lstore(0, R0);
    __syncthreads();
    for (int s = 0; s < steps; s += 2) {
        // even step s: R0 is free (stored at the previous turn)
        gload(min(s + 2, last), R0);
        compute(0);
        if (s + 1 < steps) lstore(1, R1);
        __syncthreads();
        if (s + 1 >= steps) break;
        // odd step s + 1: R1 is free
        gload(min(s + 3, last), R1);
        compute(1);
        if (s + 2 < steps) lstore(0, R0);
        __syncthreads();
    }
    if (!active) return;

    // lane l of tile (jt, it): row m0 + 64 wm + 32 it + l % 32, channels from
    // n0 + 64 wn + 32 jt
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int row = m0 + 64 * wm + 32 * it + l32;
            if (row < M) w8p_store_tile(acc[jt][it], row, n0 + 64 * wn + 32 * jt, h2, scale, N, out);
        }
}

// The large-tile form: block 256 rows x 256 channels, 8 waves as 2 x 4
// (128 rows x 64 channels each: 4 x 2 tiles of 32x32x16 fp16 MFMA).  Both
// operands of a 64-k step reach LDS by DMA (global_load_lds, 1 KB per wave
// instruction): the 256 activation rows (32 KB) and the four 4 KB weight
// tiles of the block's channel groups, copied as they lie.  The buffers
// form a ring of three steps held in separate arrays, so that the compiler
// can tell the slot being filled from the slot being read and does not wait
// for the DMA before every LDS read; the loads of step s + 2 are issued
// into the slot step s - 1 used, and one wait on the vector memory counter
// before each barrier makes step s + 1's tiles complete.  An activation row
// is 128 B; its 16-byte piece p sits in slot p ^ ((row / 2) % 8), so that
// the 16 rows a quarter-wave reads cover all 64 banks.  The weights are
// widened to fp16 from LDS.  Lane l of a 32-channel MFMA tile reads, from
// 16-row weight tile 2 jt + (l % 32) / 16, row l % 16 and the 16-byte
// pieces g' = l / 32 and l / 32 + 2 of the 64-k step (k 16 g' .. +15); MFMA
// kk (4 per step) takes 8 of them: k = 32 (kk / 2) + 16 (l / 32) + 8 (kk %
// 2) .. +7, and the activation (B) lanes read the same k.
// Measured at M = 32768 on the 4B shapes: 12-19% faster than the same tile
// with the weights loaded into registers and the activations staged through
// registers (gate|up 1060-1086 against 933-965 TFLOP/s), bit-identical.
constexpr int kPBM2 = 256;
constexpr int kPBN2 = 256;
// Rows from which the large-tile form is used: below two row blocks its
// tile would be mostly padding.
constexpr int kW8pLargeRows = 512;

typedef __attribute__((address_space(3))) void lds_void_t;
// LDS index (halves) of the 16-byte piece `piece` of activation row `row`
GDN_DEV int dswz(int row, int piece) { return row * 64 + ((piece ^ ((row >> 1) & 7)) << 3); }
// wait until at most N vector memory operations of this wave are outstanding
template <int N> GDN_DEV void wait_vm() { __builtin_amdgcn_s_waitcnt((N & 15) | 0x0F70 | ((N >> 4) << 14)); }
// barrier that waits for this wave's LDS operations only (not for its DMA)
GDN_DEV void lds_bar() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__global__ __launch_bounds__(512, 1) void w8p2_kernel(const uint16_t *__restrict__ X, int ldx,
                                                      const int8_t *__restrict__ W, const float *__restrict__ scale,
                                                      int M, int N, int K, W8Out out) {
    __shared__ __align__(16) uint16_t xa[kPBM2 * 64];
    __shared__ __align__(16) uint16_t xb[kPBM2 * 64];
    __shared__ __align__(16) uint16_t xc[kPBM2 * 64];
    __shared__ __align__(16) int8_t wa[4 * 4096];
    __shared__ __align__(16) int8_t wb[4 * 4096];
    __shared__ __align__(16) int8_t wc[4 * 4096];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int n0 = blockIdx.x * kPBN2, m0 = blockIdx.y * kPBM2;
    const int steps = K / 64;
    const int cg = n0 / 64 + wn;
    const bool active = cg < N / 64;
    const int l32 = lane & 31, h2 = lane >> 5;
    const uint16_t *xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 32 * wave + 8 * i + (lane >> 3);
        const int piece = (lane & 7) ^ ((row >> 1) & 7);
        xsrc[i] = X + (size_t)min(m0 + row, M - 1) * ldx + piece * 8;
    }
    // weight DMA: wave w moves kilobytes 2w and 2w + 1 of the block's four
    // 4 KB group tiles (group (2w + i) / 4, absent groups re-read group 0)
    const int8_t *wsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int kb = 2 * wave + i, g = kb >> 2;
        const int gg = n0 / 64 + g < N / 64 ? n0 / 64 + g : 0;
        wsrc[i] = W + (size_t)gg * steps * 4096 + (kb & 3) * 1024 + lane * 16;
    }
    auto dma = [&](int s, uint16_t *xbuf, int8_t *wbuf) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(xsrc[i] + s * 64, (lds_void_t *)(xbuf + (32 * wave + 8 * i) * 64), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(wsrc[i] + (size_t)s * 4096, (lds_void_t *)(wbuf + (2 * wave + i) * 1024), 16, 0, 0);
    };
    const int woff = wn * 4096 + (l32 >> 4) * 1024 + (16 * h2 + (l32 & 15)) * 16;
    f32x16_t acc[2][4];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int it = 0; it < 4; ++it)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[jt][it][e] = 0.f;
    auto compute = [&](const uint16_t *buf, const int8_t *wbuf) {
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) {
            f16x8_t a[2][2];
#pragma unroll
            for (int jt = 0; jt < 2; ++jt)
                i8x16_to_f16(*reinterpret_cast<const u32x4_t *>(wbuf + woff + jt * 2048 + pc * 512), a[jt][0], a[jt][1]);
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int kk = 2 * pc + k2;
                const int piece = 4 * (kk >> 1) + 2 * h2 + (kk & 1);
                f16x8_t bx[4];
#pragma unroll
                for (int it = 0; it < 4; ++it)
                    bx[it] = *reinterpret_cast<const f16x8_t *>(&buf[dswz(128 * wm + 32 * it + l32, piece)]);
#pragma unroll
                for (int jt = 0; jt < 2; ++jt)
#pragma unroll
                    for (int it = 0; it < 4; ++it)
                        acc[jt][it] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[jt][k2], bx[it], acc[jt][it], 0, 0, 0);
            }
        }
    };
    const int last = steps - 1;
    dma(0, xa, wa);
    dma(min(1, last), xb, wb);
    wait_vm<6>();  // step 0 landed
    lds_bar();
    // step s: its tiles in ring slot s % 3; the tiles of step s + 2 go into
    // the slot step s - 1 used; step s + 1's tiles must land before the
    // barrier that ends step s (after them come the 6 loads of step s + 2)
#define W8P2_STEP(S, CX, CW, NX, NW)             \
    dma(min((S) + 2, last), NX, NW);             \
    compute(CX, CW);                             \
    wait_vm<6>();                                \
    lds_bar();                                   \
    if ((S) + 1 >= steps) break;
    for (int s = 0;; s += 3) {
        W8P2_STEP(s, xa, wa, xc, wc)
        W8P2_STEP(s + 1, xb, wb, xa, wa)
        W8P2_STEP(s + 2, xc, wc, xb, wb)
    }
#undef W8P2_STEP
    wait_vm<0>();
    if (!active) return;
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int row = m0 + 128 * wm + 32 * it + l32;
            if (row < M) w8p_store_tile(acc[jt][it], row, n0 + 64 * wn + 32 * jt, h2, scale, N, out);
        }
}

// ---- causal prefill attention ------------------------------------------------

constexpr int kApQ = 64;       // positions per block
constexpr int kApK = 64;       // keys per step
constexpr int kApD = 256;      // head dim

// V^T tile in LDS: [256 dims][64 keys], 128 bytes per dim row, the 16-byte
// piece c of row d in slot c ^ (d % 8): a fragment read (16 rows x 32
// bytes) then covers every bank twice, the minimum.
GDN_DEV int vt_slot(int d, int c) { return d * kApK + ((c ^ (d & 7)) << 3); }

// Block (64 positions, kv head), 8 waves: wave w takes query head
// kv * rep + (w % 4) at positions +32 (w / 4) .. +31, as two 16-query tiles
// that share every K and V fragment the wave reads from LDS (two MFMAs per
// fragment read, against one with a tile per wave: the LDS reads bounded
// that form).  K (the cache's tiled layout, 32 KB per step, contiguous) and
// V^T (from the transposed copy) reach LDS by DMA, double buffered.
constexpr int kApT = 2;  // query tiles per wave
constexpr int kApThreads = 512;

__global__ __launch_bounds__(kApThreads) void attn_prefill_kernel(
    const uint16_t *__restrict__ q16, const uint16_t *__restrict__ Kc, const uint16_t *__restrict__ vT,
    const float *__restrict__ gate, int gate_row, uint16_t *__restrict__ out16, int T, int Hq, int Hkv, int Tmax,
    int Tv, float sc_log2) {
    __shared__ __align__(16) uint16_t ks[2][kApK * kApD];  // tiled as in the cache
    __shared__ __align__(16) uint16_t vs[2][kApD * kApK];  // [dim][key], swizzled pieces
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: the DMA addresses stay in SGPRs
    const int g = lane >> 4, r = lane & 15;
    const int qb = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest blocks first
    const int kv = blockIdx.y;
    const int rep = Hq / Hkv;
    const bool live = (wave & 3) < rep;                   // wave-uniform
    const int h = kv * rep + min(wave & 3, rep - 1);
    int qpos[kApT];
#pragma unroll
    for (int qt = 0; qt < kApT; ++qt) qpos[qt] = qb * kApQ + 32 * (wave >> 2) + 16 * qt + r;  // B column r

    // the wave's queries as B operands: dims 32 j + 8 g .. +7 of query r
    f16x8_t qf[kApT][8];
#pragma unroll
    for (int qt = 0; qt < kApT; ++qt) {
        const uint16_t *qp = q16 + ((size_t)min(qpos[qt], T - 1) * Hq + h) * kApD + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[qt][j] = *reinterpret_cast<const f16x8_t *>(qp + 32 * j);
    }
    f32x4_t o[kApT][16];  // O^T per tile: dims 16 dt + 4 g + e of query r
#pragma unroll
    for (int qt = 0; qt < kApT; ++qt)
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) o[qt][dt] = zero4();
    // running max (log2 units, all lanes of column r agree) and partial sum, per tile
    float m[kApT], l[kApT];
#pragma unroll
    for (int qt = 0; qt < kApT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.f;
    }

    const int kend = min(T, qb * kApQ + kApQ);
    const int nkb = (kend + kApK - 1) / kApK;
    const uint16_t *kbase = Kc + (size_t)kv * Tmax * kApD;
    const uint16_t *vbase = vT + (size_t)kv * kApD * Tv;
    // DMA of step kb into buffer b: wave w moves K kilobytes 4w .. 4w+3 (of
    // 16-key group w / 2: a group past the cache rows reads the last group
    // instead, its keys are masked, every key >= T lies after every query)
    // and V^T rows 32 w .. 32 w + 31 (8 per instruction)
    // per-lane parts of the DMA addresses (loop-invariant): K chunk lane of a
    // kilobyte; V^T row lane / 8 of an 8-row group (whose first row is a
    // multiple of 8, so the row's swizzle is (lane / 8) % 8), piece lane % 8
    const int koff = lane * 8;
    const int voff = (lane >> 3) * Tv + 8 * ((lane & 7) ^ (lane >> 3));
    auto dma = [&](int kb, int b) {
        const int t0 = min(kb * kApK + 16 * (wave >> 1), Tmax - 16);
        const uint16_t *kp = kbase + (size_t)t0 * kApD + (4 * (wave & 1)) * 512;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(kp + i * 512 + koff, (lds_void_t *)&ks[b][(4 * wave + i) * 512], 16, 0,
                                             0);
        const uint16_t *vp = vbase + (size_t)(32 * wave) * Tv + kb * kApK;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(vp + (size_t)(8 * i) * Tv + voff,
                                             (lds_void_t *)&vs[b][(32 * wave + 8 * i) * kApK], 16, 0, 0);
    };
    // One step: the 64 keys of buffer b as two halves of 32, each an online
    // softmax update (scores, P, then P V), so that one half's scores and P
    // fragments are live at a time (registers).
    auto step = [&](int b, int kb) {
        if (!live) return;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            // S^T tiles: keys kb * 64 + 32 half + 16 kh + 4 g + e, query r of tile qt
            f32x4_t s[kApT][2];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const int kt = 2 * half + kh;
#pragma unroll
                for (int qt = 0; qt < kApT; ++qt) s[qt][kh] = zero4();
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const f16x8_t kf = *reinterpret_cast<const f16x8_t *>(&ks[b][kt * 4096 + j * 512 + lane * 8]);
#pragma unroll
                    for (int qt = 0; qt < kApT; ++qt)
                        s[qt][kh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[qt][j], s[qt][kh], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);  // one key tile's fragments in flight at a time
            }
            f16x8_t pb[kApT];  // P^T fragments: keys 32 half + {4g .. 4g+3, 16 + 4g .. 16 + 4g+3}
#pragma unroll
            for (int qt = 0; qt < kApT; ++qt) {
                float mx = m[qt];
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int key = kb * kApK + 32 * half + 16 * kh + 4 * g + e;
                        const float v = key <= qpos[qt] ? s[qt][kh][e] * sc_log2 : -INFINITY;
                        s[qt][kh][e] = v;
                        mx = fmaxf(mx, v);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                // the first half of the first step holds key 0, which precedes
                // every query: mx is finite from then on (a later fully
                // masked half leaves m and alpha = 1 unchanged)
                const float alpha = __builtin_amdgcn_exp2f(m[qt] - mx);
                m[qt] = mx;
                // once the running maxima settle, alpha is 1 in every lane: skip
                // the 64 multiplies of O (x * 1 = x, so the result is the same)
                if (__ballot(alpha != 1.0f)) {
                    l[qt] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 16; ++dt) o[qt][dt] *= alpha;
                }
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float p = __builtin_amdgcn_exp2f(s[qt][kh][e] - mx);
                        l[qt] += p;
                        pb[qt][kh * 4 + e] = (_Float16)p;
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
            // per-lane V^T offsets of this half, recomputed here (a few VALU
            // operations) rather than kept live across the step: row r, keys
            // 32 half + 4 g .. +3 (piece 4 half + g / 2, half g % 2) and 16
            // keys further (piece + 2); row 16 dt + r adds 1024 dt
            int vlo, vhi;
            {
                int ln = lane;
                __asm__ volatile("" : "+v"(ln));
                const int gg = ln >> 4, rr = ln & 15;
                vlo = vt_slot(rr, 4 * half + (gg >> 1)) + 4 * (gg & 1);
                vhi = vt_slot(rr, 4 * half + 2 + (gg >> 1)) + 4 * (gg & 1);
            }
#pragma unroll
            for (int dt = 0; dt < 16; ++dt) {
                const uint16_t *vb = &vs[b][1024 * dt];  // rows 16 dt + r keep their swizzle (16 dt % 8 = 0)
                const u32x2_t lo = *reinterpret_cast<const u32x2_t *>(vb + vlo);
                const u32x2_t hi = *reinterpret_cast<const u32x2_t *>(vb + vhi);
                const f16x8_t a = __builtin_bit_cast(f16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
                for (int qt = 0; qt < kApT; ++qt)
                    o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[qt], o[qt][dt], 0, 0, 0);
                if ((dt & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // four V fragments in flight
            }
        }
    };

    dma(0, 0);
    wait_vm<0>();
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        if (kb + 1 < nkb) dma(kb + 1, (kb + 1) & 1);  // into the buffer step kb - 1 read
        step(kb & 1, kb);
        wait_vm<0>();
        __syncthreads();
    }
    if (!live) return;
#pragma unroll
    for (int qt = 0; qt < kApT; ++qt) {
        // lanes of one query column agree on qpos, so the shuffles stay within active lanes
        if (qpos[qt] >= T) continue;
        float lt = l[qt];
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        const float inv = 1.0f / lt;
        const float *gp = gate + (size_t)qpos[qt] * gate_row + (size_t)h * 512;
        uint16_t *op = out16 + ((size_t)qpos[qt] * Hq + h) * kApD;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
            const int d = 16 * dt + 4 * g;
            const f32x4_t gt = *reinterpret_cast<const f32x4_t *>(gp + d);
            uint32_t hv[2];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float a = (o[qt][dt][e] * inv) * (1.0f / (1.0f + expf(-gt[e])));
                const float b = (o[qt][dt][e + 1] * inv) * (1.0f / (1.0f + expf(-gt[e + 1])));
                hv[e / 2] = (uint32_t)f32_to_f16_rne(a) | ((uint32_t)f32_to_f16_rne(b) << 16);
            }
            *reinterpret_cast<uint2 *>(op + d) = make_uint2(hv[0], hv[1]);
        }
    }
}

}  // namespace

long long w8p_max_rows() { return 65535LL * kPBM2; }

hipError_t launch_w8p(const uint16_t *x, int ldx, const int8_t *W, const float *scale, int M, int N, int K,
                      const W8Out &out, hipStream_t st) {
    if (M <= 0) return hipSuccess;
    if (N <= 0 || N % 64 || K <= 0 || K % 64 || ldx < K || ldx % 8 || (uintptr_t)x % 16 ||
        (out.mode != kW8Segments && out.mode != kW8SwiGLU) || (out.mode == kW8SwiGLU && (N % 16 || !out.x16)) ||
        (out.mode == kW8Segments && (out.nseg < 1 || out.nseg > kW8MaxSegs)) ||
        (out.add_in && (out.mode != kW8Segments || out.nseg != 1)))
        return hipErrorInvalidValue;
    if (M >= kW8pLargeRows) {
        const long long mb = (M + kPBM2 - 1) / kPBM2;
        if (mb > 65535) return hipErrorInvalidValue;
        w8p2_kernel<<<dim3((unsigned)((N + kPBN2 - 1) / kPBN2), (unsigned)mb), 512, 0, st>>>(x, ldx, W, scale, M, N,
                                                                                           K, out);
        return hipGetLastError();
    }
    const long long mb = (M + kPBM - 1) / kPBM;
    w8p_kernel<<<dim3((unsigned)((N + kPBN - 1) / kPBN), (unsigned)mb), 256, 0, st>>>(x, ldx, W, scale, M, N, K, out);
    return hipGetLastError();
}

hipError_t launch_attn_prefill(const uint16_t *q16, const uint16_t *Kc, const uint16_t *vT, const float *gate,
                               int gate_row, uint16_t *out16, int T, int Hq, int Hkv, int Tmax, int Tv,
                               float scaling, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (Hkv <= 0 || Hq % Hkv || Hq / Hkv > 4 || Tmax % 16 || Tmax < T || Tv % kApK || Tv < T)
        return hipErrorInvalidValue;
    const float sc_log2 = scaling * 1.4426950408889634f;
    attn_prefill_kernel<<<dim3((unsigned)((T + kApQ - 1) / kApQ), (unsigned)Hkv), kApThreads, 0, st>>>(
        q16, Kc, vT, gate, gate_row, out16, T, Hq, Hkv, Tmax, Tv, sc_log2);
    return hipGetLastError();
}

}  // namespace gdn

// gdn_stream.hip -- HBM-streaming GDN kernels for gfx950:
//   causal depthwise conv1d K=4 (+ optional SiLU epilogue),
//   cumulative decay and diagonal gated scan (single-pass decoupled
//   look-back over sequence tiles), M=1 GEMV.
//
// All layouts are the reference kai layouts: [seq][channels] row-major with
// channels contiguous, so a wavefront reading one row of 64 channels issues
// one contiguous 256 B (or 1 KiB with float4) request.
#include <type_traits>

#include <algorithm>

#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

// ---------------------------------------------------------------------------
// Causal depthwise conv1d, K = 4
// ---------------------------------------------------------------------------
// Semantics: kai_gdn_causal_dwconv1d_f32_k4_sve.c:149-166 (scalar branch).
// Thread = VEC consecutive channels x one segment of seg_len timesteps.  The
// three history inputs of a segment are read from `in` (rows t0-3..t0-1), or
// from hist for segment 0, so segments are independent and the grid is
// (channels / VEC / 256) x (seq / seg_len) blocks.  Short segments (8 rows:
// one group of row loads per thread, issued together) keep thousands of
// workgroups streaming; the halo rows re-read from `in` were just read by
// the neighbouring segment's workgroup on the same XCD and hit in L2.  Only
// segment-0 threads touch hist: they read it first and write the new
// history last, so no two threads race on it.  FP contraction is off, making
// the K=4 dot product ((h0*w0 + h1*w1) + h2*w2) + cur*w3 bit-identical to the
// portable scalar C.

template <int VEC> struct Vec;
template <> struct Vec<1> { using T = float; };
template <> struct Vec<4> { using T = float4; };

template <int VEC, bool NT = false>
GDN_DEV typename Vec<VEC>::T vload(const float *p) {
    if constexpr (VEC == 4) return load_f4<NT>(p);
    else if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <int VEC, bool NT = false>
GDN_DEV void vstore(float *p, typename Vec<VEC>::T v) {
    if constexpr (VEC == 4) store_f4<NT>(p, v);
    else if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

GDN_DEV float conv_tap(float h0, float h1, float h2, float cur, float w0, float w1,
                       float w2, float w3, bool silu) {
#pragma clang fp contract(off)
    float acc = h0 * w0 + h1 * w1 + h2 * w2 + cur * w3;
    if (silu) acc = acc / (1.0f + expf(-acc));
    return acc;
}

GDN_DEV float4 conv_tap(float4 h0, float4 h1, float4 h2, float4 cur, float4 w0, float4 w1,
                        float4 w2, float4 w3, bool silu) {
    return make_float4(conv_tap(h0.x, h1.x, h2.x, cur.x, w0.x, w1.x, w2.x, w3.x, silu),
                       conv_tap(h0.y, h1.y, h2.y, cur.y, w0.y, w1.y, w2.y, w3.y, silu),
                       conv_tap(h0.z, h1.z, h2.z, cur.z, w0.z, w1.z, w2.z, w3.z, silu),
                       conv_tap(h0.w, h1.w, h2.w, cur.w, w0.w, w1.w, w2.w, w3.w, silu));
}

// NT: non-temporal streaming of the rows each thread reads once and of out.
template <int VEC, bool SILU, bool NT>
__global__ __launch_bounds__(256) void conv_k4_kernel(const float *__restrict__ in,
                                                      const float *__restrict__ w,
                                                      float *out, float *__restrict__ hist,
                                                      int64_t seq, int64_t ch,
                                                      int64_t seg_len) {
    using V = typename Vec<VEC>::T;
    constexpr int U = 8;  // rows in flight per thread
    const int64_t ngroups = ch / VEC;
    const int64_t cg = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (cg >= ngroups) return;
    const int64_t c = cg * VEC;
    const int64_t seg = blockIdx.y;
    const int64_t t0 = seg * seg_len;
    const int64_t t1 = min(seq, t0 + seg_len);

    const V w0 = vload<VEC>(w + 0 * ch + c), w1 = vload<VEC>(w + 1 * ch + c);
    const V w2 = vload<VEC>(w + 2 * ch + c), w3 = vload<VEC>(w + 3 * ch + c);
    V h0, h1, h2, oh0, oh1, oh2;
    if (seg == 0) {
        oh0 = h0 = vload<VEC>(hist + 0 * ch + c);
        oh1 = h1 = vload<VEC>(hist + 1 * ch + c);
        oh2 = h2 = vload<VEC>(hist + 2 * ch + c);
    } else {
        h0 = vload<VEC>(in + (t0 - 3) * ch + c);
        h1 = vload<VEC>(in + (t0 - 2) * ch + c);
        h2 = vload<VEC>(in + (t0 - 1) * ch + c);
    }

    for (int64_t t = t0; t < t1; t += U) {
        // Row loads are unconditional (rows past the end clamp to the last
        // row and are not used), so the U loads issue back to back.
        V cur[U];
#pragma unroll
        for (int i = 0; i < U; ++i) cur[i] = vload<VEC, NT>(in + min(t + i, seq - 1) * ch + c);
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (t + i < t1) {
                vstore<VEC, NT>(out + (t + i) * ch + c,
                                conv_tap(h0, h1, h2, cur[i], w0, w1, w2, w3, SILU));
                h0 = h1;
                h1 = h2;
                h2 = cur[i];
            }
        }
    }

    if (seg == 0) {
        if (gridDim.y == 1) {
            // Whole sequence in this thread: the registers hold the last three
            // inputs (old history included when seq < 3), as the reference does.
            // Also correct when out aliases in.
            vstore<VEC>(hist + 0 * ch + c, h0);
            vstore<VEC>(hist + 1 * ch + c, h1);
            vstore<VEC>(hist + 2 * ch + c, h2);
        } else {
            // Several segments (then seq > seg_len >= 4): the new history is
            // the last three input rows.
            (void)oh0; (void)oh1; (void)oh2;
            vstore<VEC>(hist + 0 * ch + c, vload<VEC>(in + (seq - 3) * ch + c));
            vstore<VEC>(hist + 1 * ch + c, vload<VEC>(in + (seq - 2) * ch + c));
            vstore<VEC>(hist + 2 * ch + c, vload<VEC>(in + (seq - 1) * ch + c));
        }
    }
}

// ---------------------------------------------------------------------------
// Cumulative decay / diagonal gated scan: decoupled look-back
// ---------------------------------------------------------------------------
// Recurrence per channel: s_t = g_t * s_{t-1} + x_t (mode 1, the kai gated
// scan, kai_gdn_gated_scan_f32_sve.c:86-95) or s_t = s_{t-1} * a_t from
// s_{-1} = 1 (mode 0, kai cumdecay, kai_gdn_cumdecay_f32_sve.c:82-90).
//
// A tile is RH * TS rows x 256 channels, held in registers by a workgroup of
// RH row groups x 256 threads: thread (row group q, lane l) owns channel l
// of rows q*TS .. q*TS+TS-1.  The kernel is persistent: a grid of as many
// workgroups as fit on the device takes tile ids from a device counter in
// order (row tiles of a column strip in sequence order), so every tile a
// workgroup waits for is held by a running workgroup and was taken earlier.
// Per tile:
//   1. each row group folds its rows into a map s -> AG*s + AX, in the
//      reference's order starting from the identity; the maps of the row
//      groups are composed in LDS into the tile's aggregate;
//   2. the tile publishes its aggregate (row tile > 0);
//   3. row group 0 looks back over predecessor tiles, composing their
//      aggregates until one has published its inclusive state;
//   4. the row groups re-run the reference recurrence over their rows one
//      after another from that carry (the carry passes between them in LDS),
//      the last publishes the tile's inclusive state, and all store.
// With PF the next tile id is taken and its rows are loaded before step 3,
// so the look-back waits overlap the next tile's reads.  Only the carry into
// a tile is re-associated; inside a tile the arithmetic is the reference's,
// and row tile 0 is bit-identical to it.  Every tile a waiting workgroup
// depends on has a smaller id; the smallest unfinished id is always some
// workgroup's current tile, whose predecessors are all finished, so the
// wait always ends.
//
// Status words are 64-bit: (epoch << 32) | float bits.  A word belongs to
// the current launch iff its tag equals `epoch`, so each word validates
// itself and no fences are needed; the arrays are never cleared between
// launches.  The wait is bounded: past kSpinLimit polls the tile records an
// error in *err and carries 0, so every wave exits.

GDN_DEV unsigned long long pack_status(uint32_t epoch, float v) {
    return ((unsigned long long)epoch << 32) | (unsigned long long)__float_as_uint(v);
}
GDN_DEV uint32_t status_tag(unsigned long long w) { return (uint32_t)(w >> 32); }
GDN_DEV float status_val(unsigned long long w) { return __uint_as_float((uint32_t)w); }

GDN_DEV unsigned long long load_status(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
GDN_DEV void store_status(unsigned long long *p, unsigned long long w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NARROW> GDN_DEV float narrow_load(const void *p, int64_t i) {
    if constexpr (NARROW == kF16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else if constexpr (NARROW == kBF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    else return static_cast<const float *>(p)[i];
}
template <int NARROW> GDN_DEV void narrow_store(void *p, int64_t i, float v) {
    if constexpr (NARROW == kF16) static_cast<uint16_t *>(p)[i] = f32_to_f16_rne(v);
    else if constexpr (NARROW == kBF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16_rne(v);
    else static_cast<float *>(p)[i] = v;
}

constexpr uint32_t kSpinLimit = 1u << 22;

// Rows of one row group, loaded unconditionally.  WHOLE: the launch has only
// whole tiles (seq and channels multiples of the tile), so plain addressing;
// otherwise rows past the sequence end and lanes past the channel end clamp
// to the last valid row / channel (their values are never used).
template <int MODE, int TS, bool NT, bool WHOLE>
GDN_DEV void scan_load_rows(const float *g, const float *x, int64_t seq, int64_t ch,
                            int64_t row0, int64_t c, float (&gv)[TS], float (&xv)[TS]) {
    const int64_t cc = WHOLE ? c : min(c, ch - 1);
#pragma unroll
    for (int i = 0; i < TS; ++i) {
        const int64_t at = (WHOLE ? row0 + i : min(row0 + i, seq - 1)) * ch + cc;
        if constexpr (NT) {
            gv[i] = __builtin_nontemporal_load(g + at);
            if constexpr (MODE == 1) xv[i] = __builtin_nontemporal_load(x + at);
        } else {
            gv[i] = g[at];
            if constexpr (MODE == 1) xv[i] = x[at];
        }
    }
}

template <int MODE, int NARROW, bool NT>
GDN_DEV void scan_store(void *out, int64_t at, float gvi, float xvi) {
    float *o32 = static_cast<float *>(out) + at;
    if constexpr (MODE == 1) {
        if constexpr (NT) __builtin_nontemporal_store(xvi, o32);
        else *o32 = xvi;
    } else if constexpr (NARROW == kF32 && NT) {
        __builtin_nontemporal_store(gvi, o32);
    } else {
        narrow_store<NARROW>(out, at, gvi);
    }
}

template <int MODE, int NARROW, int TS, int RH, bool PF, bool NT, bool WHOLE>
__global__ __launch_bounds__(kScanThreads *RH) void lookback_scan_kernel(
    const float *__restrict__ g, const float *__restrict__ x, void *out, void *state,
    int64_t seq, int64_t ch, int n_row_tiles, int n_col_tiles,
    unsigned long long *__restrict__ incl, unsigned long long *__restrict__ aggG,
    unsigned long long *__restrict__ aggX, unsigned long long *counter,
    unsigned long long counter_base, uint32_t epoch, uint32_t *err) {
#pragma clang fp contract(off)
    constexpr int TT = TS * RH;
    // The multiplicative maps of the cumulative decay (a tile's product, the
    // carry composed during the look-back and the inclusive value published
    // for the next tile) are carried in fp64 and rounded once each; the
    // values inside a tile keep the reference's fp32 order.
    using Map = std::conditional_t<MODE == 0, double, float>;
    __shared__ long long s_tile[2];
    __shared__ Map s_ag[RH][kScanThreads];
    __shared__ Map s_incl[MODE == 0 ? kScanThreads : 1];
    __shared__ float s_ax[RH][kScanThreads];
    __shared__ float s_carry[RH][kScanThreads];
    const long long n_tiles = (long long)n_row_tiles * n_col_tiles;
    const int sub = (int)threadIdx.x / kScanThreads;
    const int lc = (int)threadIdx.x % kScanThreads;
    auto take = [&]() { return (long long)(atomicAdd(counter, 1ull) - counter_base); };

    if (threadIdx.x == 0) s_tile[0] = take();
    __syncthreads();
    long long tile = s_tile[0];
    if (tile < 0) {  // only if launches were not serialised
        if (threadIdx.x == 0) atomicOr(err, 2u);
        return;
    }
    float gv[TS], xv[TS], gn[PF ? TS : 1], xn[PF ? TS : 1];
    // tile t: row tile r, first row of this row group, this thread's channel
    auto tile_rows = [&](long long t, int64_t &row0, int64_t &c) {
        const int r = (int)(t / n_col_tiles), cb = (int)(t % n_col_tiles);
        row0 = (int64_t)r * TT + (int64_t)sub * TS;
        c = (int64_t)cb * kScanThreads + lc;
        return r;
    };
    if (tile < n_tiles) {
        int64_t row0, c;
        tile_rows(tile, row0, c);
        scan_load_rows<MODE, TS, NT, WHOLE>(g, x, seq, ch, row0, c, gv, xv);
    }
    for (int it = 0; tile < n_tiles; ++it) {
        int64_t row0, c;
        const int r = tile_rows(tile, row0, c);
        const bool live = WHOLE || c < ch;
        const int nrows = WHOLE ? TS : (int)max((int64_t)0, min((int64_t)TS, seq - row0));
        long long next = n_tiles;
        if constexpr (PF)
            if (threadIdx.x == 0) s_tile[(it + 1) & 1] = take();

        // 1. this row group's map, identity start, reference order
        {
            Map AG = 1.0f;
            float AX = 0.0f;
#pragma unroll
            for (int i = 0; i < TS; ++i) {
                if (i < nrows) {
                    if constexpr (MODE == 1) AX = xv[i] + AX * gv[i];
                    AG = AG * (Map)gv[i];
                }
            }
            s_ag[sub][lc] = AG;
            if constexpr (MODE == 1) s_ax[sub][lc] = AX;
        }
        __syncthreads();
        if constexpr (PF) {
            next = s_tile[(it + 1) & 1];
            if (next < n_tiles) {
                int64_t nrow0, nc_;
                tile_rows(next, nrow0, nc_);
                scan_load_rows<MODE, TS, NT, WHOLE>(g, x, seq, ch, nrow0, nc_, gn, xn);
            }
        }

        if (sub == 0) {
            float carry = 0.f;
            Map carry_m = 0.f;
            // the tile's map: row-group maps composed in row order
            Map AG = s_ag[0][lc];
            float AX = (MODE == 1) ? s_ax[0][lc] : 0.f;
#pragma unroll
            for (int q = 1; q < RH; ++q) {
                if constexpr (MODE == 1) AX = s_ax[q][lc] + AX * s_ag[q][lc];
                AG = AG * s_ag[q][lc];
            }
            if (r == 0) {
                if (live) carry = (MODE == 0) ? 1.0f : narrow_load<NARROW>(state, c);
                carry_m = 1.0f;
            } else if (live) {
                // 2. publish it
                const int64_t me = (int64_t)r * ch + c;
                store_status(aggG + me, pack_status(epoch, (float)AG));
                if constexpr (MODE == 1) store_status(aggX + me, pack_status(epoch, AX));
                // 3. look back
                Map GA = 1.0f;
                float XA = 0.0f;
                int p = r - 1;
                uint32_t spins = 0;
                for (;;) {
                    const int64_t at = (int64_t)p * ch + c;
                    const unsigned long long wi = load_status(incl + at);
                    if (status_tag(wi) == epoch) {
                        const float sp = status_val(wi);
                        if constexpr (MODE == 0) {
                            carry_m = GA * (Map)sp;
                            carry = (float)carry_m;
                        } else {
                            carry = GA * sp + XA;
                        }
                        break;
                    }
                    const unsigned long long wg = load_status(aggG + at);
                    const unsigned long long wx = (MODE == 1) ? load_status(aggX + at) : wg;
                    if (p > 0 && status_tag(wg) == epoch && status_tag(wx) == epoch) {
                        if constexpr (MODE == 1) XA = GA * status_val(wx) + XA;
                        GA = GA * (Map)status_val(wg);
                        --p;
                        spins = 0;
                        continue;
                    }
                    if (++spins > kSpinLimit) {
                        atomicOr(err, 1u);
                        carry = 0.f;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            s_carry[0][lc] = carry;
            if constexpr (MODE == 0) s_incl[lc] = carry_m * AG;  // this tile's inclusive value
        }

        // 4. the reference recurrence from the carry, row group by row group
        float run = 0.f;
#pragma unroll
        for (int q = 0; q < RH; ++q) {
            __syncthreads();
            if (sub == q) {
                run = s_carry[q][lc];
#pragma unroll
                for (int i = 0; i < TS; ++i) {
                    if (i < nrows) {
                        if constexpr (MODE == 1) {
                            run = xv[i] + run * gv[i];
                            xv[i] = run;
                        } else {
                            run = run * gv[i];
                            gv[i] = run;
                        }
                    }
                }
                if (q + 1 < RH) s_carry[q + 1][lc] = run;
            }
        }
        if (live && sub == RH - 1) {
            if (r + 1 < n_row_tiles) {
                float iv = run;
                if constexpr (MODE == 0) iv = (float)s_incl[lc];
                store_status(incl + (int64_t)r * ch + c, pack_status(epoch, iv));
            }
            if constexpr (MODE == 1)
                if (r == n_row_tiles - 1) narrow_store<NARROW>(state, c, run);
        }
        // Whole tiles store unpredicated: per-row predicates split the stores
        // into separate blocks and cost about 15% of the bandwidth.
        if constexpr (WHOLE) {
#pragma unroll
            for (int i = 0; i < TS; ++i) scan_store<MODE, NARROW, NT>(out, (row0 + i) * ch + c, gv[i], xv[i]);
        } else if (live) {
#pragma unroll
            for (int i = 0; i < TS; ++i)
                if (i < nrows) scan_store<MODE, NARROW, NT>(out, (row0 + i) * ch + c, gv[i], xv[i]);
        }

        if constexpr (PF) {
#pragma unroll
            for (int i = 0; i < TS; ++i) {
                gv[i] = gn[i];
                if constexpr (MODE == 1) xv[i] = xn[i];
            }
        } else {
            __syncthreads();
            if (threadIdx.x == 0) s_tile[(it + 1) & 1] = take();
            __syncthreads();
            next = s_tile[(it + 1) & 1];
            if (next < n_tiles) {
                int64_t nrow0, nc_;
                tile_rows(next, nrow0, nc_);
                scan_load_rows<MODE, TS, NT, WHOLE>(g, x, seq, ch, nrow0, nc_, gv, xv);
            }
        }
        tile = next;
    }
}

// ---------------------------------------------------------------------------
// GEMV, M = 1: c[j] = sum_k a[k] * b[k][j]
// ---------------------------------------------------------------------------
// One thread per output column, k-loop in the reference order
// (kai_gdn_gemv_f32_f32_f32_1x4_neon.c:78-86) with contraction off: the
// result is bit-identical to the portable scalar C.  Rows of b are read
// coalesced across the wavefront.
__global__ __launch_bounds__(256) void gemv_kernel(const float *__restrict__ a,
                                                   const float *__restrict__ b,
                                                   float *__restrict__ c, int64_t k,
                                                   int64_t n) {
#pragma clang fp contract(off)
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    float acc = 0.0f;
    int64_t kk = 0;
    for (; kk + 8 <= k; kk += 8) {
        float bv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) bv[i] = b[(kk + i) * n + j];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = acc + a[kk + i] * bv[i];
    }
    for (; kk < k; ++kk) acc = acc + a[kk] * b[kk * n + j];
    c[j] = acc;
}

// ---------------------------------------------------------------------------
// Delta-rule matmul: C[i][j] = sum_k A[i][k] * B[k][j]
// ---------------------------------------------------------------------------
// One thread per output element, row i = blockIdx.y (+ multiples of gridDim.y),
// k-loop in order with contraction off: the naive fp32 loop of the reference's
// test (test_gdn_delta_matmul.c:32-41) bit for bit.  Rows of B are read
// coalesced across the wavefront; A[i][k] is the same for every lane.
__global__ __launch_bounds__(256) void matmul_kernel(const float *__restrict__ A, const float *__restrict__ B,
                                                     float *__restrict__ Cm, int64_t m, int64_t k, int64_t n) {
#pragma clang fp contract(off)
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    for (int64_t i = blockIdx.y; i < m; i += gridDim.y) {
        const float *a = A + i * k;
        float acc = 0.0f;
        int64_t kk = 0;
        for (; kk + 8 <= k; kk += 8) {
            float bv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) bv[u] = B[(kk + u) * n + j];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + a[kk + u] * bv[u];
        }
        for (; kk < k; ++kk) acc = acc + a[kk] * B[kk * n + j];
        Cm[i * n + j] = acc;
    }
}

}  // namespace

// Production configuration of the streaming kernels, measured on MI355X at
// [4096][8192] with buffers rotated so every launch streams from HBM:
// non-temporal traffic and 8-row conv segments, 4096 workgroups (46.9 us;
// 64-row segments 57.1 us, cached loads 52.2 us).
constexpr bool kConvNT = true;
constexpr int64_t kConvTargetBlocks = 4096;
constexpr int64_t kConvMinSeg = 8;

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

hipError_t launch_conv_k4(const float *in, const float *w, float *out, float *hist,
                          size_t seq, size_t ch, bool silu, hipStream_t st) {
    if (seq == 0 || ch == 0) return hipSuccess;
    const uintptr_t align = (uintptr_t)in | (uintptr_t)w | (uintptr_t)out | (uintptr_t)hist;
    const bool vec4 = (ch % 4 == 0) && (align % 16 == 0);
    const int VEC = vec4 ? 4 : 1;
    const int64_t groups = (int64_t)ch / VEC;
    const int64_t bx = (groups + 255) / 256;
    // Segments: aim for >= ~4096 workgroups over the chip, at least 8 rows
    // each.  Aliased in/out keeps one segment per thread (the whole sequence),
    // which is what makes in-place operation correct.
    const bool alias = ((const char *)out < (const char *)in + seq * ch * 4) &&
                       ((const char *)in < (const char *)out + seq * ch * 4);
    int64_t seg_len = (int64_t)seq;
    if (!alias) {
        int64_t want_segs = (kConvTargetBlocks + bx - 1) / bx;
        seg_len = ((int64_t)seq + want_segs - 1) / want_segs;
        if (seg_len < kConvMinSeg) seg_len = kConvMinSeg;
        seg_len = (seg_len + 7) / 8 * 8;
        if (seg_len >= (int64_t)seq) seg_len = (int64_t)seq;
    }
    const int64_t nseg = ((int64_t)seq + seg_len - 1) / seg_len;
    dim3 grid((unsigned)bx, (unsigned)nseg), block(256);
    constexpr bool NT = kConvNT;
    if (vec4) {
        if (silu) conv_k4_kernel<4, true, NT><<<grid, block, 0, st>>>(in, w, out, hist, seq, ch, seg_len);
        else conv_k4_kernel<4, false, NT><<<grid, block, 0, st>>>(in, w, out, hist, seq, ch, seg_len);
    } else {
        if (silu) conv_k4_kernel<1, true, NT><<<grid, block, 0, st>>>(in, w, out, hist, seq, ch, seg_len);
        else conv_k4_kernel<1, false, NT><<<grid, block, 0, st>>>(in, w, out, hist, seq, ch, seg_len);
    }
    return hipGetLastError();
}

// GDN-2 gates: gp = g * b, xp = w * x, each product rounded once (the
// reference's portable branch, gdn_sve.c:861-874, rounds both before the
// scan's sum).  Four elements per thread when the arrays allow.
namespace {
template <bool VEC4>
__global__ __launch_bounds__(256) void gdn2_gates_kernel(const float *__restrict__ g, const float *__restrict__ b,
                                                         const float *__restrict__ w, const float *__restrict__ x,
                                                         float *__restrict__ gp, float *__restrict__ xp, size_t n) {
#pragma clang fp contract(off)
    const size_t stride = (size_t)gridDim.x * 256;
    if constexpr (VEC4) {
        for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n / 4; i += stride) {
            const float4 gv = reinterpret_cast<const float4 *>(g)[i], bv = reinterpret_cast<const float4 *>(b)[i];
            const float4 wv = reinterpret_cast<const float4 *>(w)[i], xv = reinterpret_cast<const float4 *>(x)[i];
            reinterpret_cast<float4 *>(gp)[i] = make_float4(gv.x * bv.x, gv.y * bv.y, gv.z * bv.z, gv.w * bv.w);
            reinterpret_cast<float4 *>(xp)[i] = make_float4(wv.x * xv.x, wv.y * xv.y, wv.z * xv.z, wv.w * xv.w);
        }
    } else {
        for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
            gp[i] = g[i] * b[i];
            xp[i] = w[i] * x[i];
        }
    }
}
}  // namespace

hipError_t launch_gdn2_gates(const float *g, const float *b, const float *w, const float *x, float *gp, float *xp,
                             size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const uintptr_t al = (uintptr_t)g | (uintptr_t)b | (uintptr_t)w | (uintptr_t)x | (uintptr_t)gp | (uintptr_t)xp;
    const bool vec4 = n % 4 == 0 && al % 16 == 0;
    const size_t work = vec4 ? n / 4 : n;
    const unsigned blocks = (unsigned)std::min<size_t>((work + 255) / 256, 8192);
    if (vec4) gdn2_gates_kernel<true><<<blocks, 256, 0, st>>>(g, b, w, x, gp, xp, n);
    else gdn2_gates_kernel<false><<<blocks, 256, 0, st>>>(g, b, w, x, gp, xp, n);
    return hipGetLastError();
}

hipError_t launch_gemv(const float *a, const float *b, float *c, size_t k, size_t n,
                       hipStream_t st) {
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    gemv_kernel<<<grid, block, 0, st>>>(a, b, c, (int64_t)k, (int64_t)n);
    return hipGetLastError();
}

hipError_t launch_matmul(const float *A, const float *B, float *Cm, size_t m, size_t k, size_t n, hipStream_t st) {
    if (m == 0 || n == 0) return hipSuccess;
    if (n > (size_t)0x7FFFFFFF * 256) return hipErrorInvalidValue;
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)std::min<size_t>(m, 65535)), block(256);
    matmul_kernel<<<grid, block, 0, st>>>(A, B, Cm, (int64_t)m, (int64_t)k, (int64_t)n);
    return hipGetLastError();
}

// Scan tiles: cumdecay 2 row groups x 64 rows, gated scan 2 x 32 (two input
// streams), both prefetching the next tile.  Measured at [4096][8192]
// cumdecay: 45.7 us (one-shot 64-row tiles without look-ahead: 59.7 us).
template <int MODE> struct ScanCfg;
template <> struct ScanCfg<0> { static constexpr int TS = kScanRowsDecay / 2, RH = 2; };
template <> struct ScanCfg<1> { static constexpr int TS = kScanRowsGated / 2, RH = 2; };
constexpr bool kScanNT = true;

template <int MODE, int NARROW, bool WHOLE>
static hipError_t launch_scan_t(const float *g, const float *x, void *out, void *state,
                                size_t seq, size_t ch, int nr, int nc, const ScanScratch &s,
                                unsigned long long base, uint32_t epoch,
                                unsigned long long *ids_used, hipStream_t st) {
    using Cfg = ScanCfg<MODE>;
    auto kern = lookback_scan_kernel<MODE, NARROW, Cfg::TS, Cfg::RH, true, kScanNT, WHOLE>;
    constexpr int threads = kScanThreads * Cfg::RH;
    // Persistent grid: as many workgroups as are resident at once.
    static int cached = -1;  // same code object on every device
    int per_cu = __atomic_load_n(&cached, __ATOMIC_RELAXED);
    if (per_cu < 0) {
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0);
        if (e != hipSuccess) return e;
        __atomic_store_n(&cached, per_cu, __ATOMIC_RELAXED);
    }
    if (per_cu < 1) return hipErrorLaunchOutOfResources;
    const long long n_tiles = (long long)nr * nc;
    const long long slots = (long long)per_cu * (s.cu_count > 0 ? s.cu_count : 1);
    const unsigned grid = (unsigned)(n_tiles < slots ? n_tiles : slots);
    kern<<<dim3(grid), dim3(threads), 0, st>>>(g, x, out, state, (int64_t)seq, (int64_t)ch, nr,
                                               nc, s.incl, s.aggG, s.aggX, s.counter, base,
                                               epoch, s.err);
    // every workgroup takes one id past the last tile before it exits
    *ids_used = (unsigned long long)n_tiles + grid;
    return hipGetLastError();
}

hipError_t launch_lookback_scan(int mode, int narrow, const float *g, const float *x, void *out,
                                void *state, size_t seq, size_t ch, const ScanScratch &scr,
                                unsigned long long counter_base, uint32_t epoch,
                                unsigned long long *ids_used, hipStream_t st) {
    *ids_used = 0;
    if (seq == 0 || ch == 0) return hipSuccess;
    if (mode != 0 && mode != 1) return hipErrorInvalidValue;
    const int nr = (int)scan_row_tiles(seq, mode);
    const int nc = (int)scan_col_tiles(ch);
    if ((size_t)nr * ch > scr.words) return hipErrorInvalidValue;
    // Shapes made of whole tiles take the unpredicated kernel.
    const bool whole = seq % scan_tile_rows(mode) == 0 && ch % kScanThreads == 0;
#define GDN_SCAN_CASE(M, N)                                                                     \
    if (mode == M && narrow == N)                                                               \
        return whole ? launch_scan_t<M, N, true>(g, x, out, state, seq, ch, nr, nc, scr,        \
                                                 counter_base, epoch, ids_used, st)             \
                     : launch_scan_t<M, N, false>(g, x, out, state, seq, ch, nr, nc, scr,       \
                                                  counter_base, epoch, ids_used, st);
    GDN_SCAN_CASE(0, kF32)
    GDN_SCAN_CASE(0, kF16)
    GDN_SCAN_CASE(0, kBF16)
    GDN_SCAN_CASE(1, kF32)
    GDN_SCAN_CASE(1, kF16)
    GDN_SCAN_CASE(1, kBF16)
#undef GDN_SCAN_CASE
    return hipErrorInvalidValue;
}

}  // namespace gdn

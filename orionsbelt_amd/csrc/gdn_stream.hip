// gdn_stream.hip -- HBM-streaming GDN kernels for gfx950:
//   causal depthwise conv1d K=4 (+ optional SiLU epilogue),
//   cumulative decay and diagonal gated scan (single-pass decoupled
//   look-back over sequence tiles), M=1 GEMV.
//
// All layouts are the reference kai layouts: [seq][channels] row-major with
// channels contiguous, so a wavefront reading one row of 64 channels issues
// one contiguous 256 B (or 1 KiB with float4) request.
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
// (channels / VEC / 256) x (seq / seg_len) blocks.  Only segment-0 threads
// touch hist: they read it first and write the new history last, so no two
// threads race on it.  FP contraction is off, making the K=4 dot product
// ((h0*w0 + h1*w1) + h2*w2) + cur*w3 bit-identical to the portable scalar C.

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
        V cur[U];
        const int n = (int)min((int64_t)U, t1 - t);
#pragma unroll
        for (int i = 0; i < U; ++i)
            if (i < n) cur[i] = vload<VEC, NT>(in + (t + i) * ch + c);
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (i < n) {
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
// s_{-1} = 1 (mode 0, kai cumdecay, kai_gdn_cumdecay_f32_sve.c:122-129).
//
// A tile is kScanTileT rows x 256 channels (one channel per thread, the tile
// held in registers).  Tiles take ids from a device counter in order, row
// tiles of a column strip in sequence order, so every tile a workgroup waits
// for was started earlier by a running workgroup and never waits on a later
// one: the wait always ends.  Per tile:
//   1. load the tile; fold it into its aggregate map s -> AG*s + AX, in the
//      reference's own order starting from the identity;
//   2. publish the aggregate (row tile > 0);
//   3. look back over predecessor tiles, composing aggregates until one
//      publishes its inclusive state;
//   4. re-run the reference recurrence over the tile from that carry,
//      publish the inclusive state, store the tile.
// Only the carry into a tile is re-associated; inside a tile the arithmetic
// is the reference's, and row tile 0 is bit-identical to it.
// Status words are 64-bit: (epoch << 32) | float bits.  A word belongs to
// the current launch iff its tag equals `epoch`, so each word validates
// itself and no fences are needed; the arrays are never cleared between
// launches.  The wait is bounded: past spin_limit polls the tile records an
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

template <int MODE, int NARROW, int TT, bool NT>
__global__ __launch_bounds__(kScanThreads) void lookback_scan_kernel(
    const float *__restrict__ g, const float *__restrict__ x, void *out, void *state,
    int64_t seq, int64_t ch, int n_row_tiles, int n_col_tiles,
    unsigned long long *__restrict__ incl, unsigned long long *__restrict__ aggG,
    unsigned long long *__restrict__ aggX, unsigned long long *counter,
    unsigned long long counter_base, uint32_t epoch, uint32_t *err) {
#pragma clang fp contract(off)
    __shared__ long long s_tile;
    if (threadIdx.x == 0) s_tile = (long long)(atomicAdd(counter, 1ull) - counter_base);
    __syncthreads();
    const long long tile = s_tile;
    const long long n_tiles = (long long)n_row_tiles * n_col_tiles;
    if (tile < 0 || tile >= n_tiles) {  // only if launches were not serialised
        if (threadIdx.x == 0) atomicOr(err, 2u);
        return;
    }
    const int r = (int)(tile / n_col_tiles);
    const int cb = (int)(tile % n_col_tiles);
    const int64_t c = (int64_t)cb * kScanThreads + threadIdx.x;
    const bool live = c < ch;
    const int64_t t0 = (int64_t)r * TT;
    const int nt = (int)min((int64_t)TT, seq - t0);

    float gv[TT], xv[TT];
#pragma unroll
    for (int i = 0; i < TT; ++i) {
        if (live && i < nt) {
            if constexpr (NT) {
                gv[i] = __builtin_nontemporal_load(g + (t0 + i) * ch + c);
                if constexpr (MODE == 1) xv[i] = __builtin_nontemporal_load(x + (t0 + i) * ch + c);
            } else {
                gv[i] = g[(t0 + i) * ch + c];
                if constexpr (MODE == 1) xv[i] = x[(t0 + i) * ch + c];
            }
        }
    }

    float carry = 0.f;
    if (r == 0) {
        if (live) carry = (MODE == 0) ? 1.0f : narrow_load<NARROW>(state, c);
    } else if (live) {
        // 1. aggregate of this tile, identity start, reference order
        float AG = 1.0f, AX = 0.0f;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            if (i < nt) {
                if constexpr (MODE == 1) AX = xv[i] + AX * gv[i];
                AG = AG * gv[i];
            }
        }
        // 2. publish it
        const int64_t me = (int64_t)r * ch + c;
        store_status(aggG + me, pack_status(epoch, AG));
        if constexpr (MODE == 1) store_status(aggX + me, pack_status(epoch, AX));
        // 3. look back
        float GA = 1.0f, XA = 0.0f;
        int p = r - 1;
        uint32_t spins = 0;
        for (;;) {
            const int64_t at = (int64_t)p * ch + c;
            const unsigned long long wi = load_status(incl + at);
            if (status_tag(wi) == epoch) {
                const float sp = status_val(wi);
                carry = (MODE == 0) ? GA * sp : GA * sp + XA;
                break;
            }
            const unsigned long long wg = load_status(aggG + at);
            const unsigned long long wx = (MODE == 1) ? load_status(aggX + at) : wg;
            if (p > 0 && status_tag(wg) == epoch && status_tag(wx) == epoch) {
                if constexpr (MODE == 1) XA = GA * status_val(wx) + XA;
                GA = GA * status_val(wg);
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

    // 4. the reference recurrence from the carry, in registers
    float run = carry;
#pragma unroll
    for (int i = 0; i < TT; ++i) {
        if (i < nt) {
            if constexpr (MODE == 1) {
                run = xv[i] + run * gv[i];
                xv[i] = run;
            } else {
                run = run * gv[i];
                gv[i] = run;
            }
        }
    }
    if (live) {
        if (r + 1 < n_row_tiles) store_status(incl + (int64_t)r * ch + c, pack_status(epoch, run));
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            if (i < nt) {
                float *o32 = static_cast<float *>(out) + (t0 + i) * ch + c;
                if constexpr (MODE == 1) {
                    if constexpr (NT) __builtin_nontemporal_store(xv[i], o32);
                    else *o32 = xv[i];
                } else if constexpr (NARROW == kF32 && NT) {
                    __builtin_nontemporal_store(gv[i], o32);
                } else {
                    narrow_store<NARROW>(out, (t0 + i) * ch + c, gv[i]);
                }
            }
        }
        if constexpr (MODE == 1)
            if (r == n_row_tiles - 1) narrow_store<NARROW>(state, c, run);
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

}  // namespace

// Production configuration of the streaming kernels, measured on MI355X at
// [4096][8192] with buffers rotated so every launch streams from HBM:
// non-temporal traffic and 64-row conv segments (55.4 us vs 59.7 us cached
// with 32-row segments); 64-row scan tiles (59.4 us; 32 rows: 76 us).
constexpr bool kConvNT = true;
constexpr int64_t kConvTargetBlocks = 4096;
constexpr int64_t kConvMinSeg = 64;
constexpr bool kScanNT = true;

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

hipError_t launch_gemv(const float *a, const float *b, float *c, size_t k, size_t n,
                       hipStream_t st) {
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
    gemv_kernel<<<grid, block, 0, st>>>(a, b, c, (int64_t)k, (int64_t)n);
    return hipGetLastError();
}

template <int MODE, int NARROW, int TT = kScanTileT, bool NT = kScanNT>
static void launch_scan_t(const float *g, const float *x, void *out, void *state, size_t seq,
                          size_t ch, int nr, int nc, const ScanScratch &s,
                          unsigned long long base, uint32_t epoch, hipStream_t st) {
    dim3 grid((unsigned)((size_t)nr * nc)), block(kScanThreads);
    lookback_scan_kernel<MODE, NARROW, TT, NT><<<grid, block, 0, st>>>(
        g, x, out, state, (int64_t)seq, (int64_t)ch, nr, nc, s.incl, s.aggG, s.aggX, s.counter,
        base, epoch, s.err);
}

hipError_t launch_lookback_scan(int mode, int narrow, const float *g, const float *x, void *out,
                                void *state, size_t seq, size_t ch, const ScanScratch &scr,
                                unsigned long long counter_base, uint32_t epoch,
                                hipStream_t st) {
    if (seq == 0 || ch == 0) return hipSuccess;
    const int nr = (int)scan_row_tiles(seq);
    const int nc = (int)scan_col_tiles(ch);
    if ((size_t)nr * ch > scr.words) return hipErrorInvalidValue;
#define GDN_SCAN_CASE(M, N)                                                                  \
    if (mode == M && narrow == N) {                                                          \
        launch_scan_t<M, N>(g, x, out, state, seq, ch, nr, nc, scr, counter_base, epoch, st); \
        return hipGetLastError();                                                            \
    }
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

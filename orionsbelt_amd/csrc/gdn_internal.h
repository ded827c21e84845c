// gdn_internal.h -- launchers shared between the kernel files and the C-ABI
// layer (kai_shim.hip).  Not installed; callers use include/kai_gdn_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gdn {

// Narrow storage formats of the mixed-precision variants.
enum Narrow : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// ---- streaming kernels (gdn_stream.hip) ------------------------------------

hipError_t launch_conv_k4(const float *in, const float *w, float *out, float *hist,
                          size_t seq, size_t ch, bool silu, hipStream_t st);

hipError_t launch_matmul(const float *A, const float *B, float *Cm, size_t m, size_t k, size_t n, hipStream_t st);
hipError_t launch_gemv(const float *a, const float *b, float *c, size_t k, size_t n,
                       hipStream_t st);

// GDN-2 gates for the gated scan: gp = g * b, xp = w * x (n elements).
hipError_t launch_gdn2_gates(const float *g, const float *b, const float *w, const float *x, float *gp, float *xp,
                             size_t n, hipStream_t st);

// Scratch of the decoupled look-back scan: a monotonically increasing tile
// counter, three status arrays of n_row_tiles * channels 64-bit words and an
// error word.  Owned per device by the C-ABI layer, which serialises scan
// launches and advances `counter_base` and `epoch` itself.
struct ScanScratch {
    unsigned long long *counter;
    unsigned long long *incl;
    unsigned long long *aggG;
    unsigned long long *aggX;
    uint32_t *err;
    size_t words;   // capacity of each status array
    int cu_count;   // compute units of the device (sizes the persistent grid)
};

constexpr int kScanThreads = 256;   // channels per tile (one per thread of a row group)
// Rows per tile: cumulative decay (one input stream) and gated scan (two).
constexpr int kScanRowsDecay = 128;
constexpr int kScanRowsGated = 64;

inline size_t scan_tile_rows(int mode) { return mode == 0 ? kScanRowsDecay : kScanRowsGated; }
inline size_t scan_row_tiles(size_t seq, int mode) {
    return (seq + scan_tile_rows(mode) - 1) / scan_tile_rows(mode);
}
inline size_t scan_col_tiles(size_t ch) { return (ch + kScanThreads - 1) / kScanThreads; }

// mode 0: cumdecay (out = prefix product of g; `narrow` applies to out)
// mode 1: gated scan (s fp32; `narrow` applies to state)
// On success *ids_used is the number of tile ids the launch takes from the
// counter (the caller's next counter_base is counter_base + *ids_used).
hipError_t launch_lookback_scan(int mode, int narrow, const float *g, const float *x,
                                void *out, void *state, size_t seq, size_t ch,
                                const ScanScratch &scr, unsigned long long counter_base,
                                uint32_t epoch, unsigned long long *ids_used,
                                hipStream_t st);

// ---- decode (gdn_decode.hip) ------------------------------------------------

hipError_t launch_delta_decode(int narrow_state, void *S, const float *q, const float *k,
                               const float *v, const float *g, const float *beta, float *o,
                               int B, int Hv, int Hk, int dk, int dv, float q_scale,
                               hipStream_t st);

// One GDN layer's decode step after the in-projection, fused (d = 128, fp32
// state): conv update + SiLU on HF's cache, q/k L2 norm, gates, the delta
// rule, and the gated RMSNorm rounded to fp16 into out16 [B][Hv * 128].
// x [B][(2 Hk + Hv) * 128] (the in-projection's qkv rows); the conv cache
// [B][(2 Hk + Hv) * 128][4] is read from conv_in and written shifted to
// conv_out (distinct arrays); a, b [B][Hv], S [B][Hv][128][128], z [B][Hv][128].
hipError_t launch_gdn_step_fused(const float *x, const float *conv_in, float *conv_out, const float *conv_w,
                                 const float *a, const float *b, const float *A_log, const float *dt_bias, float *S,
                                 const float *z, const float *norm_w, uint16_t *out16, int B, int Hk, int Hv,
                                 float q_scale, float eps, hipStream_t st);

// ---- chunked prefill (gdn_prefill.hip) --------------------------------------

constexpr int kChunk = 64;
constexpr int kHeadDim = 128;

// Chunkwise prefill, parallel over the sequence.  `carry` holds
// prefill_carry_bytes(B, T, Hv) bytes of device memory (segment transitions
// and start states); calls that share it must not overlap.
size_t prefill_carry_bytes(int B, int T, int Hv);
// (sequence, head) pairs of the last call that ran windowed (synchronises).
int prefill_windowed_heads();
hipError_t launch_prefill_seq(int narrow_state, const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, const float *g, const float *beta, uint16_t *o,
                              void *S, int B, int T, int Hv, int Hk, float q_scale, void *carry,
                              hipStream_t st);

// ---- layer glue (gdn_layer.hip) ---------------------------------------------

// Gating prologue: conv output x [rows][(2 Hk + Hv) * 128] -> q, k (L2-normalised)
// [rows][Hk][128], v [rows][Hv][128] (bf16 bit patterns or fp32), g, beta [rows][Hv].
// The prefill's causal conv (K = 4, SiLU; tap-major weights conv_wt [4][C],
// the three previous inputs in hist [3][C]) fused with the gating prologue
// into bf16 q, k, v and fp32 g, beta: bit for bit launch_conv_k4 followed by
// launch_gating_prologue, without the conv's output array.
hipError_t launch_conv_gating(const float *x, const float *conv_wt, const float *hist, const float *a,
                              const float *b, const float *A_log, const float *dt_bias, uint16_t *q, uint16_t *k,
                              uint16_t *v, float *g, float *beta, int64_t T, int Hk, int Hv, hipStream_t st);
hipError_t launch_gating_prologue(bool bf16, const float *x, const float *a, const float *b,
                                  const float *A_log, const float *dt_bias, void *q, void *k,
                                  void *v, float *g, float *beta, size_t rows, int Hk, int Hv,
                                  hipStream_t st);
// Gated RMSNorm over rows of 128 values (bf16 bit patterns or fp32).
hipError_t launch_gated_rmsnorm(bool bf16, const void *o, const void *z, const void *w, void *y,
                                size_t rows, float eps, hipStream_t st);

// ---- state hand-off formats and the decode-step conv (gdn_state.hip) -------

// HF causal_conv1d_update on x, out [B][T][C], conv_state [B][C][4], w [C][4].
hipError_t launch_conv_update(const float *x, float *conv_state, const float *w, float *out, int B,
                              int T, size_t C, bool silu, hipStream_t st);
// conv_state [B][C][4] from the last four rows of x [B][T][C] (zero-padded).
hipError_t launch_conv_state_from_inputs(const float *x, float *conv_state, int B, size_t T, size_t C,
                                         hipStream_t st);
// hist [B][3][C] <-> conv_state [B][C][4].
hipError_t launch_conv_hist_state(bool to_hist, float *hist, float *conv_state, int B, size_t C,
                                  hipStream_t st);
// Element conversion between kF32, kF16 and kBF16 arrays.
hipError_t launch_convert(const void *src, int sf, void *dst, int df, size_t n, hipStream_t st);

// ---- hybrid decode loop matmuls (gdn_model.hip) ------------------------------

// y[M][N] fp32 = scale[N] * (x[M][K] fp16 . Wq[N][K]^T int8), M <= 16,
// N % 16 == 0, K % 256 == 0; `workspace` holds w8_workspace_bytes(M, N, K).
int w8_splits(int N, int K);
size_t w8_workspace_bytes(int M, int N, int K);
hipError_t launch_w8_gemm(const uint16_t *x, const int8_t *W, const float *scale, float *y, int M,
                          int N, int K, float *workspace, hipStream_t st);
// The model's fused int8 GEMM (rows of several matrices that share the input
// concatenated), weights pre-tiled by launch_w8f_tile from row-major [N][K]:
// N % 64 == 0, M <= 16, K a multiple of splits * waves * depth * 64.  Output
// by `out`: kW8Segments writes channel ranges [seg[q-1].n_end, seg[q].n_end)
// (16-multiples) to seg[q].dst with row stride seg[q].ld (channels past the
// last segment are padding and not stored); kW8SwiGLU reads the rows as
// gate/up interleaved in groups of 8 and writes x16 [M][N / 2] fp16.  With
// splits > 1, `part` holds w8f_workspace_floats(M, N, K) floats and `cnt`
// N / 64 counters that are zero before the first launch (each launch leaves
// them zero); launches sharing them must not overlap.
enum W8Mode : int { kW8Segments = 0, kW8SwiGLU = 1 };
constexpr int kW8MaxSegs = 4;
struct W8Seg {
    float *dst;
    int ld;
    int n_end;
};
struct W8Out {
    W8Seg seg[kW8MaxSegs];
    int nseg;
    int mode;
    uint16_t *x16;
    // Normalised input (the decode GEMM, M <= kW8NormInRows, K <= kW8NormInMaxK):
    // with nin_h set, the matrix's input is fp16(rmsnorm(h') * (1 + nin_w))
    // with h' = nin_h + nin_add (nin_add may be null), formed by every block
    // in LDS with the residual norm's arithmetic; the block of the first
    // channel group writes h' to nin_hout (when set).  x is then unused.
    const float *nin_h;
    const float *nin_add;
    float *nin_hout;
    const float *nin_w;
    float nin_eps;
    // Residual add in the epilogue (kW8Segments with one segment):
    // seg[0].dst[m][n] = add_in[m * add_ld + n] + y[m][n].
    const float *add_in;
    int add_ld;
};
constexpr int kW8NormInRows = 1;
constexpr int kW8NormInMaxK = 4096;
// Launch shape: waves per block (4 or 8), 64-k steps in flight per wave (1,
// 2 or 4), k-splits across blocks (0: chosen by w8f_shape).
struct W8fShape {
    int waves, depth, splits;
};
W8fShape w8f_shape(int N, int K);
size_t w8f_workspace_floats(int M, int N, int K);
hipError_t launch_w8f_tile(const int8_t *src, int8_t *dst, int N, int K, hipStream_t st);
hipError_t launch_w8f(const uint16_t *x, const int8_t *W, const float *scale, int M, int N, int K,
                      const W8Out &out, float *part, uint32_t *cnt, hipStream_t st,
                      W8fShape shape = W8fShape{0, 0, 0});
// Per-output-channel symmetric int8 quantisation of W[N][K] fp32.
hipError_t launch_w8_quantize(const float *W, int8_t *Wq, float *scale, int N, int K, hipStream_t st);

// ---- hybrid model prefill (gdn_prefill_model.hip) ---------------------------

// The model's int8 GEMM for many rows: x [M][ldx] fp16 (16-byte aligned
// rows), weights tiled by launch_w8f_tile (N % 64 == 0, K % 64 == 0); `out`
// as for launch_w8f in kW8Segments or kW8SwiGLU mode.
// The largest M launch_w8p accepts (its grid's y limit).
long long w8p_max_rows();
hipError_t launch_w8p(const uint16_t *x, int ldx, const int8_t *W, const float *scale, int M, int N, int K,
                      const W8Out &out, hipStream_t st);
// Causal attention of one sequence's T positions: q16 [T][Hq][256] fp16,
// Kc [Hkv][Tmax][256] tiled by 16 positions (kv_tiled_offset), vT
// [Hkv][256][Tv] fp16 (V transposed; Tv % 64 == 0, Tv >= T, finite past T),
// gate rows [T] of gate_row floats (head h's gate at h * 512 + d);
// out16 [T][Hq][256] = fp16(softmax(q k^T * scaling) v * sigmoid(gate)).
hipError_t launch_attn_prefill(const uint16_t *q16, const uint16_t *Kc, const uint16_t *vT, const float *gate,
                               int gate_row, uint16_t *out16, int T, int Hq, int Hkv, int Tmax, int Tv,
                               float scaling, hipStream_t st);
// Attention decode over an fp16 KV cache (head_dim 256, Hq / Hkv <= 4):
// out [B][Hq][256] fp32; `workspace` holds attn_workspace_bytes(B, Hq, L),
// or attn_workspace_bytes_tiled(B, Hq, L) for a k_tiled launch (whose
// spans shrink to as few as 64 positions when the grid is small).
// With `gate` (non-null), the output is instead out16 [B][Hq][256] fp16 =
// fp16(o * sigmoid(gate[(b * Hq + h) * gate_stride + d])).
// k_tiled: K is stored tiled by 16 positions (Tmax % 16 == 0), element
// (t, d) of a (sequence, kv head) at kv_tiled_offset(t, d); V stays
// row-major.
size_t attn_workspace_bytes(int B, int Hq, int L);
size_t attn_workspace_bytes_tiled(int B, int Hq, int L);  // the k_tiled launches' (shorter spans allowed)
hipError_t launch_attn_decode(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, float *out,
                              int B, int Hq, int Hkv, int Tmax, int L, float scaling, float *workspace,
                              hipStream_t st, const float *gate = nullptr, int gate_stride = 0,
                              uint16_t *out16 = nullptr, bool k_tiled = false);
// Offset (in halfs, from the row of position 0) of K[t][d] in the tiled
// layout: group t / 16 holds 8 x 512 halfs; chunk j (dims 32 j .. 32 j + 31)
// holds lane (g, r) = (d / 8 % 4, t % 16)'s 8 dims at lane * 8.
__host__ __device__ inline size_t kv_tiled_offset(int t, int d) {
    return (size_t)(t & ~15) * 256 + (size_t)(d >> 5) * 512 + (size_t)(((d >> 3) & 3) * 16 + (t & 15)) * 8 + (d & 7);
}

// ---- measurement probes (gdn_probe.hip) -----------------------------------

size_t probe_sink_words(int cu_count);
hipError_t launch_probe_stream(const void *src, void *dst, size_t bytes, int mode, uint32_t *sink, int cu_count,
                               hipStream_t st);
hipError_t launch_probe_mfma(float *sink, int iters, int shape, int cu_count, unsigned long long *flops,
                             hipStream_t st);

}  // namespace gdn

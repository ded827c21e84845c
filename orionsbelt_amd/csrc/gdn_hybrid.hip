// gdn_hybrid.hip -- the end-to-end hybrid decode loop (include/kai_gdn_hybrid.h)
// for gfx950: model construction, drawn states, and one decode step as a
// sequence of this library's kernels on one stream.
//
// Per step, batch B, residual stream h [B][hidden] fp32:
//   h = embed(tokens)
//   per layer: x = rmsnorm(h) fp16; mixer(x) -> d; h += d; x = rmsnorm(h);
//              h += down(silu(gate(x)) * up(x))
//     GDN mixer: in_proj_qkv/z/b/a (int8 GEMM) -> conv update on HF's cache
//                -> gating prologue -> delta-rule decode step (fp32 state)
//                -> gated RMSNorm with z -> out_proj
//     attention: q_proj (q and output gate per head), k_proj, v_proj ->
//                q/k RMSNorm, partial rotary embedding, KV append -> decode
//                attention over the cache -> o * sigmoid(gate) -> o_proj
//   logits = lm_head(rmsnorm(h)), next = argmax
// The residual add is fused into the following RMSNorm, the projections that
// share an input are one int8 GEMM launch (qkv|z|b|a; q|k|v; gate|up with
// the SiLU product in its epilogue), and the output gate is applied in the
// attention's span combine.  Everything a matmul reads is fp16 (the model's
// activation dtype), everything it writes fp32 (the MLP activation fp16).
#include <algorithm>
#include <cmath>
#include <initializer_list>
#include <new>
#include <vector>

#include "gdn_common.h"
#include "gdn_internal.h"
#include "../../include/kai_gdn_hip.h"
#include "../../include/kai_gdn_hybrid.h"

namespace gdn {
namespace {

#define GDN_HD __host__ __device__ __forceinline__

// ---- drawn values: counter-based hash, identical on host and device --------
GDN_HD uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// (2u - 1) * amp + center, u in [0, 1) from 24 hash bits; the arithmetic
// is exact up to the final product and sum (no contraction).
GDN_HD float hash_value(uint64_t seed, uint64_t stream, uint64_t i, float amp, float center) {
#pragma clang fp contract(off)
    const uint64_t h = mix64(mix64(seed ^ (stream * 0x100000001B3ull)) + i);
    const float u = (float)(h >> 40) * (1.0f / 16777216.0f);
    return (u * 2.0f - 1.0f) * amp + center;
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float *dst, size_t n, uint64_t seed,
                                                       uint64_t stream, float amp, float center) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = hash_value(seed, stream, i, amp, center);
}
__global__ __launch_bounds__(256) void fill_f16_kernel(uint16_t *dst, size_t n, uint64_t seed,
                                                       uint64_t stream, float amp, float center) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        dst[i] = f32_to_f16_rne(hash_value(seed, stream, i, amp, center));
}
// K/V cache rows [rows][Tmax][256] (storage Tmax >= the logical length
// Tlog), positions < len drawn, the rest zero.  The value of (row, t, d) is
// the hash of its row-major index with Tlog positions per row (the CPU
// model's layout); with TILED the element is stored at its tiled place
// (kv_tiled_offset).
template <bool TILED>
__global__ __launch_bounds__(256) void fill_cache_kernel(uint16_t *dst, size_t rows, int Tmax, int Tlog, int len,
                                                         uint64_t seed, uint64_t stream, float amp) {
    const size_t n = rows * (size_t)Tmax * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t row = i / ((size_t)Tmax * 256);
        const int t = (int)((i / 256) % Tmax), d = (int)(i % 256);
        const size_t li = (row * Tlog + t) * 256 + d;
        const uint16_t v = t < len ? f32_to_f16_rne(hash_value(seed, stream, li, amp, 0.f)) : 0;
        dst[row * Tmax * 256 + (TILED ? kv_tiled_offset(t, d) : (size_t)t * 256 + d)] = v;
    }
}
unsigned fill_blocks(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 8192); }

// ---- step kernels ------------------------------------------------------------

GDN_DEV float block_sum(float x, float *red) {  // 256 threads
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

// h[b] = embed[token[b]] (token ids clamped into the vocabulary).
__global__ __launch_bounds__(256) void embed_kernel(const int32_t *tokens, const uint16_t *table,
                                                    float *h, int H, int vocab) {
    const int b = blockIdx.x;
    const int t = min(max(tokens[b], 0), vocab - 1);
    for (int i = threadIdx.x; i < H; i += 256) h[(size_t)b * H + i] = f16_to_f32(table[(size_t)t * H + i]);
}

// Qwen3_5RMSNorm (modeling_qwen3_5.py:720-737) with the residual add fused:
// h += d (when d), out = fp16(h / sqrt(mean(h^2) + eps) * (1 + w)).  One
// block per row; thread t holds the float4 chunks t, t + 256, ... (H / 4 <=
// 256 kNormChunks), all loaded before any arithmetic.
constexpr int kNormChunks = 8;
__global__ __launch_bounds__(256) void addnorm_kernel(float *__restrict__ h, const float *__restrict__ d,
                                                      const float *__restrict__ w, uint16_t *__restrict__ out,
                                                      int H, float eps) {
    __shared__ float red[4];
    const size_t b = blockIdx.x;
    float4 *hr = reinterpret_cast<float4 *>(h + b * H);
    const int n4 = H / 4;
    float4 x[kNormChunks], dv[kNormChunks];
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            x[j] = hr[i];
            if (d) dv[j] = reinterpret_cast<const float4 *>(d + b * H)[i];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            if (d) {
                x[j].x += dv[j].x;
                x[j].y += dv[j].y;
                x[j].z += dv[j].z;
                x[j].w += dv[j].w;
                hr[i] = x[j];
            }
            ss += x[j].x * x[j].x + x[j].y * x[j].y + x[j].z * x[j].z + x[j].w * x[j].w;
        }
    }
    const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
    for (int j = 0; j < kNormChunks; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            const float4 wv = reinterpret_cast<const float4 *>(w)[i];
            uint2 o;
            o.x = (uint32_t)f32_to_f16_rne(x[j].x * inv * (1.0f + wv.x)) |
                  ((uint32_t)f32_to_f16_rne(x[j].y * inv * (1.0f + wv.y)) << 16);
            o.y = (uint32_t)f32_to_f16_rne(x[j].z * inv * (1.0f + wv.z)) |
                  ((uint32_t)f32_to_f16_rne(x[j].w * inv * (1.0f + wv.w)) << 16);
            reinterpret_cast<uint2 *>(out + b * H)[i] = o;
        }
    }
}

// Attention prologue (Qwen3_5Attention.forward:656-681): block (slot, row),
// 256 threads = the head's dims.  Slots [0, Hq): query heads from qg
// [rows][Hq][512] (q = dims 0..255, gate = 256..511) -> q_norm -> rotary ->
// q16 [rows][Hq][256]; [Hq, Hq + Hkv): key heads -> k_norm -> rotary -> K
// cache; [Hq + Hkv, Hq + 2 Hkv): value heads -> V cache (and, with vT, the
// transposed copy vT [Hkv][256][Tv] that the prefill attention reads).
// Norm outputs are rounded to fp16 (type_as) before the rotary embedding,
// which acts on dims 0..63 with inv_freq[i] = 1 / theta^(2i / 64) and
// rotate_half.  Decode (seq < 0): row b is sequence b at position pos.
// Prefill (seq >= 0): row t is position t of sequence seq.
__global__ __launch_bounds__(256) void attn_prologue_kernel(
    const float *qg, const float *kx, const float *vx, const float *q_norm, const float *k_norm,
    uint16_t *q16, uint16_t *Kc, uint16_t *Vc, int Hq, int Hkv, int Tmax, int seq, int pos, float theta,
    float eps, uint16_t *vT, int Tv) {
    __shared__ float red[4];
    __shared__ float rot[64];
    // rows on grid x (a prefill's T can exceed grid y's 65535), heads on y
    const int slot = blockIdx.y, row = blockIdx.x, d = threadIdx.x;
    const int b = seq < 0 ? row : seq;
    const int p = seq < 0 ? pos : row;
    if (slot >= Hq + Hkv) {  // value head: copy into the cache
        const int kv = slot - Hq - Hkv;
        const uint16_t v = f32_to_f16_rne(vx[((size_t)row * Hkv + kv) * 256 + d]);
        Vc[(((size_t)b * Hkv + kv) * Tmax + p) * 256 + d] = v;
        if (vT) vT[((size_t)kv * 256 + d) * Tv + p] = v;
        return;
    }
    const bool is_q = slot < Hq;
    const float x = is_q ? qg[((size_t)row * Hq + slot) * 512 + d] : kx[((size_t)row * Hkv + (slot - Hq)) * 256 + d];
    const float *wn = is_q ? q_norm : k_norm;
    const float inv = 1.0f / sqrtf(block_sum(x * x, red) / 256.0f + eps);
    const float xn = f16_to_f32(f32_to_f16_rne(x * inv * (1.0f + wn[d])));
    float y = xn;
    if (d < 64) rot[d] = xn;
    __syncthreads();
    if (d < 64) {
        const int i = d & 31;
        const float inv_freq = 1.0f / powf(theta, (float)(2 * i) / 64.0f);
        const float f = inv_freq * (float)p;
        const float c = cosf(f), s = sinf(f);
        y = d < 32 ? xn * c - rot[d + 32] * s : xn * c + rot[d - 32] * s;
    }
    const uint16_t o = f32_to_f16_rne(y);
    if (is_q) q16[((size_t)row * Hq + slot) * 256 + d] = o;
    else Kc[((size_t)b * Hkv + (slot - Hq)) * Tmax * 256 + kv_tiled_offset(p, d)] = o;  // K is tiled
}

// The attention prologue of a prefill, eight rows per wave: block (32 rows,
// slot), 4 waves.  Lane l holds dims l + 64 c (c = 0..3) of a row, so each
// norm sums as block_sum does (one butterfly per 64 dims, then (s0 + s1) +
// (s2 + s3)) and the per-element arithmetic is attn_prologue_kernel's; a
// wave keeps its rows' loads in flight together (one row per 256-thread
// block left every block waiting on one load), and the transposed V copy
// takes 8 positions of a dim per 16-byte store.  Row t is position t of
// sequence seq; V^T positions past T in the last group are written as 0.
constexpr int kApRows = 8;
__global__ __launch_bounds__(256) void attn_prologue_rows_kernel(
    const float *__restrict__ qg, const float *__restrict__ kx, const float *__restrict__ vx,
    const float *__restrict__ q_norm, const float *__restrict__ k_norm, uint16_t *__restrict__ q16,
    uint16_t *__restrict__ Kc, uint16_t *__restrict__ Vc, int Hq, int Hkv, int Tmax, int T, int seq, float theta,
    float eps, uint16_t *__restrict__ vT, int Tv) {
    const int slot = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = ((int)blockIdx.x * 4 + wave) * kApRows;
    if (r0 >= T) return;  // the whole wave
    const int nr = min(kApRows, T - r0);
    if (slot >= Hq + Hkv) {  // value head: the cache, and the transposed copy
        const int kv = slot - Hq - Hkv;
        uint16_t v[kApRows][4];
#pragma unroll
        for (int j = 0; j < kApRows; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                v[j][c] = j < nr ? f32_to_f16_rne(vx[((size_t)(r0 + j) * Hkv + kv) * 256 + 64 * c + lane]) : 0;
#pragma unroll
        for (int j = 0; j < kApRows; ++j)
            if (j < nr)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    Vc[(((size_t)seq * Hkv + kv) * Tmax + r0 + j) * 256 + 64 * c + lane] = v[j][c];
        if (vT) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint4 w;
                w.x = (uint32_t)v[0][c] | ((uint32_t)v[1][c] << 16);
                w.y = (uint32_t)v[2][c] | ((uint32_t)v[3][c] << 16);
                w.z = (uint32_t)v[4][c] | ((uint32_t)v[5][c] << 16);
                w.w = (uint32_t)v[6][c] | ((uint32_t)v[7][c] << 16);
                *reinterpret_cast<uint4 *>(vT + ((size_t)kv * 256 + 64 * c + lane) * Tv + r0) = w;
            }
        }
        return;
    }
    const bool is_q = slot < Hq;
    const float *wn = is_q ? q_norm : k_norm;
    float w1[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) w1[c] = 1.0f + wn[64 * c + lane];
    float x[kApRows][4];
#pragma unroll
    for (int j = 0; j < kApRows; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            x[j][c] = j >= nr ? 0.f
                      : is_q ? qg[((size_t)(r0 + j) * Hq + slot) * 512 + 64 * c + lane]
                             : kx[((size_t)(r0 + j) * Hkv + (slot - Hq)) * 256 + 64 * c + lane];
    // rotary frequency of dim lane (< 64): rotate_half pairs it with lane ^ 32
    const float inv_freq = 1.0f / powf(theta, (float)(2 * (lane & 31)) / 64.0f);
#pragma unroll
    for (int j = 0; j < kApRows; ++j) {
        if (j >= nr) break;
        float r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float xx = x[j][c] * x[j][c];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) xx += __shfl_xor(xx, o);
            r[c] = xx;
        }
        const float inv = 1.0f / sqrtf(((r[0] + r[1]) + (r[2] + r[3])) / 256.0f + eps);
        float y[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = f16_to_f32(f32_to_f16_rne(x[j][c] * inv * w1[c]));
        const int p = r0 + j;
        const float f = inv_freq * (float)p;
        const float cs = cosf(f), sn = sinf(f);
        const float other = __shfl_xor(y[0], 32);
        y[0] = lane < 32 ? y[0] * cs - other * sn : y[0] * cs + other * sn;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint16_t o = f32_to_f16_rne(y[c]);
            const int d = 64 * c + lane;
            if (is_q) q16[((size_t)p * Hq + slot) * 256 + d] = o;
            else Kc[((size_t)seq * Hkv + (slot - Hq)) * Tmax * 256 + kv_tiled_offset(p, d)] = o;
        }
    }
}

// The GDN output's gated RMSNorm for the prefill (the decode step's
// step 4 in gdn_step_fused_kernel, on the prefill's bf16 output): rows of
// 128, o bf16 [rows][128], z fp32 [rows][128] -> out16 fp16 =
// w * (o / sqrt(mean(o^2) + eps)) * silu(z).  32 lanes per row, 4 values
// each; 8 rows per block.
__global__ __launch_bounds__(256) void prefill_gated_norm_kernel(const uint16_t *__restrict__ o,
                                                                 const float *__restrict__ z,
                                                                 const float *__restrict__ w,
                                                                 uint16_t *__restrict__ out16, size_t rows,
                                                                 float eps) {
#pragma clang fp contract(off)
    const size_t row = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int c = (threadIdx.x & 31) * 4;
    if (row >= rows) return;  // whole 32-lane groups leave together
    const uint2 ob = *reinterpret_cast<const uint2 *>(o + row * 128 + c);
    const float4 o4 = make_float4(bf16_to_f32((uint16_t)(ob.x & 0xFFFF)), bf16_to_f32((uint16_t)(ob.x >> 16)),
                                  bf16_to_f32((uint16_t)(ob.y & 0xFFFF)), bf16_to_f32((uint16_t)(ob.y >> 16)));
    float q2 = o4.x * o4.x + o4.y * o4.y + o4.z * o4.z + o4.w * o4.w;
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) q2 += __shfl_xor(q2, s, 32);
    const float inv = 1.0f / sqrtf(q2 / 128.0f + eps);
    const float4 zz = *reinterpret_cast<const float4 *>(z + row * 128 + c);
    const float4 ww = *reinterpret_cast<const float4 *>(w + c);
    auto gn = [&](float ov, float zv, float wv) { return (wv * (ov * inv)) * (zv / (1.0f + expf(-zv))); };
    uint2 r;
    r.x = (uint32_t)f32_to_f16_rne(gn(o4.x, zz.x, ww.x)) | ((uint32_t)f32_to_f16_rne(gn(o4.y, zz.y, ww.y)) << 16);
    r.y = (uint32_t)f32_to_f16_rne(gn(o4.z, zz.z, ww.z)) | ((uint32_t)f32_to_f16_rne(gn(o4.w, zz.w, ww.w)) << 16);
    *reinterpret_cast<uint2 *>(out16 + row * 128 + c) = r;
}

// conv weights [C][4] (HF) -> [4][C] (the kai conv's tap-major layout)
__global__ __launch_bounds__(256) void conv_w_transpose_kernel(const float *__restrict__ w, float *__restrict__ wt,
                                                               int C) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    const float4 v = *reinterpret_cast<const float4 *>(w + (size_t)c * 4);
    wt[c] = v.x;
    wt[(size_t)C + c] = v.y;
    wt[(size_t)2 * C + c] = v.z;
    wt[(size_t)3 * C + c] = v.w;
}

// next[b] = the first index of the largest logit of row b.  Block (j, b)
// scans slice j of the row into part[b][j] = (value, index); the last block
// of row b to finish (counter cnt[b], returned to 0 for the next launch) merges
// the slices: the largest value, the smallest index among equals, so the
// result does not depend on the order the blocks finish.
constexpr int kArgBlocks = 64;
GDN_DEV void arg_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}
GDN_DEV void arg_block(float &v, int &i, float *sv, int *si) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) arg_merge(v, i, __shfl_xor(v, o), __shfl_xor(i, o));
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = v;
        si[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
    for (int k = 1; k < 4; ++k) arg_merge(v, i, sv[k], si[k]);
}
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ logits, int32_t *__restrict__ next,
                                                     int V, uint64_t *__restrict__ part, uint32_t *__restrict__ cnt) {
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ bool last;
    const int b = blockIdx.y, j = blockIdx.x;
    const int per = (V + kArgBlocks - 1) / kArgBlocks;
    const int lo = j * per, hi = min(V, lo + per);
    const float *row = logits + (size_t)b * V;
    float best = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = lo + threadIdx.x; i < hi; i += 256) arg_merge(best, bi, row[i], i);
    arg_block(best, bi, sv, si);
    if (threadIdx.x == 0) {
        store_agent(&part[b * kArgBlocks + j], ((uint64_t)__float_as_uint(best) << 32) | (uint32_t)bi);
        stores_done();
        last = arrive_last(&cnt[b], kArgBlocks);
    }
    __syncthreads();
    if (!last) return;
    float v = -INFINITY;
    int i = 0x7FFFFFFF;
    if (threadIdx.x < kArgBlocks) {
        const uint64_t pv = load_agent(&part[b * kArgBlocks + threadIdx.x]);
        v = __uint_as_float((uint32_t)(pv >> 32));
        i = (int)(uint32_t)pv;
    }
    __syncthreads();
    arg_block(v, i, sv, si);
    if (threadIdx.x == 0) next[b] = i;
}

// ---- model -------------------------------------------------------------------

// Tensor streams of the hash: per layer 64 ids from 64 (l + 1); global 0..63;
// drawn states 1 << 20 onwards.
enum : int {
    kLnIn = 0, kLnPost, kQkv, kZ, kBp, kAp, kOut, kConvW, kDtBias, kALog, kNormW,
    kQp, kKp, kVp, kOp, kQn, kKn, kGate, kUp, kDown,
};
enum : int { kEmbed = 1, kFinalNorm = 2, kLmHead = 3 };
enum : int { kStConv = 0, kStS = 1, kStK = 2, kStV = 3 };
constexpr float kWAmp = 0.034641016f;  // uniform amplitude of std 0.02

// An int8 weight matrix [N][K] with per-output-channel scales.  The
// matrices of a layer that read the same input are one Mat, their rows
// concatenated (GDN: in_proj_qkv | in_proj_z | in_proj_b | in_proj_a;
// attention: q_proj | k_proj | v_proj) or interleaved (MLP: gate_proj and
// up_proj in alternating groups of 8 rows), zero rows padding N to a
// multiple of 64.
struct Mat {
    int8_t *q = nullptr;
    float *s = nullptr;
    int N = 0, K = 0;
};

struct Layer {
    bool attn = false;
    float *ln_in = nullptr, *ln_post = nullptr;
    Mat in, out;  // GDN: [qkv | z | b | a], out_proj; attention: [q | k | v], o_proj
    float *conv_w = nullptr, *dt_bias = nullptr, *A_log = nullptr, *norm_w = nullptr;
    float *conv_wt = nullptr;                    // conv_w tap-major [4][conv_dim], for the prefill
    float *q_norm = nullptr, *k_norm = nullptr;
    Mat gate_up, down;
    float *S = nullptr;                          // [B][Hv][128][128]
    float *conv_state[2] = {nullptr, nullptr};   // [B][conv_dim][4], the current one is conv_state[parity]
    uint16_t *Kc = nullptr, *Vc = nullptr;      // [B][Hkv][tmax][256], K tiled by 16 positions
};

// Rows of the interleaved gate/up matrix: row R takes row 8 (R / 16) + R % 8
// of gate (R % 16 < 8) or of up.
__global__ __launch_bounds__(256) void interleave_rows_kernel(const int8_t *__restrict__ ga,
                                                              const int8_t *__restrict__ up,
                                                              const float *__restrict__ sg,
                                                              const float *__restrict__ su,
                                                              int8_t *__restrict__ out, float *__restrict__ so,
                                                              int K) {
    const int R = blockIdx.x;
    const int w = R & 15;
    const int n = (R >> 4) * 8 + (w & 7);
    const int8_t *src = (w < 8 ? ga : up) + (size_t)n * K;
    for (int i = threadIdx.x * 16; i < K; i += 256 * 16)
        *reinterpret_cast<uint4 *>(out + (size_t)R * K + i) = *reinterpret_cast<const uint4 *>(src + i);
    if (threadIdx.x == 0) so[R] = w < 8 ? sg[n] : su[n];
}

}  // namespace
}  // namespace gdn

struct kai_gdn_hybrid {
    kai_gdn_hybrid_config cfg{};
    int conv_dim = 0, value_dim = 0;
    std::vector<gdn::Layer> layers;
    uint16_t *embed = nullptr;
    float *final_norm = nullptr;
    gdn::Mat lm;
    // step buffers
    float *h = nullptr, *mix = nullptr, *mlp = nullptr;
    // small batches: the residual stream alternates between h and h2, and
    // the next matrix normalises its own input from the pending branch
    float *h2 = nullptr, *hcur = nullptr, *hnext = nullptr;
    const float *pend_w = nullptr;
    float *qkv = nullptr, *zb = nullptr, *ab = nullptr, *bb = nullptr;
    float *qg = nullptr, *kx = nullptr, *vx = nullptr, *logits = nullptr;
    int32_t *next = nullptr;
    uint64_t *arg_part = nullptr;  // [max_batch][kArgBlocks]
    uint32_t *arg_cnt = nullptr;   // [max_batch], zero between launches
    uint16_t *x16 = nullptr, *act16 = nullptr, *q16 = nullptr, *o16 = nullptr;
    float *gemm_part = nullptr, *attn_ws = nullptr;
    uint32_t *gemm_cnt = nullptr;  // zero between launches
    // prefill buffers, allocated by the first prefill for max_context rows
    struct Prefill {
        int rows = 0, tv = 0;  // capacity (positions) and the V^T row length
        float *h = nullptr, *qkv = nullptr, *z = nullptr, *a = nullptr, *b = nullptr;
        float *g = nullptr, *beta = nullptr, *kx = nullptr, *vx = nullptr, *hist = nullptr;
        uint16_t *x16 = nullptr, *act16 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
        uint16_t *q16 = nullptr, *vT = nullptr;
    } pf;
    std::vector<void *> allocs;
    size_t bytes = 0, weight_bytes = 0;
    int batch = 0, pos = 0;
    int parity = 0;  // which conv cache of each GDN layer is current
    int tmax = 0;    // KV cache positions: max_context rounded up to 16 (K is tiled by 16)
    // phase timing (kai_gdn_hybrid_set_timing): events recorded so far in
    // this round of sums, the phase each interval (event i-1 .. i) closes
    struct Timing {
        bool on = false;
        std::vector<hipEvent_t> pool;
        std::vector<int> phase;
        size_t used = 0;
        double sum_us[KAI_GDN_PHASE_COUNT] = {};
    } timing;
};

namespace gdn {
namespace {

hipError_t alloc(kai_gdn_hybrid *m, void **p, size_t n) {
    if (n == 0) n = 16;
    hipError_t e = hipMalloc(p, n);
    if (e != hipSuccess) return e;
    m->allocs.push_back(*p);
    m->bytes += n;
    return hipSuccess;
}
template <typename T> hipError_t alloc_t(kai_gdn_hybrid *m, T **p, size_t count) {
    return alloc(m, reinterpret_cast<void **>(p), count * sizeof(T));
}

hipError_t fill(float *dst, size_t n, uint64_t seed, uint64_t stream, float amp, float center) {
    fill_f32_kernel<<<fill_blocks(n), 256>>>(dst, n, seed, stream, amp, center);
    return hipGetLastError();
}

#define TRY(x)                              \
    do {                                    \
        hipError_t e_ = (x);                \
        if (e_ != hipSuccess) return e_;    \
    } while (0)

int pad64(int n) { return (n + 63) / 64 * 64; }

// Timing mode: an event on `st` that closes an interval of phase `ph` (the
// first event of a call opens one, ph < 0).  No-op when timing is off.
hipError_t mark(kai_gdn_hybrid *m, int ph, hipStream_t st) {
    auto &t = m->timing;
    if (!t.on) return hipSuccess;
    if (t.used == t.pool.size()) {
        hipEvent_t e;
        TRY(hipEventCreate(&e));
        t.pool.push_back(e);
        t.phase.push_back(-1);
    }
    t.phase[t.used] = ph;
    return hipEventRecord(t.pool[t.used++], st);
}

// Adds the recorded intervals to the sums and empties the event list.
hipError_t collect(kai_gdn_hybrid *m) {
    auto &t = m->timing;
    if (t.used == 0) return hipSuccess;
    TRY(hipEventSynchronize(t.pool[t.used - 1]));
    for (size_t i = 1; i < t.used; ++i) {
        if (t.phase[i] < 0) continue;
        float ms = 0.f;
        TRY(hipEventElapsedTime(&ms, t.pool[i - 1], t.pool[i]));
        t.sum_us[t.phase[i]] += (double)ms * 1e3;
    }
    t.used = 0;
    return hipSuccess;
}

struct Part {
    int rows;
    uint64_t stream;
};

// Staging of the matrix builders: fp32 draws, row-major int8 (twice).
struct Staging {
    float *f = nullptr;
    int8_t *q = nullptr, *q2 = nullptr;
    float *s = nullptr;
};

// Drawn matrices concatenated by rows into one Mat; each part is drawn from
// its own hash stream and quantised per output channel, then the whole
// matrix is tiled for the GEMM.
hipError_t make_fused(kai_gdn_hybrid *m, Mat &w, std::initializer_list<Part> parts, int K, uint64_t seed,
                      const Staging &tmp) {
    int used = 0;
    for (const Part &p : parts) used += p.rows;
    w.N = pad64(used);
    w.K = K;
    TRY(alloc_t(m, &w.q, (size_t)w.N * K));
    TRY(alloc_t(m, &w.s, (size_t)w.N));
    if (w.N > used) {
        TRY(hipMemset(tmp.q + (size_t)used * K, 0, (size_t)(w.N - used) * K));
        TRY(fill(w.s + used, (size_t)(w.N - used), 0, 0, 0.f, 1.0f));
    }
    int off = 0;
    for (const Part &p : parts) {
        TRY(fill(tmp.f, (size_t)p.rows * K, seed, p.stream, kWAmp, 0.f));
        TRY(launch_w8_quantize(tmp.f, tmp.q + (size_t)off * K, w.s + off, p.rows, K, nullptr));
        off += p.rows;
    }
    TRY(launch_w8f_tile(tmp.q, w.q, w.N, K, nullptr));
    m->weight_bytes += (size_t)w.N * K + (size_t)w.N * 4;
    return hipDeviceSynchronize();
}

// gate_proj and up_proj [I][K], interleaved in groups of 8 rows, tiled.
hipError_t make_gate_up(kai_gdn_hybrid *m, Mat &w, int I, int K, uint64_t seed, uint64_t sg, uint64_t su,
                        const Staging &tmp) {
    w.N = 2 * I;
    w.K = K;
    TRY(alloc_t(m, &w.q, (size_t)w.N * K));
    TRY(alloc_t(m, &w.s, (size_t)w.N));
    TRY(fill(tmp.f, (size_t)I * K, seed, sg, kWAmp, 0.f));
    TRY(launch_w8_quantize(tmp.f, tmp.q, tmp.s, I, K, nullptr));
    TRY(fill(tmp.f, (size_t)I * K, seed, su, kWAmp, 0.f));
    TRY(launch_w8_quantize(tmp.f, tmp.q + (size_t)I * K, tmp.s + I, I, K, nullptr));
    interleave_rows_kernel<<<w.N, 256>>>(tmp.q, tmp.q + (size_t)I * K, tmp.s, tmp.s + I, tmp.q2, w.s, K);
    TRY(hipGetLastError());
    TRY(launch_w8f_tile(tmp.q2, w.q, w.N, K, nullptr));
    m->weight_bytes += (size_t)w.N * K + (size_t)w.N * 4;
    return hipDeviceSynchronize();
}

hipError_t make_vec(kai_gdn_hybrid *m, float **v, size_t n, uint64_t seed, uint64_t stream, float amp,
                    float center) {
    hipError_t e = alloc_t(m, v, n);
    return e != hipSuccess ? e : fill(*v, n, seed, stream, amp, center);
}

W8Out segments(std::initializer_list<W8Seg> segs) {
    W8Out o{};
    int q = 0;
    for (const W8Seg &sg : segs) o.seg[q++] = sg;
    o.nseg = q;
    o.mode = kW8Segments;
    return o;
}

hipError_t gemm(kai_gdn_hybrid *m, const uint16_t *x, const Mat &w, const W8Out &o, hipStream_t st) {
    return launch_w8f(x, w.q, w.s, m->batch, w.N, w.K, o, m->gemm_part, m->gemm_cnt, st);
}
hipError_t gemm_to(kai_gdn_hybrid *m, const uint16_t *x, const Mat &w, float *y, int ld, hipStream_t st) {
    return gemm(m, x, w, segments({{y, ld, w.N}}), st);
}

// At batch 1 the matrices that read the residual stream's norm (the
// in-projections, gate|up, lm_head) form it themselves: every block
// normalises the row into LDS while its weights are in flight
// (W8Out::nin_*), and the branch matrix before them adds its branch to the
// residual stream in its epilogue (W8Out::add_in).  That replaces the norm
// kernel.  From batch 2, one block per row in a kernel of its own is faster
// than every block normalising every row; both forms compute the same sums
// in the same order, so a sequence's logits do not depend on the batch.
bool norm_in(const kai_gdn_hybrid *m) { return m->batch <= kW8NormInRows && m->cfg.hidden <= kW8NormInMaxK; }

// d = x W^T (the branch); h += d; x16 = fp16(rmsnorm(h) * (1 + norm_w)),
// or, at batch 1, h' = h + d from the matrix's epilogue and the norm left
// to the next matrix
hipError_t gemm_addnorm(kai_gdn_hybrid *m, const uint16_t *x, const Mat &w, float *d, const float *norm_w,
                        hipStream_t st) {
    const int B = m->batch, H = m->cfg.hidden;
    if (norm_in(m)) {
        W8Out o = segments({{m->hnext, H, w.N}});
        o.add_in = m->hcur;
        o.add_ld = H;
        TRY(gemm(m, x, w, o, st));
        std::swap(m->hcur, m->hnext);
        m->pend_w = norm_w;
        return hipSuccess;
    }
    TRY(gemm_to(m, x, w, d, H, st));
    addnorm_kernel<<<B, 256, 0, st>>>(m->h, d, norm_w, m->x16, H, m->cfg.rms_eps);
    return hipGetLastError();
}

// o = norm(h) W^T: from x16, or, at batch 1, normalising the residual
// stream in the matrix's own blocks
hipError_t gemm_in(kai_gdn_hybrid *m, const Mat &w, W8Out o, hipStream_t st) {
    if (!norm_in(m)) return gemm(m, m->x16, w, o, st);
    o.nin_h = m->hcur;
    o.nin_w = m->pend_w;
    o.nin_eps = m->cfg.rms_eps;
    return gemm(m, nullptr, w, o, st);
}

hipError_t build(kai_gdn_hybrid *m, uint64_t seed) {
    const kai_gdn_hybrid_config &c = m->cfg;
    const int H = c.hidden, I = c.inter, Hk = c.gdn_k_heads, Hv = c.gdn_v_heads, Hq = c.attn_q_heads,
              Hkv = c.attn_kv_heads, Bm = c.max_batch;
    m->conv_dim = 2 * Hk * 128 + Hv * 128;
    m->value_dim = Hv * 128;
    m->tmax = (c.max_context + 15) / 16 * 16;
    // staging for the builders: the largest matrix (padded), fp32 and int8
    const size_t tmp_n = std::max({(size_t)pad64(c.vocab) * H, (size_t)2 * I * H, (size_t)I * H,
                                   (size_t)pad64(m->conv_dim + m->value_dim + 2 * Hv) * H,
                                   (size_t)pad64(Hq * 512 + 2 * Hkv * 256) * H, (size_t)H * m->value_dim,
                                   (size_t)H * Hq * 256});
    Staging tmp;
    auto run = [&]() -> hipError_t {
        TRY(hipMalloc(&tmp.f, tmp_n * 4));
        TRY(hipMalloc(&tmp.q, tmp_n));
        TRY(hipMalloc(&tmp.q2, (size_t)2 * I * H));
        TRY(hipMalloc(&tmp.s, (size_t)2 * I * 4));
        m->layers.resize(c.layers);
        for (int l = 0; l < c.layers; ++l) {
            Layer &L = m->layers[l];
            const uint64_t base = 64ull * (l + 1);
            L.attn = (l + 1) % c.attn_every == 0;
            TRY(make_vec(m, &L.ln_in, H, seed, base + kLnIn, 0.1f, 0.f));
            TRY(make_vec(m, &L.ln_post, H, seed, base + kLnPost, 0.1f, 0.f));
            if (!L.attn) {
                TRY(make_fused(m, L.in, {{m->conv_dim, base + kQkv}, {m->value_dim, base + kZ}, {Hv, base + kBp},
                                         {Hv, base + kAp}}, H, seed, tmp));
                TRY(make_fused(m, L.out, {{H, base + kOut}}, m->value_dim, seed, tmp));
                TRY(make_vec(m, &L.conv_w, (size_t)m->conv_dim * 4, seed, base + kConvW, 0.5f, 0.f));
                TRY(alloc_t(m, &L.conv_wt, (size_t)m->conv_dim * 4));
                conv_w_transpose_kernel<<<(m->conv_dim + 255) / 256, 256>>>(L.conv_w, L.conv_wt, m->conv_dim);
                TRY(hipGetLastError());
                TRY(make_vec(m, &L.dt_bias, Hv, seed, base + kDtBias, 0.5f, 1.0f));
                TRY(make_vec(m, &L.A_log, Hv, seed, base + kALog, 1.3862944f, 1.3862944f));  // U(0, ln 16)
                TRY(make_vec(m, &L.norm_w, 128, seed, base + kNormW, 0.1f, 1.0f));
                TRY(alloc_t(m, &L.S, (size_t)Bm * Hv * 128 * 128));
                TRY(alloc_t(m, &L.conv_state[0], (size_t)Bm * m->conv_dim * 4));
                TRY(alloc_t(m, &L.conv_state[1], (size_t)Bm * m->conv_dim * 4));
            } else {
                TRY(make_fused(m, L.in, {{Hq * 512, base + kQp}, {Hkv * 256, base + kKp}, {Hkv * 256, base + kVp}},
                               H, seed, tmp));
                TRY(make_fused(m, L.out, {{H, base + kOp}}, Hq * 256, seed, tmp));
                TRY(make_vec(m, &L.q_norm, 256, seed, base + kQn, 0.1f, 0.f));
                TRY(make_vec(m, &L.k_norm, 256, seed, base + kKn, 0.1f, 0.f));
                TRY(alloc_t(m, &L.Kc, (size_t)Bm * Hkv * m->tmax * 256));
                TRY(alloc_t(m, &L.Vc, (size_t)Bm * Hkv * m->tmax * 256));
            }
            TRY(make_gate_up(m, L.gate_up, I, H, seed, base + kGate, base + kUp, tmp));
            TRY(make_fused(m, L.down, {{H, base + kDown}}, I, seed, tmp));
        }
        TRY(alloc_t(m, &m->embed, (size_t)c.vocab * H));
        fill_f16_kernel<<<fill_blocks((size_t)c.vocab * H), 256>>>(m->embed, (size_t)c.vocab * H, seed, kEmbed,
                                                                   1.0f, 0.f);
        TRY(hipGetLastError());
        TRY(make_vec(m, &m->final_norm, H, seed, kFinalNorm, 0.1f, 0.f));
        TRY(make_fused(m, m->lm, {{c.vocab, kLmHead}}, H, seed, tmp));
        // step buffers
        const size_t wide16 = std::max({(size_t)H, (size_t)m->value_dim, (size_t)Hq * 256});
        TRY(alloc_t(m, &m->h, (size_t)Bm * H));
        TRY(alloc_t(m, &m->h2, (size_t)Bm * H));
        TRY(alloc_t(m, &m->mix, (size_t)Bm * H));
        TRY(alloc_t(m, &m->mlp, (size_t)Bm * H));
        TRY(alloc_t(m, &m->qkv, (size_t)Bm * m->conv_dim));
        TRY(alloc_t(m, &m->zb, (size_t)Bm * m->value_dim));
        TRY(alloc_t(m, &m->ab, (size_t)Bm * Hv));
        TRY(alloc_t(m, &m->bb, (size_t)Bm * Hv));
        TRY(alloc_t(m, &m->qg, (size_t)Bm * Hq * 512));
        TRY(alloc_t(m, &m->kx, (size_t)Bm * Hkv * 256));
        TRY(alloc_t(m, &m->vx, (size_t)Bm * Hkv * 256));
        TRY(alloc_t(m, &m->logits, (size_t)Bm * c.vocab));
        TRY(alloc_t(m, &m->next, (size_t)Bm));
        TRY(alloc_t(m, &m->arg_part, (size_t)Bm * kArgBlocks));
        TRY(alloc_t(m, &m->arg_cnt, (size_t)Bm));
        TRY(hipMemset(m->arg_cnt, 0, (size_t)Bm * sizeof(uint32_t)));
        TRY(alloc_t(m, &m->x16, (size_t)Bm * wide16));
        TRY(alloc_t(m, &m->o16, (size_t)Bm * wide16));
        TRY(alloc_t(m, &m->act16, (size_t)Bm * I));
        TRY(alloc_t(m, &m->q16, (size_t)Bm * Hq * 256));
        // GEMM split-K partials and counters: the largest over the model's matrices
        size_t part = 0, groups = 0;
        auto need = [&](const Mat &w) {
            part = std::max(part, w8f_workspace_floats(Bm, w.N, w.K));
            groups = std::max(groups, (size_t)w.N / 64);
        };
        for (const Layer &L : m->layers) {
            need(L.in);
            need(L.out);
            need(L.gate_up);
            need(L.down);
        }
        need(m->lm);
        TRY(alloc_t(m, &m->gemm_part, part));
        TRY(alloc_t(m, &m->gemm_cnt, groups));
        TRY(hipMemset(m->gemm_cnt, 0, groups * sizeof(uint32_t)));
        TRY(alloc(m, reinterpret_cast<void **>(&m->attn_ws), attn_workspace_bytes_tiled(Bm, Hq, c.max_context)));
        return hipDeviceSynchronize();
    };
    const hipError_t e = run();
    for (void *p : {(void *)tmp.f, (void *)tmp.q, (void *)tmp.q2, (void *)tmp.s})
        if (p) (void)hipFree(p);
    return e;
}

hipError_t gdn_mixer(kai_gdn_hybrid *m, Layer &L, hipStream_t st) {
    const kai_gdn_hybrid_config &c = m->cfg;
    const int B = m->batch, Hk = c.gdn_k_heads, Hv = c.gdn_v_heads, C = m->conv_dim, V = m->value_dim;
    TRY(gemm_in(m, L.in, segments({{m->qkv, C, C}, {m->zb, V, C + V}, {m->bb, Hv, C + V + Hv},
                                        {m->ab, Hv, C + V + 2 * Hv}}), st));
    TRY(mark(m, KAI_GDN_PHASE_GDN_PROJ, st));
    // conv update, gating prologue, delta rule, gated RMSNorm -> fp16: one kernel
    TRY(launch_gdn_step_fused(m->qkv, L.conv_state[m->parity], L.conv_state[m->parity ^ 1], L.conv_w, m->ab,
                              m->bb, L.A_log, L.dt_bias, L.S, m->zb, L.norm_w, m->o16, B, Hk, Hv,
                              1.0f / sqrtf(128.0f), c.rms_eps, st));
    TRY(mark(m, KAI_GDN_PHASE_GDN_CORE, st));
    TRY(gemm_addnorm(m, m->o16, L.out, m->mix, L.ln_post, st));
    return mark(m, KAI_GDN_PHASE_GDN_OPROJ, st);
}

hipError_t attn_mixer(kai_gdn_hybrid *m, Layer &L, hipStream_t st) {
    const kai_gdn_hybrid_config &c = m->cfg;
    const int B = m->batch, Hq = c.attn_q_heads, Hkv = c.attn_kv_heads;
    const int nq = Hq * 512, nkv = Hkv * 256;
    TRY(gemm_in(m, L.in, segments({{m->qg, nq, nq}, {m->kx, nkv, nq + nkv}, {m->vx, nkv, nq + 2 * nkv}}),
             st));
    attn_prologue_kernel<<<dim3(B, Hq + 2 * Hkv), 256, 0, st>>>(m->qg, m->kx, m->vx, L.q_norm, L.k_norm, m->q16,
                                                                 L.Kc, L.Vc, Hq, Hkv, m->tmax, -1, m->pos,
                                                                 c.rope_theta, c.rms_eps, nullptr, 0);
    TRY(hipGetLastError());
    // o * sigmoid(gate) -> fp16 in the span combine; gate = dims 256..511 of each qg head
    TRY(launch_attn_decode(m->q16, L.Kc, L.Vc, nullptr, B, Hq, Hkv, m->tmax, m->pos + 1, 1.0f / 16.0f,
                           m->attn_ws, st, m->qg + 256, 512, m->o16, /*k_tiled=*/true));
    TRY(gemm_addnorm(m, m->o16, L.out, m->mix, L.ln_post, st));
    return mark(m, KAI_GDN_PHASE_ATTN, st);
}

hipError_t step(kai_gdn_hybrid *m, const int32_t *tokens, int32_t *next, float *logits, hipStream_t st) {
    const kai_gdn_hybrid_config &c = m->cfg;
    const int B = m->batch, H = c.hidden;
    TRY(mark(m, -1, st));
    embed_kernel<<<B, 256, 0, st>>>(tokens, m->embed, m->h, H, c.vocab);
    TRY(hipGetLastError());
    W8Out swiglu{};
    swiglu.mode = kW8SwiGLU;
    swiglu.x16 = m->act16;
    // each residual branch's matrix (out, down) adds the branch to h and
    // normalises h for the next matrix: the next layer's input norm, or the
    // final norm after the last layer
    m->hcur = m->h;
    m->hnext = m->h2;
    m->pend_w = m->layers[0].ln_in;
    if (!norm_in(m)) {
        addnorm_kernel<<<B, 256, 0, st>>>(m->h, nullptr, m->layers[0].ln_in, m->x16, H, c.rms_eps);
        TRY(hipGetLastError());
    }
    TRY(mark(m, KAI_GDN_PHASE_OTHER, st));
    for (size_t l = 0; l < m->layers.size(); ++l) {
        Layer &L = m->layers[l];
        TRY(L.attn ? attn_mixer(m, L, st) : gdn_mixer(m, L, st));
        TRY(gemm_in(m, L.gate_up, swiglu, st));
        const float *next_norm = l + 1 < m->layers.size() ? m->layers[l + 1].ln_in : m->final_norm;
        TRY(gemm_addnorm(m, m->act16, L.down, m->mlp, next_norm, st));
        TRY(mark(m, KAI_GDN_PHASE_FFN, st));
    }
    float *lg = logits ? logits : m->logits;
    TRY(gemm_in(m, m->lm, segments({{lg, c.vocab, c.vocab}}), st));
    argmax_kernel<<<dim3(kArgBlocks, B), 256, 0, st>>>(lg, next ? next : m->next, c.vocab, m->arg_part,
                                                       m->arg_cnt);
    TRY(hipGetLastError());
    TRY(mark(m, KAI_GDN_PHASE_OTHER, st));
    ++m->pos;
    m->parity ^= 1;
    return hipSuccess;
}

// ---- prefill -------------------------------------------------------------------

hipError_t prefill_alloc(kai_gdn_hybrid *m) {
    if (m->pf.rows) return hipSuccess;
    const kai_gdn_hybrid_config &c = m->cfg;
    const size_t R = (size_t)c.max_context;
    const int H = c.hidden, C = m->conv_dim, V = m->value_dim, Hk = c.gdn_k_heads, Hv = c.gdn_v_heads,
              Hq = c.attn_q_heads, Hkv = c.attn_kv_heads;
    kai_gdn_hybrid::Prefill &p = m->pf;
    p.tv = (int)((R + 63) / 64 * 64);
    const size_t x16w = std::max({(size_t)H, (size_t)V, (size_t)Hq * 256});
    TRY(alloc_t(m, &p.h, R * H));
    TRY(alloc_t(m, &p.qkv, R * std::max((size_t)C, (size_t)Hq * 512)));
    TRY(alloc_t(m, &p.z, R * V));
    TRY(alloc_t(m, &p.a, R * Hv));
    TRY(alloc_t(m, &p.b, R * Hv));
    TRY(alloc_t(m, &p.g, R * Hv));
    TRY(alloc_t(m, &p.beta, R * Hv));
    TRY(alloc_t(m, &p.kx, R * Hkv * 256));
    TRY(alloc_t(m, &p.vx, R * Hkv * 256));
    TRY(alloc_t(m, &p.hist, (size_t)3 * C));
    TRY(alloc_t(m, &p.x16, R * x16w));
    TRY(alloc_t(m, &p.act16, R * c.inter));
    TRY(alloc_t(m, &p.q, R * Hk * 128));
    TRY(alloc_t(m, &p.k, R * Hk * 128));
    TRY(alloc_t(m, &p.v, R * V));
    TRY(alloc_t(m, &p.o, R * V));
    TRY(alloc_t(m, &p.q16, R * Hq * 256));
    TRY(alloc_t(m, &p.vT, (size_t)Hkv * 256 * p.tv));
    // V^T past a prefill's length is read (with weight 0): keep it finite
    TRY(hipMemset(p.vT, 0, (size_t)Hkv * 256 * p.tv * sizeof(uint16_t)));
    p.rows = (int)R;
    return hipDeviceSynchronize();
}

hipError_t w8p(const uint16_t *x, int ldx, const Mat &w, int M, const W8Out &o, hipStream_t st) {
    return launch_w8p(x, ldx, w.q, w.s, M, w.N, w.K, o, st);
}
// A branch matrix: h[t] += x[t] W^T for the T rows, the residual add in the
// GEMM's epilogue (in place), so no branch array is written and read back.
hipError_t w8p_residual(const uint16_t *x, int ldx, const Mat &w, int M, float *h, int H, hipStream_t st) {
    W8Out o = segments({{h, H, H}});
    o.add_in = h;
    o.add_ld = H;
    return w8p(x, ldx, w, M, o, st);
}

// One sequence's prompt through every layer at once: T rows of sequence b.
// Leaves its states (recurrent state, conv cache, K/V cache) where the
// decode step reads them and the normalised last row in x16 row b.
hipError_t prefill_seq(kai_gdn_hybrid *m, const int32_t *tokens, int b, int T, hipStream_t st) {
    const kai_gdn_hybrid_config &c = m->cfg;
    const int H = c.hidden, C = m->conv_dim, V = m->value_dim, Hk = c.gdn_k_heads, Hv = c.gdn_v_heads,
              Hq = c.attn_q_heads, Hkv = c.attn_kv_heads, I = c.inter;
    kai_gdn_hybrid::Prefill &p = m->pf;
    TRY(mark(m, -1, st));
    embed_kernel<<<T, 256, 0, st>>>(tokens, m->embed, p.h, H, c.vocab);
    TRY(hipGetLastError());
    addnorm_kernel<<<T, 256, 0, st>>>(p.h, nullptr, m->layers[0].ln_in, p.x16, H, c.rms_eps);
    TRY(hipGetLastError());
    TRY(mark(m, KAI_GDN_PHASE_OTHER, st));
    W8Out swiglu{};
    swiglu.mode = kW8SwiGLU;
    swiglu.x16 = p.act16;
    for (size_t l = 0; l < m->layers.size(); ++l) {
        Layer &L = m->layers[l];
        if (!L.attn) {
            TRY(w8p(p.x16, H, L.in, T, segments({{p.qkv, C, C}, {p.z, V, C + V}, {p.b, Hv, C + V + Hv},
                                                  {p.a, Hv, C + V + 2 * Hv}}), st));
            TRY(mark(m, KAI_GDN_PHASE_GDN_PROJ, st));
            // the decode step's conv cache: the last four conv inputs
            TRY(launch_conv_state_from_inputs(p.qkv, L.conv_state[0] + (size_t)b * C * 4, 1, T, C, st));
            TRY(hipMemsetAsync(p.hist, 0, (size_t)3 * C * sizeof(float), st));
            TRY(launch_conv_gating(p.qkv, L.conv_wt, p.hist, p.a, p.b, L.A_log, L.dt_bias, p.q, p.k, p.v, p.g,
                                   p.beta, T, Hk, Hv, st));
            float *S = L.S + (size_t)b * Hv * 128 * 128;
            TRY(hipMemsetAsync(S, 0, (size_t)Hv * 128 * 128 * sizeof(float), st));
            const int rc = kai_run_gdn_chunk_delta_rule_bf16_f32_hip(p.q, p.k, p.v, p.g, p.beta, p.o, S, 1, T, Hv,
                                                                    Hk, 1.0f / sqrtf(128.0f), st);
            if (rc) return (hipError_t)rc;
            const size_t rows = (size_t)T * Hv;
            prefill_gated_norm_kernel<<<(unsigned)((rows + 7) / 8), 256, 0, st>>>(p.o, p.z, L.norm_w, p.x16, rows,
                                                                                  c.rms_eps);
            TRY(hipGetLastError());
            TRY(mark(m, KAI_GDN_PHASE_GDN_CORE, st));
            TRY(w8p_residual(p.x16, V, L.out, T, p.h, H, st));
            TRY(mark(m, KAI_GDN_PHASE_GDN_OPROJ, st));
        } else {
            const int nq = Hq * 512, nkv = Hkv * 256;
            TRY(w8p(p.x16, H, L.in, T, segments({{p.qkv, nq, nq}, {p.kx, nkv, nq + nkv}, {p.vx, nkv, nq + 2 * nkv}}),
                    st));
            attn_prologue_rows_kernel<<<dim3((T + 4 * kApRows - 1) / (4 * kApRows), Hq + 2 * Hkv), 256, 0, st>>>(
                p.qkv, p.kx, p.vx, L.q_norm, L.k_norm, p.q16, L.Kc, L.Vc, Hq, Hkv, m->tmax, T, b, c.rope_theta,
                c.rms_eps, p.vT, p.tv);
            TRY(hipGetLastError());
            const size_t kvrow = (size_t)b * Hkv * m->tmax * 256;
            TRY(launch_attn_prefill(p.q16, L.Kc + kvrow, p.vT, p.qkv + 256, nq, p.x16, T, Hq, Hkv, m->tmax, p.tv,
                                    1.0f / 16.0f, st));
            TRY(w8p_residual(p.x16, Hq * 256, L.out, T, p.h, H, st));
            TRY(mark(m, KAI_GDN_PHASE_ATTN, st));
        }
        addnorm_kernel<<<T, 256, 0, st>>>(p.h, nullptr, L.ln_post, p.x16, H, c.rms_eps);
        TRY(hipGetLastError());
        TRY(w8p(p.x16, H, L.gate_up, T, swiglu, st));
        TRY(w8p_residual(p.act16, I, L.down, T, p.h, H, st));
        const float *next_norm = l + 1 < m->layers.size() ? m->layers[l + 1].ln_in : m->final_norm;
        addnorm_kernel<<<T, 256, 0, st>>>(p.h, nullptr, next_norm, p.x16, H, c.rms_eps);
        TRY(hipGetLastError());
        TRY(mark(m, KAI_GDN_PHASE_FFN, st));
    }
    return hipMemcpyAsync(m->x16 + (size_t)b * H, p.x16 + (size_t)(T - 1) * H, (size_t)H * sizeof(uint16_t),
                          hipMemcpyDeviceToDevice, st);
}

hipError_t prefill(kai_gdn_hybrid *m, const int32_t *tokens, int batch, int T, int32_t *next, float *logits,
                   hipStream_t st) {
    const kai_gdn_hybrid_config &c = m->cfg;
    TRY(prefill_alloc(m));
    // a step may still run on another stream: the states below are rewritten
    TRY(hipDeviceSynchronize());
    m->batch = batch;
    m->pos = 0;
    m->parity = 0;
    for (int b = 0; b < batch; ++b) TRY(prefill_seq(m, tokens + (size_t)b * T, b, T, st));
    float *lg = logits ? logits : m->logits;
    TRY(mark(m, -1, st));
    TRY(gemm(m, m->x16, m->lm, segments({{lg, c.vocab, c.vocab}}), st));
    argmax_kernel<<<dim3(kArgBlocks, batch), 256, 0, st>>>(lg, next ? next : m->next, c.vocab, m->arg_part,
                                                           m->arg_cnt);
    TRY(hipGetLastError());
    TRY(mark(m, KAI_GDN_PHASE_OTHER, st));
    m->pos = T;
    return hipSuccess;
}

hipError_t reset(kai_gdn_hybrid *m, int batch, int context, uint64_t seed) {
    const kai_gdn_hybrid_config &c = m->cfg;
    // a step may still run on any stream the caller used: the fills below
    // (null stream) overwrite the states and caches it reads
    TRY(hipDeviceSynchronize());
    m->batch = batch;
    m->pos = context;
    m->parity = 0;
    for (size_t l = 0; l < m->layers.size(); ++l) {
        Layer &L = m->layers[l];
        const uint64_t base = (1ull << 20) + 16ull * l;
        if (!L.attn) {
            const size_t ns = (size_t)batch * c.gdn_v_heads * 128 * 128, nc = (size_t)batch * m->conv_dim * 4;
            if (context > 0) {
                TRY(fill(L.S, ns, seed, base + kStS, 0.034641016f, 0.f));
                TRY(fill(L.conv_state[0], nc, seed, base + kStConv, 1.0f, 0.f));
            } else {
                TRY(hipMemset(L.S, 0, ns * 4));
                TRY(hipMemset(L.conv_state[0], 0, nc * 4));
            }
        } else {
            const size_t rows = (size_t)batch * c.attn_kv_heads;
            const size_t n = rows * m->tmax * 256;
            fill_cache_kernel<true><<<fill_blocks(n), 256>>>(L.Kc, rows, m->tmax, c.max_context, context, seed,
                                                             base + kStK, 1.0f);
            fill_cache_kernel<false><<<fill_blocks(n), 256>>>(L.Vc, rows, m->tmax, c.max_context, context, seed,
                                                              base + kStV, 1.0f);
            TRY(hipGetLastError());
        }
    }
    return hipDeviceSynchronize();
}

}  // namespace
}  // namespace gdn

extern "C" kai_gdn_hybrid_config kai_gdn_hybrid_qwen35_4b(int max_batch, int max_context) {
    kai_gdn_hybrid_config c{};
    c.layers = 32;
    c.attn_every = 4;
    c.hidden = 2560;
    c.inter = 9216;
    c.vocab = 151936;
    c.gdn_k_heads = 16;
    c.gdn_v_heads = 32;
    c.attn_q_heads = 16;
    c.attn_kv_heads = 4;
    c.max_batch = max_batch;
    c.max_context = max_context;
    c.rope_theta = 1.0e7f;
    c.rms_eps = 1e-6f;
    return c;
}

extern "C" void kai_gdn_hybrid_destroy(kai_gdn_hybrid *m) {
    if (!m) return;
    for (void *p : m->allocs) (void)hipFree(p);
    for (hipEvent_t e : m->timing.pool) (void)hipEventDestroy(e);
    delete m;
}

extern "C" int kai_gdn_hybrid_create(const kai_gdn_hybrid_config *cfg, unsigned long long seed,
                                     kai_gdn_hybrid **out) {
    if (!cfg || !out) return (int)hipErrorInvalidValue;
    const kai_gdn_hybrid_config &c = *cfg;
    const bool ok = c.layers > 0 && c.attn_every > 0 && c.hidden > 0 && c.hidden % 256 == 0 &&
                    c.hidden <= 4 * 256 * gdn::kNormChunks && c.inter > 0 &&
                    c.inter % 256 == 0 && c.vocab > 0 && c.vocab % 16 == 0 && c.gdn_k_heads > 0 &&
                    c.gdn_v_heads % 16 == 0 && c.gdn_v_heads % c.gdn_k_heads == 0 && c.gdn_v_heads > 0 &&
                    c.attn_kv_heads > 0 && c.attn_q_heads > 0 && c.attn_q_heads % c.attn_kv_heads == 0 &&
                    c.attn_q_heads / c.attn_kv_heads <= 4 && c.max_batch >= 1 && c.max_batch <= 16 &&
                    c.max_context >= 1 && c.max_context <= (1 << 24) && c.rms_eps >= 0.f && c.rope_theta > 0.f;
    if (!ok) return (int)hipErrorInvalidValue;
    // no C++ exception may cross the C ABI: allocation failures become codes
    kai_gdn_hybrid *m = new (std::nothrow) kai_gdn_hybrid;
    if (!m) return (int)hipErrorOutOfMemory;
    hipError_t e;
    try {
        m->cfg = c;
        e = gdn::build(m, seed);
    } catch (...) {
        e = hipErrorOutOfMemory;
    }
    if (e != hipSuccess) {
        kai_gdn_hybrid_destroy(m);
        return (int)e;
    }
    m->batch = c.max_batch;
    *out = m;
    return 0;
}

extern "C" int kai_gdn_hybrid_reset(kai_gdn_hybrid *m, int batch, int context, unsigned long long seed) {
    if (!m || batch < 1 || batch > m->cfg.max_batch || context < 0 || context >= m->cfg.max_context)
        return (int)hipErrorInvalidValue;
    return (int)gdn::reset(m, batch, context, seed);
}

namespace {
// Device (or managed) memory: a host pointer handed to a step would fault
// the GPU, so it is refused before anything is launched.
bool device_ptr(const void *p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}
}  // namespace

extern "C" int kai_gdn_hybrid_step(kai_gdn_hybrid *m, const int32_t *tokens, int32_t *next, float *logits,
                                   void *stream) {
    if (!m || !tokens || !device_ptr(tokens) || (next && !device_ptr(next)) || (logits && !device_ptr(logits)))
        return (int)hipErrorInvalidValue;
    if (m->pos >= m->cfg.max_context) return (int)hipErrorInvalidValue;  // the KV cache is full
    return (int)gdn::step(m, tokens, next, logits, (hipStream_t)stream);
}

extern "C" int kai_gdn_hybrid_prefill(kai_gdn_hybrid *m, const int32_t *tokens, int batch, int length,
                                      int32_t *next, float *logits, void *stream) {
    // every launch of the prefill accepts `length` rows (checked here, so a
    // refused call leaves the model's states untouched)
    if (!m || !tokens || batch < 1 || batch > m->cfg.max_batch || length < 1 || length >= m->cfg.max_context ||
        length > gdn::w8p_max_rows() || !device_ptr(tokens) || (next && !device_ptr(next)) ||
        (logits && !device_ptr(logits)))
        return (int)hipErrorInvalidValue;
    return (int)gdn::prefill(m, tokens, batch, length, next, logits, (hipStream_t)stream);
}

extern "C" int kai_gdn_hybrid_set_timing(kai_gdn_hybrid *m, int on) {
    if (!m) return (int)hipErrorInvalidValue;
    auto &t = m->timing;
    t.on = on != 0;
    t.used = 0;
    for (double &v : t.sum_us) v = 0.0;
    return 0;
}

extern "C" int kai_gdn_hybrid_phase_times(kai_gdn_hybrid *m, double *us, int n) {
    if (!m || !us || n < 0 || n > KAI_GDN_PHASE_COUNT) return (int)hipErrorInvalidValue;
    const hipError_t e = gdn::collect(m);
    if (e != hipSuccess) return (int)e;
    for (int i = 0; i < n; ++i) us[i] = m->timing.sum_us[i];
    for (double &v : m->timing.sum_us) v = 0.0;
    return 0;
}

extern "C" int kai_gdn_hybrid_position(const kai_gdn_hybrid *m) { return m ? m->pos : -1; }
extern "C" size_t kai_gdn_hybrid_device_bytes(const kai_gdn_hybrid *m) { return m ? m->bytes : 0; }
extern "C" size_t kai_gdn_hybrid_weight_bytes(const kai_gdn_hybrid *m) { return m ? m->weight_bytes : 0; }

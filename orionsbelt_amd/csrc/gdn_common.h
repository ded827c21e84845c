// gdn_common.h -- device helpers shared by the GDN kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define GDN_DEV __device__ __forceinline__

// ---- narrow formats --------------------------------------------------------

// float -> bfloat16 bits, round to nearest even by bias-and-truncate: the
// same rule as the reference's f32_to_bf16_rne (gdn_sve.c:81-87).
GDN_DEV uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

GDN_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Two floats -> packed bf16 pair with the gfx950 hardware convert
// (v_cvt_pk_bf16_f32, round to nearest even; equal to f32_to_bf16_rne for
// every finite input).  Used for MFMA operands, where only the value matters.
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
GDN_DEV uint32_t pack2_bf16_hw(float a, float b) {
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
GDN_DEV uint16_t f32_to_bf16_hw(float a) { return __builtin_bit_cast(uint16_t, (__bf16)a); }

// IEEE binary16 <-> binary32 with the hardware converts (v_cvt_f16_f32 rounds
// to nearest even, keeps subnormals).
GDN_DEV uint16_t f32_to_f16_rne(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

GDN_DEV float f16_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// ---- MFMA: v_mfma_f32_16x16x32_bf16 -----------------------------------------
// Operand layout (lane l, g = l >> 4, r = l & 15):
//   A fragment: A[r][8g + 0..7]     (16 x 32, row r, 8 consecutive k)
//   B fragment: B[8g + 0..7][r]     (32 x 16, column r, 8 consecutive k)
//   C fragment: C[4g + 0..3][r]     (16 x 16, column r, 4 consecutive rows)
// The k index inside a 32-wide step is a pure reduction index: any
// permutation applied identically to A and B leaves the product unchanged.

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

GDN_DEV f32x4_t mfma_16x16x32_bf16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Pack 8 floats into a bf16x8 fragment (round to nearest even).
GDN_DEV bf16x8_t pack_bf16x8(const float *f) {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)f32_to_bf16_rne(f[2 * i]) |
               ((uint32_t)f32_to_bf16_rne(f[2 * i + 1]) << 16);
    return __builtin_bit_cast(bf16x8_t, w);
}

GDN_DEV bf16x8_t as_bf16x8(u32x4_t w) { return __builtin_bit_cast(bf16x8_t, w); }

GDN_DEV f32x4_t zero4() { return f32x4_t{0.f, 0.f, 0.f, 0.f}; }

// ---- fp16 MFMA operands and int8 weights -------------------------------------
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Four int8 (one dword) -> four fp16, exactly.
GDN_DEV void i8x4_to_f16(uint32_t w, f16x2_t &lo, f16x2_t &hi) {
    const uint32_t t = w ^ 0x80808080u;  // u = q + 128 per byte
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u);  // [u0, 0x64, u1, 0x64]
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u);  // [u2, 0x64, u3, 0x64]
    const f16x2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(f16x2_t, a) - bias;
    hi = __builtin_bit_cast(f16x2_t, b) - bias;
}
// 16 int8 -> two MFMA operands of 8 fp16 (k = 0..7 and 8..15 of the 16).
GDN_DEV void i8x16_to_f16(const u32x4_t &w, f16x8_t &k0, f16x8_t &k1) {
    f16x2_t p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) i8x4_to_f16(w[i], p[2 * i], p[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        k0[2 * i] = p[i][0];
        k0[2 * i + 1] = p[i][1];
        k1[2 * i] = p[4 + i][0];
        k1[2 * i + 1] = p[4 + i][1];
    }
}

// ---- plain / non-temporal vector memory access ------------------------------
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

template <bool NT> GDN_DEV float4 load_f4(const float *p) {
    const f32x4_t *q = reinterpret_cast<const f32x4_t *>(p);
    f32x4_t v;
    if constexpr (NT) v = __builtin_nontemporal_load(q);
    else v = *q;
    return make_float4(v[0], v[1], v[2], v[3]);
}
template <bool NT> GDN_DEV void store_f4(float *p, float4 x) {
    f32x4_t v = {x.x, x.y, x.z, x.w};
    f32x4_t *q = reinterpret_cast<f32x4_t *>(p);
    if constexpr (NT) __builtin_nontemporal_store(v, q);
    else *q = v;
}
template <bool NT> GDN_DEV u32x2_t load_u2(const void *p) {
    const u32x2_t *q = reinterpret_cast<const u32x2_t *>(p);
    if constexpr (NT) return __builtin_nontemporal_load(q);
    else return *q;
}
template <bool NT> GDN_DEV void store_u2(void *p, u32x2_t v) {
    u32x2_t *q = reinterpret_cast<u32x2_t *>(p);
    if constexpr (NT) __builtin_nontemporal_store(v, q);
    else *q = v;
}
template <bool NT> GDN_DEV u32x4_t load_u4(const void *p) {
    const u32x4_t *q = reinterpret_cast<const u32x4_t *>(p);
    if constexpr (NT) return __builtin_nontemporal_load(q);
    else return *q;
}
template <bool NT> GDN_DEV void store_u4(void *p, u32x4_t v) {
    u32x4_t *q = reinterpret_cast<u32x4_t *>(p);
    if constexpr (NT) __builtin_nontemporal_store(v, q);
    else *q = v;
}

// ---- device-wide hand-off between the blocks of one launch -----------------
// The "last block finishes the reduction" pattern.  An agent-scope fence
// (__threadfence) writes back and invalidates this XCD's whole L2 on gfx950,
// so the data that crosses blocks travels by agent-scope relaxed atomics
// instead (stores written through, loads from the coherence point): a block
// stores its partials with store_agent, waits for their acknowledgement
// (stores_done), then bumps the counter with an agent-scope
// atomic; the block that sees the last count reads every partial with
// load_agent.  Ordinary loads and stores keep their caches.
GDN_DEV void store_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GDN_DEV void store_agent(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
GDN_DEV float load_agent(float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GDN_DEV uint64_t load_agent(uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// This wave's stores acknowledged before what follows (a workgroup-scope
// release emits no wait for global stores on gfx950, an agent-scope one
// writes back the L2).
GDN_DEV void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Increment the counter; true for the caller that brings it to `total` (it
// also returns the counter to 0 for the next launch).
GDN_DEV bool arrive_last(uint32_t *cnt, uint32_t total) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old != total - 1) return false;
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

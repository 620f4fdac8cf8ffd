// Device-side helpers shared by the trit_hip kernels (gfx950, wave64).
// Every fused multiply-add is an explicit __builtin_fmaf: the library is
// built with -ffp-contract=off so that every other product and sum rounds
// on its own, as Trit's Rust code does.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace trit {

constexpr int WAVE = 64;

__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, 2);
    return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_f16(float v) {
    _Float16 h = (_Float16)v;
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    return bits;
}

// f32 -> f16 (nearest even) -> f32, as Trit stores Q8_0 scales
// (src/cpu/tensors.rs:542-595).
__device__ __forceinline__ float f16_round(float v) { return (float)(_Float16)v; }

// Cephes expf with the steps of Trit's fused paths
// (src/cpu/activation.rs:8-38,357-375; src/cpu/v2/activation.rs:45-56).
__device__ __forceinline__ float exp_trit(float x) {
    constexpr float LOG2E = 1.44269504088896340736f;
    constexpr float LN2_HI = 0.693359375f;
    constexpr float LN2_LO = -2.12194440e-4f;
    x = __builtin_fminf(__builtin_fmaxf(x, -87.3f), 88.0f);
    int n_int = (int)__builtin_rintf(x * LOG2E);
    float n = (float)n_int;
    float r = __builtin_fmaf(-n, LN2_HI, x);
    r = __builtin_fmaf(-n, LN2_LO, r);
    float p = 1.9875691e-4f;
    p = __builtin_fmaf(p, r, 1.3981999e-3f);
    p = __builtin_fmaf(p, r, 8.333452e-3f);
    p = __builtin_fmaf(p, r, 4.1665796e-2f);
    p = __builtin_fmaf(p, r, 0.16666665f);
    p = __builtin_fmaf(p, r, 0.5f);
    float y = __builtin_fmaf(p, r * r, r + 1.0f);
    return y * __builtin_bit_cast(float, (uint32_t)(n_int + 127) << 23);
}

// v / (1 + exp(0 - v)) (src/cpu/activation.rs:54-56,330).
__device__ __forceinline__ float silu_trit(float v) { return v / (1.0f + exp_trit(0.0f - v)); }

// The exact GELU in the fused form of every Trit path (src/cpu/v2/
// activation.rs:33-39): v * erfc(-v / sqrt 2) / 2 with Numerical Recipes'
// erfcc, erfc(z) = t * exp(-z^2 + P(t)), t = 1 / (1 + z / 2)
// (src/cpu/activation.rs:15-28).
__device__ __forceinline__ float gelu_trit(float v) {
    const float z = __builtin_fabsf(v) * 0.70710678118654752440f;
    const float t = 1.0f / __builtin_fmaf(z, 0.5f, 1.0f);
    float p = 0.17087277f;
    p = __builtin_fmaf(p, t, -0.82215223f);
    p = __builtin_fmaf(p, t, 1.4885159f);
    p = __builtin_fmaf(p, t, -1.135204f);
    p = __builtin_fmaf(p, t, 0.27886807f);
    p = __builtin_fmaf(p, t, -0.18628806f);
    p = __builtin_fmaf(p, t, 0.09678418f);
    p = __builtin_fmaf(p, t, 0.37409196f);
    p = __builtin_fmaf(p, t, 1.0000237f);
    p = __builtin_fmaf(p, t, -1.2655122f);
    const float tail = t * exp_trit(__builtin_fmaf(-z, z, p));
    return (0.5f * v) * (v >= 0.0f ? 2.0f - tail : tail);
}

// Activation code: round to nearest even, then the +-127 limits; a NaN
// becomes -127 as cvtps2dq + clamp gives it (src/cpu/v2/quantize.rs:140-149).
__device__ __forceinline__ int act_code(float scaled) {
    float r = __builtin_rintf(scaled);
    r = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Global-memory views of device pointers. A pointer the compiler cannot
// trace to a kernel argument (one read from a table in memory) is generic
// to it, and its accesses become flat instructions; a flat load also holds
// the LDS wait counter, so every later LDS read would wait for it too (a
// weight stream in flight would stall each LDS access). Accesses through
// these views are global instructions.
#define TRIT_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const TRIT_GLOBAL T* gmem(const T* p) {
    return (const TRIT_GLOBAL T*)p;
}
template <class T>
__device__ __forceinline__ TRIT_GLOBAL T* gmem(T* p) {
    return (TRIT_GLOBAL T*)p;
}

// 16-, 8- and 4-float loads through the global view (HIP's vector structs
// do not copy from another address space; the native vectors do).
__device__ __forceinline__ uint4 gload_u4(const void* p) {
    const u32x4 v = *(const TRIT_GLOBAL u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gload_u2(const void* p) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = *(const TRIT_GLOBAL u32x2*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float4 gload_f4(const void* p) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = *(const TRIT_GLOBAL f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float2 gload_f2(const void* p) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = *(const TRIT_GLOBAL f32x2*)p;
    return make_float2(v.x, v.y);
}

// A 16-byte load of streamed weights (read once per token): nontemporal,
// so it does not displace the activations in the caches.
__device__ __forceinline__ uint4 load_stream(const void* p) {
    const u32x4 v = __builtin_nontemporal_load((const TRIT_GLOBAL u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// DPP lane moves (gfx9 encodings): quad_perm [1,0,3,2] (xor 1), [2,3,0,1]
// (xor 2), row_half_mirror (lane i <-> 7-i in each 8), row_mirror (i <->
// 15-i in each 16), row_ror:2 (lane i takes lane i-2 in its row of 16).
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140, DPP_ROR2 = 0x122,
             DPP_ROR8 = 0x128,
             // row_newbcast:n (0x150 + n): every lane of a 16-lane row reads lane n of that row.
             DPP_ROW_BCAST0 = 0x150 };

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Lane n of each 16-lane row, in every lane of that row (row_newbcast).
// n must fold to a constant (an index of an unrolled loop).
__device__ __forceinline__ float row_bcast(float v, int n) {
    switch (n & 15) {
        case 0: return dpp<DPP_ROW_BCAST0 + 0>(v);
        case 1: return dpp<DPP_ROW_BCAST0 + 1>(v);
        case 2: return dpp<DPP_ROW_BCAST0 + 2>(v);
        case 3: return dpp<DPP_ROW_BCAST0 + 3>(v);
        case 4: return dpp<DPP_ROW_BCAST0 + 4>(v);
        case 5: return dpp<DPP_ROW_BCAST0 + 5>(v);
        case 6: return dpp<DPP_ROW_BCAST0 + 6>(v);
        case 7: return dpp<DPP_ROW_BCAST0 + 7>(v);
        case 8: return dpp<DPP_ROW_BCAST0 + 8>(v);
        case 9: return dpp<DPP_ROW_BCAST0 + 9>(v);
        case 10: return dpp<DPP_ROW_BCAST0 + 10>(v);
        case 11: return dpp<DPP_ROW_BCAST0 + 11>(v);
        case 12: return dpp<DPP_ROW_BCAST0 + 12>(v);
        case 13: return dpp<DPP_ROW_BCAST0 + 13>(v);
        case 14: return dpp<DPP_ROW_BCAST0 + 14>(v);
        default: return dpp<DPP_ROW_BCAST0 + 15>(v);
    }
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

}  // namespace trit

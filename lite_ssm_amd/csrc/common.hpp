// common.hpp — device types, conversions and wave-level helpers for gfx950.
//
// Activations live in HBM as fp16 (the reference's only activation type,
// shaders/common.metal:4-9), bf16 or fp32; all math is fp32.  Rounding to the
// storage type is round-to-nearest-even, the same as the reference's half()
// conversions.  Wavefronts are 64 lanes wide.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lssm.h"

namespace lssm {

using f16 = _Float16;
using bf16 = __bf16;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;

__device__ __forceinline__ float to_f(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f(bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f(float v) { return v; }

template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }
// fp32 -> fp16 rounds the fp32 value as it stands (the reference computes in
// float and converts to half).  The empty asm keeps the compiler from folding
// the conversion into the multiply or FMA that produced v: the mixed-precision
// FMA it would use rounds the exact result straight to fp16, which differs in
// rare ties from rounding to fp32 first.
template <> __device__ __forceinline__ f16 from_f<f16>(float v) {
    asm("" : "+v"(v));
    return (f16)v;
}

// r(): round to the storage type and back.
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f(from_f<T>(v)); }

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }
// SiLU with the hardware exp and reciprocal (about 1 ulp each): the reference
// kernels are built with fast math (CMakeLists.txt:122), so this is within
// their own rounding; used in decode epilogues where the full-precision
// division is a measurable share of the instructions.
__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}
__device__ __forceinline__ float softplus_f(float v) { return (v > 20.0f) ? v : logf(1.0f + expf(v)); }

// Value of the 16-bit pattern b of a T (fp16 or bf16).
template <typename T> __device__ __forceinline__ float f_of_bits(uint16_t b) {
    return to_f(__builtin_bit_cast(T, b));
}

__device__ __forceinline__ float fp16_bits_to_f(uint16_t b) {
    union { uint16_t u; f16 h; } c;
    c.u = b;
    return (float)c.h;
}

// Lane sums without LDS round trips: DPP within 16-lane rows (quad perms,
// half-row and row mirrors), then the gfx950 row-swap permutes across rows.
// Every step adds two partial sums that some other lane adds in the other
// order (fp32 addition commutes), so all lanes of a group end with the same
// bits, and the order of the additions is fixed (deterministic).
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swap_add16(float v) {           // rows 2j, 2j+1
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float swap_add32(float v) {           // lane halves
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Inclusive prefix sum over the 64 lanes of a wave, in a fixed order: within
// each 16-lane row by DPP row shifts (1, 2, 4, 8), then across rows by the
// row broadcasts of lanes 15 (into rows 1 and 3) and 31 (into rows 2 and 3).
// Lanes and rows without a source add 0.
template <int CTRL, int ROWS> __device__ __forceinline__ float dpp_rows0(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, true));
}
__device__ __forceinline__ float wave_prefix_sum(float v) {
    v += dpp_rows0<0x111, 0xF>(v);   // row_shr:1
    v += dpp_rows0<0x112, 0xF>(v);   // row_shr:2
    v += dpp_rows0<0x114, 0xF>(v);   // row_shr:4
    v += dpp_rows0<0x118, 0xF>(v);   // row_shr:8
    v += dpp_rows0<0x142, 0xA>(v);   // row_bcast:15
    v += dpp_rows0<0x143, 0xC>(v);   // row_bcast:31
    return v;
}

// Value of lane `l` (wave-uniform) of v, as bits: the builtin takes an int,
// and a float argument would be converted by value.
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// softplus with the hardware exp and log (about 1 ulp each; the reference's
// kernels are built with fast math, CMakeLists.txt:122)
__device__ __forceinline__ float softplus_fast(float v) {
    return (v > 20.0f) ? v : __logf(1.0f + __expf(v));
}

// Sum over aligned groups of `W` lanes (W a power of two <= 64); the result in
// every lane of the group.
template <int W> __device__ __forceinline__ float group_sum(float v) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group");
    if constexpr (W >= 2) v += dpp_f32<0xB1>(v);                 // quad_perm 1,0,3,2
    if constexpr (W >= 4) v += dpp_f32<0x4E>(v);                 // quad_perm 2,3,0,1
    if constexpr (W >= 8) v += dpp_f32<0x141>(v);                // row_half_mirror
    if constexpr (W >= 16) v += dpp_f32<0x140>(v);               // row_mirror
    if constexpr (W >= 32) v = swap_add16(v);
    if constexpr (W >= 64) v = swap_add32(v);
    return v;
}

// Half-word index of element (m, k) of x in the single-pass MFMA decode
// GEMV's fragment order (int4 group 64 x bf16; quads = K / 128): octet k / 8 =
// 16 qa + 4 ch + p4 of row m is the 16 bytes lane 16 lg + m % 16 supplies to
// k-slice sl = 2 (ch >> 1) + (p4 & 1) of quad qa, lg = (ch & 1) + 2 (p4 >> 1),
// at 16-byte unit ((m / 16) quads + qa) 4 + sl) 64 + 16 lg + m % 16; inside
// it the octet's elements sit as pairs (0, 2), (4, 6), (1, 3), (5, 7).
__device__ __forceinline__ size_t frag_half(uint32_t m, uint32_t k, uint32_t quads) {
    const uint32_t cc = k / 8, e = k % 8, qa = cc / 16, ch = (cc % 16) / 4, p4 = cc % 4;
    const uint32_t sl = 2 * (ch >> 1) + (p4 & 1), lg = (ch & 1) + 2 * (p4 >> 1);
    const size_t u = (((size_t)(m / 16) * quads + qa) * 4 + sl) * 64 + 16 * lg + m % 16;
    return u * 8 + (((e & 1) << 1) | (e >> 2)) * 2 + ((e >> 1) & 1);
}

// Sum over a full 64-lane wave; result in every lane.
__device__ __forceinline__ float wave_sum(float v) { return group_sum<WAVE>(v); }

// sampler.cpp:13-21: first index of the maximum.  (v, i) beats (v', i') iff
// v > v' or (v == v' and i < i'); a NaN never wins.
__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Block-wide sum for blockDim.x == NT threads; `red` is >= NT/64 floats of LDS.
template <int NT> __device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / WAVE;
    if ((threadIdx.x % WAVE) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / WAVE; ++i) t += red[i];
    __syncthreads();
    return t;
}

}  // namespace lssm

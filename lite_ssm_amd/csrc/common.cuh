// common.cuh — device types, conversions and wave-level helpers for gfx950.
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

// Sum over a full 64-lane wave; result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
}

// Sum over aligned groups of `W` lanes (W a power of two <= 64).
template <int W> __device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
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

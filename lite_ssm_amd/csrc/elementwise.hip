// elementwise.hip — RMSNorm, gated RMSNorm, SiLU family, depthwise causal
// conv1d (prefill / decode update / state seed), embedding gather, argmax.
//
// Arithmetic follows shaders/norm.metal:52-79, activations.metal:12-87 and
// conv1d.metal:35-137; storage is fp16 / bf16 / fp32, math fp32.
#include <cfloat>
#include <initializer_list>
#include <utility>

#include "common.hpp"
#include "internal.hpp"

namespace lssm {

#define LSSM_DISPATCH_ACT(act, T, ...)                   \
    do {                                                 \
        if ((act) == LSSM_F16) {                         \
            using T = f16;                               \
            __VA_ARGS__;                                 \
        } else if ((act) == LSSM_BF16) {                 \
            using T = bf16;                              \
            __VA_ARGS__;                                 \
        } else {                                         \
            using T = float;                             \
            __VA_ARGS__;                                 \
        }                                                \
    } while (0)

// 8 fp16 / bf16 values in a 16-byte vector register.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
template <typename T> __device__ __forceinline__ float el8(v4u v, int e) {
    const uint32_t d = v[e / 2];
    return f_of_bits<T>((uint16_t)((e & 1) ? (d >> 16) : (d & 0xFFFF)));
}
template <typename T> __device__ __forceinline__ uint32_t bits_t(float f) {
    return __builtin_bit_cast(uint16_t, from_f<T>(f));
}
template <typename T> __device__ __forceinline__ v4u pack8(const float (&f)[8]) {
    v4u r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = bits_t<T>(f[2 * i]) | (bits_t<T>(f[2 * i + 1]) << 16);
    return r;
}

constexpr int NT = 256;

// norm.metal:52-79 — one block per row; y = r(x*w*rsqrt(mean(x^2)+eps)).
template <typename T>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(const T* __restrict__ x, uint32_t xs,
                                                     const T* __restrict__ w, T* __restrict__ y,
                                                     uint32_t ys, uint32_t dim, float eps) {
    __shared__ float red[NT / WAVE];
    const T* xr = x + (size_t)blockIdx.x * xs;
    T* yr = y + (size_t)blockIdx.x * ys;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += NT) {
        float v = to_f(xr[i]);
        ss += v * v;
    }
    ss = block_sum<NT>(ss, red);
    const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dim; i += NT) yr[i] = from_f<T>(to_f(xr[i]) * to_f(w[i]) * rrms);
}

// activations.metal:76-87 then norm.metal:52-79 (gate-then-norm,
// mamba2_block.cpp:230-238): g = r(silu(z)*y); out = r(g*w*rsqrt(mean g^2+eps)).
template <typename T>
__global__ __launch_bounds__(NT) void gated_rmsnorm_kernel(const T* __restrict__ z, uint32_t zs,
                                                           const T* __restrict__ yv, uint32_t yst,
                                                           const T* __restrict__ w,
                                                           T* __restrict__ out, uint32_t dim,
                                                           float eps) {
    __shared__ float red[NT / WAVE];
    const T* zr = z + (size_t)blockIdx.x * zs;
    const T* yr = yv + (size_t)blockIdx.x * yst;
    T* o = out + (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dim; i += NT) {
        float g = rnd<T>(silu_f(to_f(zr[i])) * to_f(yr[i]));
        ss += g * g;
    }
    ss = block_sum<NT>(ss, red);
    const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dim; i += NT) {
        float g = rnd<T>(silu_f(to_f(zr[i])) * to_f(yr[i]));
        o[i] = from_f<T>(g * to_f(w[i]) * rrms);
    }
}

// Vectorized norms: one wave per row, 8 elements (16 bytes) per lane per
// chunk, the row held in registers between the sum of squares and the
// scaled store, so every input is read once.  NCH = chunks of 512 elements
// per row (dim <= 512 NCH).  Same arithmetic as the kernels above; the SiLU
// of the gate uses the hardware exp / reciprocal (the reference builds its
// kernels with fast math).
template <typename T, int NCH>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const T* __restrict__ x, uint32_t xs,
                                                          const T* __restrict__ w, T* __restrict__ y,
                                                          uint32_t ys, uint32_t rows, uint32_t dim,
                                                          float eps) {
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (row >= rows) return;
    const uint32_t lane = threadIdx.x % WAVE;
    const T* xr = x + (size_t)row * xs;
    v4u xv[NCH];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t i = (c * WAVE + lane) * 8;
        xv[c] = i < dim ? *reinterpret_cast<const v4u*>(xr + i) : v4u{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = el8<T>(xv[c], e);
            ss += v * v;
        }
    }
    ss = wave_sum(ss);
    const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
    T* yr = y + (size_t)row * ys;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t i = (c * WAVE + lane) * 8;
        if (i >= dim) break;
        const v4u wv = *reinterpret_cast<const v4u*>(w + i);
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = el8<T>(xv[c], e) * el8<T>(wv, e) * rrms;
        *reinterpret_cast<v4u*>(yr + i) = pack8<T>(o);
    }
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void gated_rmsnorm_wave_kernel(
    const T* __restrict__ z, uint32_t zs, const T* __restrict__ yv, uint32_t yst,
    const T* __restrict__ w, T* __restrict__ out, uint32_t rows, uint32_t dim, float eps) {
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / WAVE;
    if (row >= rows) return;
    const uint32_t lane = threadIdx.x % WAVE;
    const T* zr = z + (size_t)row * zs;
    const T* yr = yv + (size_t)row * yst;
    v4u zv[NCH], yy[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t i = (c * WAVE + lane) * 8;
        zv[c] = i < dim ? *reinterpret_cast<const v4u*>(zr + i) : v4u{0, 0, 0, 0};
        yy[c] = i < dim ? *reinterpret_cast<const v4u*>(yr + i) : v4u{0, 0, 0, 0};
    }
    v4u gv[NCH];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        float g[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            g[e] = rnd<T>(silu_fast(el8<T>(zv[c], e)) * el8<T>(yy[c], e));
            ss += g[e] * g[e];
        }
        gv[c] = pack8<T>(g);
    }
    ss = wave_sum(ss);
    const float rrms = 1.0f / sqrtf(ss / (float)dim + eps);
    T* o = out + (size_t)row * dim;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t i = (c * WAVE + lane) * 8;
        if (i >= dim) break;
        const v4u wv = *reinterpret_cast<const v4u*>(w + i);
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = el8<T>(gv[c], e) * el8<T>(wv, e) * rrms;
        *reinterpret_cast<v4u*>(o + i) = pack8<T>(r);
    }
}

template <typename T>
__global__ void silu_kernel(const T* __restrict__ x, T* __restrict__ y, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = from_f<T>(silu_f(to_f(x[i])));
}

template <typename T>
__global__ void add_kernel(T* y, const T* __restrict__ x, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = from_f<T>(to_f(y[i]) + to_f(x[i]));
}

template <typename T>
__global__ void silu_gated_kernel(const T* __restrict__ x, const T* __restrict__ g,
                                  T* __restrict__ y, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = from_f<T>(silu_f(to_f(x[i])) * to_f(g[i]));
}

// activations.metal:49-73
template <typename T>
__global__ void split_silu_kernel(const T* __restrict__ xBC, T* __restrict__ xo,
                                  T* __restrict__ Bo, T* __restrict__ Co, uint32_t rows,
                                  uint32_t d_inner, uint32_t GN) {
    const uint32_t dim = d_inner + 2u * GN;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * dim) return;
    uint32_t t = (uint32_t)(i / dim), f = (uint32_t)(i % dim);
    T v = from_f<T>(silu_f(to_f(xBC[i])));
    if (f < d_inner) xo[(size_t)t * d_inner + f] = v;
    else if (f < d_inner + GN) Bo[(size_t)t * GN + (f - d_inner)] = v;
    else Co[(size_t)t * GN + (f - d_inner - GN)] = v;
}

// conv1d.metal:63-93 — y[b,t,d] = r(bias + sum_tap w[d,tap] x[b,t-(K-1-tap),d]),
// zero left padding.  SILU additionally applies r(silu(.)) to the rounded conv
// output (the split_silu pass fused in).
template <typename T, bool SILU>
__global__ void conv1d_kernel(const T* __restrict__ x, uint32_t xs, const T* __restrict__ w,
                              const T* __restrict__ bias, T* __restrict__ y, uint32_t ys,
                              uint32_t L, uint32_t D, uint32_t K, const T* __restrict__ hist) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t t = blockIdx.y;
    const uint32_t b = blockIdx.z;
    if (d >= D) return;
    const size_t row0 = (size_t)b * L;
    float acc = bias ? to_f(bias[d]) : 0.0f;
    for (uint32_t tap = 0; tap < K; ++tap) {
        int src = (int)t - (int)(K - 1 - tap);
        float v = 0.0f;
        if (src >= 0) v = to_f(x[(row0 + (uint32_t)src) * xs + d]);
        else if (hist) v = to_f(hist[(size_t)d * K + (K + src)]);   // the sequence's earlier rows
        acc += to_f(w[(size_t)d * K + tap]) * v;
    }
    float o = rnd<T>(acc);
    if (SILU) o = silu_f(o);
    y[(row0 + t) * ys + d] = from_f<T>(o);
}

// Vector form of conv1d_kernel for 2-byte dtypes and K == 4: a thread owns 8
// consecutive channels (16-byte loads and stores) and CT consecutive time
// steps, with the CT + 3 input rows it needs held in registers, so every
// input row is read once per thread (not once per tap) and the taps and
// bias once per thread.  Same sums in the same order as conv1d_kernel.
constexpr int CONV_CT = 16;

template <typename T, bool SILU>
__global__ __launch_bounds__(256) void conv1d_vec_kernel(const T* __restrict__ x, uint32_t xs,
                                                         const T* __restrict__ w,
                                                         const T* __restrict__ bias,
                                                         T* __restrict__ y, uint32_t ys, uint32_t L,
                                                         uint32_t D, const T* __restrict__ hist) {
  if constexpr (sizeof(T) == 2) {                    // launched for fp16 / bf16 only
    const uint32_t d0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (d0 >= D) return;
    const uint32_t t0 = blockIdx.y * CONV_CT;
    const uint32_t b = blockIdx.z;
    const T* xb = x + (size_t)b * L * xs + d0;
    // the window as vector registers; elements are taken out by shifts (an
    // element address would put the array in scratch memory)
    v4u win[CONV_CT + 3];
#pragma unroll
    for (int i = 0; i < CONV_CT + 3; ++i) {
        const int t = (int)t0 + i - 3;
        win[i] = (t >= 0 && t < (int)L) ? *reinterpret_cast<const v4u*>(xb + (size_t)t * xs)
                                        : v4u{0, 0, 0, 0};
    }
    // rows before the first (t0 == 0 only): the sequence's earlier rows, the
    // last K entries of each channel's conv state (entry K + t for row t < 0)
    if (hist && t0 == 0) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            uint32_t h[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint16_t lo = __builtin_bit_cast(uint16_t, hist[(size_t)(d0 + 2 * q) * 4 + 1 + i]);
                const uint16_t hi = __builtin_bit_cast(uint16_t, hist[(size_t)(d0 + 2 * q + 1) * 4 + 1 + i]);
                h[q] = (uint32_t)lo | ((uint32_t)hi << 16);
            }
            win[i] = v4u{h[0], h[1], h[2], h[3]};
        }
    }
    // taps w[d][0..3] of the 8 channels: 64 contiguous bytes
    float wf[8][4], bf[8];
    {
        const v4u* w4 = reinterpret_cast<const v4u*>(w + (size_t)d0 * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4u v = w4[q];
#pragma unroll
            for (int e = 0; e < 8; ++e) wf[2 * q + e / 4][e % 4] = el8<T>(v, e);
        }
        const v4u bv = bias ? *reinterpret_cast<const v4u*>(bias + d0) : v4u{0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 8; ++c) bf[c] = el8<T>(bv, c);
    }
    T* yb = y + ((size_t)b * L + t0) * ys + d0;
#pragma unroll
    for (int i = 0; i < CONV_CT; ++i) {
        float o[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float acc = bf[c];
#pragma unroll
            for (int tap = 0; tap < 4; ++tap) acc = fmaf(wf[c][tap], el8<T>(win[i + tap], c), acc);
            o[c] = rnd<T>(acc);
            if (SILU) o[c] = silu_fast(o[c]);
        }
        if (t0 + i < L) *reinterpret_cast<v4u*>(yb + (size_t)i * ys) = pack8<T>(o);
    }
  }
}

// conv1d.metal:108-137 — shift the window left, append x, y = r(bias + sum s*w).
template <typename T>
__global__ void conv1d_update_kernel(const T* __restrict__ x_new, T* state, const T* __restrict__ w,
                                     const T* __restrict__ bias, T* __restrict__ y, uint32_t D,
                                     uint32_t K) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (d >= D) return;
    T* sd = state + ((size_t)b * D + d) * K;
    const T* wd = w + (size_t)d * K;
    for (uint32_t k = 0; k + 1 < K; ++k) sd[k] = sd[k + 1];
    sd[K - 1] = x_new[(size_t)b * D + d];
    float acc = bias ? to_f(bias[d]) : 0.0f;
    for (uint32_t k = 0; k < K; ++k) acc += to_f(sd[k]) * to_f(wd[k]);
    y[(size_t)b * D + d] = from_f<T>(acc);
}

// conv1d_update_kernel fused with SiLU, strided rows (engine decode, batch > 4):
// y = r(silu(r(bias + sum s*w))).
template <typename T>
__global__ void conv1d_update_silu_kernel(const T* __restrict__ x_new, uint32_t xs, T* state,
                                          const T* __restrict__ w, const T* __restrict__ bias,
                                          T* __restrict__ y, uint32_t ys, uint32_t D, uint32_t K) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (d >= D) return;
    T* sd = state + ((size_t)b * D + d) * K;
    const T* wd = w + (size_t)d * K;
    for (uint32_t k = 0; k + 1 < K; ++k) sd[k] = sd[k + 1];
    sd[K - 1] = x_new[(size_t)b * xs + d];
    float acc = bias ? to_f(bias[d]) : 0.0f;
    for (uint32_t k = 0; k < K; ++k) acc += to_f(sd[k]) * to_f(wd[k]);
    y[(size_t)b * ys + d] = from_f<T>(silu_f(rnd<T>(acc)));
}

// Zero all but the newest tap of each window (the seed of a 1-token prefill,
// conv1d.metal:45-50 with L = 1).
template <typename T>
__global__ void conv1d_keep_last_kernel(T* state, uint32_t n_windows, uint32_t K) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n_windows * (K - 1)) return;
    const size_t wdx = i / (K - 1), k = i % (K - 1);
    state[wdx * K + k] = from_f<T>(0.0f);
}

// conv1d.metal:35-51 — state[b,d,k] = xBC[b, L-K+k, d] or 0.
template <typename T>
__global__ void conv1d_seed_kernel(const T* __restrict__ xBC, uint32_t xs, T* __restrict__ state,
                                   uint32_t L, uint32_t D, uint32_t K) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (d >= D) return;
    for (uint32_t k = 0; k < K; ++k) {
        int src = (int)L - (int)K + (int)k;
        T v = from_f<T>(0.0f);
        if (src >= 0) v = xBC[((size_t)b * L + (uint32_t)src) * xs + d];
        state[((size_t)b * D + d) * K + k] = v;
    }
}

// mamba2_model.cpp:128-137 on device.  The ids live in device memory, so the
// range check of mamba2_model.cpp:129-131 happens here: an id outside
// [0, vocab) gives a zero row (the table is never read out of bounds) and sets
// STATUS_BAD_TOKEN in the context's status word, which the host turns into
// the reference's out_of_range error at its next synchronisation point.
template <typename T>
__global__ void embed_kernel(const T* __restrict__ table, const int32_t* __restrict__ ids,
                             T* __restrict__ out, uint32_t n, uint32_t d_model, uint32_t vocab,
                             uint32_t* __restrict__ status, uint32_t* __restrict__ seq) {
    if (seq != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *seq += 1u;
    const size_t total = (size_t)n * d_model;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const size_t i = e / d_model, c = e % d_model;
        const int32_t id = ids[i];
        const bool ok = id >= 0 && (uint32_t)id < vocab;
        out[e] = ok ? table[(size_t)id * d_model + c] : from_f<T>(0.0f);
        if (!ok && c == 0) atomicOr(status, STATUS_BAD_TOKEN);
    }
}

template <int NTHR>
__device__ __forceinline__ void block_argmax(float& bv, int& bi) {
    __shared__ float sv[NTHR / WAVE];
    __shared__ int si[NTHR / WAVE];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float ov = __shfl_xor(bv, off, WAVE);
        int oi = __shfl_xor(bi, off, WAVE);
        argmax_merge(bv, bi, ov, oi);
    }
    const int wv = threadIdx.x / WAVE;
    if ((threadIdx.x % WAVE) == 0) {
        sv[wv] = bv;
        si[wv] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int i = 1; i < NTHR / WAVE; ++i) argmax_merge(bv, bi, sv[i], si[i]);
    __syncthreads();
}

// Stage 1: block (blk, row) reduces a slice.  Stage 2 (or single pass when
// gridDim.x == 1) writes the id.
template <typename T, int NTHR>
__global__ __launch_bounds__(NTHR) void argmax_partial_kernel(const T* __restrict__ logits,
                                                              uint32_t vocab, float* pv, int* pi,
                                                              int32_t* ids) {
    const uint32_t row = blockIdx.y;
    const uint32_t per = (vocab + gridDim.x - 1) / gridDim.x;
    const uint32_t lo = blockIdx.x * per;
    const uint32_t hi = min(vocab, lo + per);
    const T* lr = logits + (size_t)row * vocab;
    float bv = -FLT_MAX;
    int bi = 0x7fffffff;
    for (uint32_t i = lo + threadIdx.x; i < hi; i += NTHR) argmax_merge(bv, bi, to_f(lr[i]), (int)i);
    block_argmax<NTHR>(bv, bi);
    if (threadIdx.x == 0) {
        if (gridDim.x == 1) {
            ids[row] = (bi == 0x7fffffff) ? 0 : bi;
        } else {
            pv[(size_t)row * gridDim.x + blockIdx.x] = bv;
            pi[(size_t)row * gridDim.x + blockIdx.x] = bi;
        }
    }
}

// nblk_dev (optional): the partial count, written by the kernel before (the
// lm_head GEMV's argmax epilogue writes one partial per block of its grid).
__global__ __launch_bounds__(256) void argmax_final_kernel(const float* pv, const int* pi,
                                                           uint32_t nblk, const uint32_t* nblk_dev,
                                                           int32_t* ids) {
    const uint32_t row = blockIdx.x;
    if (nblk_dev) nblk = *nblk_dev;
    float bv = -FLT_MAX;
    int bi = 0x7fffffff;
    for (uint32_t i = threadIdx.x; i < nblk; i += 256)
        argmax_merge(bv, bi, pv[(size_t)row * nblk + i], pi[(size_t)row * nblk + i]);
    block_argmax<256>(bv, bi);
    if (threadIdx.x == 0) ids[row] = (bi == 0x7fffffff) ? 0 : bi;
}

// Greedy-id history of a decode run (runtime/inference.cpp:55-67 collects the
// generated ids into a vector): row `*pos` of log [cap][B] gets this step's
// ids, then *pos advances.  Every thread reads *pos before the barrier and
// thread 0 writes it after, so the block sees one value.  Steps past `cap`
// are counted and not stored.
__global__ __launch_bounds__(64) void id_log_kernel(const int32_t* __restrict__ next, uint32_t B,
                                                    int32_t* __restrict__ log, uint32_t cap,
                                                    uint32_t* __restrict__ pos) {
    const uint32_t p = *pos;
    __syncthreads();
    if (threadIdx.x < B && p < cap) log[(size_t)p * B + threadIdx.x] = next[threadIdx.x];
    if (threadIdx.x == 0) *pos = p + 1u;
}

static inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Chunks of 512 elements per row for the wave-per-row norms (0 = use the
// block-per-row kernels): 16-byte aligned rows of fp16 / bf16, dim <= 8192.
static int norm_chunks(int act, uint32_t dim, std::initializer_list<std::pair<const void*, uint32_t>> rows_) {
    if (act == LSSM_F32 || dim % 8 != 0 || dim > 8192) return 0;
    for (auto& r : rows_)
        if ((uintptr_t)r.first % 16 != 0 || r.second % 8 != 0) return 0;
    const uint32_t n = (dim + 511) / 512;
    return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : n <= 8 ? 8 : 16;
}

#define LSSM_NCH_DISPATCH(nch, NCH, ...)                            \
    switch (nch) {                                                  \
        case 1: { constexpr int NCH = 1; __VA_ARGS__; break; }      \
        case 2: { constexpr int NCH = 2; __VA_ARGS__; break; }      \
        case 4: { constexpr int NCH = 4; __VA_ARGS__; break; }      \
        case 8: { constexpr int NCH = 8; __VA_ARGS__; break; }      \
        default: { constexpr int NCH = 16; __VA_ARGS__; break; }    \
    }

hipError_t launch_rmsnorm(hipStream_t s, const void* x, uint32_t xs, const void* w, void* y,
                          uint32_t ys, uint32_t rows, uint32_t dim, float eps, int act) {
    if (rows == 0) return hipSuccess;
    if (const int nch = norm_chunks(act, dim, {{x, xs}, {w, 8}, {y, ys}})) {
        if (act == LSSM_F16) {
            LSSM_NCH_DISPATCH(nch, NCH, rmsnorm_wave_kernel<f16, NCH><<<cdiv(rows, 4), 256, 0, s>>>(
                (const f16*)x, xs, (const f16*)w, (f16*)y, ys, rows, dim, eps));
        } else {
            LSSM_NCH_DISPATCH(nch, NCH, rmsnorm_wave_kernel<bf16, NCH><<<cdiv(rows, 4), 256, 0, s>>>(
                (const bf16*)x, xs, (const bf16*)w, (bf16*)y, ys, rows, dim, eps));
        }
        return hipGetLastError();
    }
    LSSM_DISPATCH_ACT(act, T,
                      rmsnorm_kernel<T><<<rows, NT, 0, s>>>((const T*)x, xs, (const T*)w, (T*)y, ys,
                                                            dim, eps));
    return hipGetLastError();
}

hipError_t launch_gated_rmsnorm(hipStream_t s, const void* z, uint32_t zs, const void* y,
                                uint32_t yst, const void* w, void* out, uint32_t rows, uint32_t dim,
                                float eps, int act) {
    if (rows == 0) return hipSuccess;
    if (const int nch = norm_chunks(act, dim, {{z, zs}, {y, yst}, {w, 8}, {out, dim}})) {
        if (act == LSSM_F16) {
            LSSM_NCH_DISPATCH(nch, NCH, gated_rmsnorm_wave_kernel<f16, NCH><<<cdiv(rows, 4), 256, 0, s>>>(
                (const f16*)z, zs, (const f16*)y, yst, (const f16*)w, (f16*)out, rows, dim, eps));
        } else {
            LSSM_NCH_DISPATCH(nch, NCH, gated_rmsnorm_wave_kernel<bf16, NCH><<<cdiv(rows, 4), 256, 0, s>>>(
                (const bf16*)z, zs, (const bf16*)y, yst, (const bf16*)w, (bf16*)out, rows, dim, eps));
        }
        return hipGetLastError();
    }
    LSSM_DISPATCH_ACT(act, T,
                      gated_rmsnorm_kernel<T><<<rows, NT, 0, s>>>((const T*)z, zs, (const T*)y, yst,
                                                                  (const T*)w, (T*)out, dim, eps));
    return hipGetLastError();
}

hipError_t launch_silu(hipStream_t s, const void* x, void* y, uint32_t n, int act) {
    if (n == 0) return hipSuccess;
    LSSM_DISPATCH_ACT(act, T, silu_kernel<T><<<cdiv(n, NT), NT, 0, s>>>((const T*)x, (T*)y, n));
    return hipGetLastError();
}

hipError_t launch_add(hipStream_t s, void* y, const void* x, uint32_t n, int act) {
    if (n == 0) return hipSuccess;
    LSSM_DISPATCH_ACT(act, T, add_kernel<T><<<cdiv(n, NT), NT, 0, s>>>((T*)y, (const T*)x, n));
    return hipGetLastError();
}

hipError_t launch_silu_gated(hipStream_t s, const void* x, const void* g, void* y, uint32_t n,
                             int act) {
    if (n == 0) return hipSuccess;
    LSSM_DISPATCH_ACT(act, T,
                      silu_gated_kernel<T><<<cdiv(n, NT), NT, 0, s>>>((const T*)x, (const T*)g,
                                                                      (T*)y, n));
    return hipGetLastError();
}

hipError_t launch_split_silu(hipStream_t s, const void* xBC, void* x, void* B, void* C,
                             uint32_t rows, uint32_t d_inner, uint32_t GN, int act) {
    size_t n = (size_t)rows * (d_inner + 2u * GN);
    if (n == 0) return hipSuccess;
    LSSM_DISPATCH_ACT(act, T,
                      split_silu_kernel<T><<<cdiv(n, NT), NT, 0, s>>>((const T*)xBC, (T*)x, (T*)B,
                                                                      (T*)C, rows, d_inner, GN));
    return hipGetLastError();
}

hipError_t launch_conv1d(hipStream_t s, const void* x, uint32_t xs, const void* w, const void* bias,
                         void* y, uint32_t ys, uint32_t B, uint32_t L, uint32_t D, uint32_t K,
                         int act, bool silu, const void* hist) {
    if ((size_t)B * L * D == 0) return hipSuccess;
    if (hist && B != 1) return hipErrorInvalidValue;
    const bool vec = act != LSSM_F32 && K == 4 && D % 8 == 0 && xs % 8 == 0 && ys % 8 == 0 &&
                     (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && (uintptr_t)w % 16 == 0 &&
                     (bias == nullptr || (uintptr_t)bias % 16 == 0);
    if (vec) {
        dim3 gv(cdiv(D / 8, 256), cdiv(L, CONV_CT), B);
        if (silu) {
            LSSM_DISPATCH_ACT(act, T,
                              conv1d_vec_kernel<T, true><<<gv, 256, 0, s>>>((const T*)x, xs, (const T*)w,
                                                                            (const T*)bias, (T*)y, ys, L, D, (const T*)hist));
        } else {
            LSSM_DISPATCH_ACT(act, T,
                              conv1d_vec_kernel<T, false><<<gv, 256, 0, s>>>((const T*)x, xs, (const T*)w,
                                                                             (const T*)bias, (T*)y, ys, L, D, (const T*)hist));
        }
        return hipGetLastError();
    }
    dim3 grid(cdiv(D, NT), L, B);
    if (silu) {
        LSSM_DISPATCH_ACT(act, T,
                          conv1d_kernel<T, true><<<grid, NT, 0, s>>>((const T*)x, xs, (const T*)w,
                                                                     (const T*)bias, (T*)y, ys, L,
                                                                     D, K, (const T*)hist));
    } else {
        LSSM_DISPATCH_ACT(act, T,
                          conv1d_kernel<T, false><<<grid, NT, 0, s>>>((const T*)x, xs, (const T*)w,
                                                                      (const T*)bias, (T*)y, ys, L,
                                                                      D, K, (const T*)hist));
    }
    return hipGetLastError();
}

hipError_t launch_conv1d_update(hipStream_t s, const void* x_new, void* state, const void* w,
                                const void* bias, void* y, uint32_t B, uint32_t D, uint32_t K,
                                int act) {
    if ((size_t)B * D == 0) return hipSuccess;
    dim3 grid(cdiv(D, NT), B);
    LSSM_DISPATCH_ACT(act, T,
                      conv1d_update_kernel<T><<<grid, NT, 0, s>>>((const T*)x_new, (T*)state,
                                                                  (const T*)w, (const T*)bias,
                                                                  (T*)y, D, K));
    return hipGetLastError();
}

hipError_t launch_conv1d_seed(hipStream_t s, const void* xBC, uint32_t xs, void* state, uint32_t B,
                              uint32_t L, uint32_t D, uint32_t K, int act) {
    if ((size_t)B * D == 0) return hipSuccess;
    dim3 grid(cdiv(D, NT), B);
    LSSM_DISPATCH_ACT(act, T,
                      conv1d_seed_kernel<T><<<grid, NT, 0, s>>>((const T*)xBC, xs, (T*)state, L, D,
                                                                K));
    return hipGetLastError();
}

hipError_t launch_conv1d_update_silu(hipStream_t s, const void* x_new, uint32_t xs, void* state,
                                     const void* w, const void* bias, void* y, uint32_t ys,
                                     uint32_t B, uint32_t D, uint32_t K, int act) {
    if ((size_t)B * D == 0) return hipSuccess;
    dim3 grid(cdiv(D, NT), B);
    LSSM_DISPATCH_ACT(act, T,
                      conv1d_update_silu_kernel<T><<<grid, NT, 0, s>>>((const T*)x_new, xs, (T*)state,
                                                                       (const T*)w, (const T*)bias,
                                                                       (T*)y, ys, D, K));
    return hipGetLastError();
}

hipError_t launch_conv1d_keep_last(hipStream_t s, void* state, uint32_t n_windows, uint32_t K,
                                   int act) {
    const size_t n = (size_t)n_windows * (K - 1);
    if (n == 0) return hipSuccess;
    LSSM_DISPATCH_ACT(act, T,
                      conv1d_keep_last_kernel<T><<<cdiv(n, NT), NT, 0, s>>>((T*)state, n_windows, K));
    return hipGetLastError();
}

hipError_t launch_embed(hipStream_t s, const void* table, const int32_t* ids, void* out, uint32_t n,
                        uint32_t d_model, uint32_t vocab, int act, uint32_t* status, uint32_t* seq) {
    if (n == 0) return hipSuccess;
    const size_t total = (size_t)n * d_model;
    const unsigned blocks = (unsigned)((total + NT - 1) / NT < 65536 ? (total + NT - 1) / NT : 65536);
    LSSM_DISPATCH_ACT(act, T,
                      embed_kernel<T><<<blocks, NT, 0, s>>>((const T*)table, ids, (T*)out, n,
                                                            d_model, vocab, status, seq));
    return hipGetLastError();
}

// scratch == nullptr: single pass, one 1024-thread block per row.
// scratch != nullptr: 128 blocks per row, then a final pass; scratch must hold
// rows * 128 * (sizeof(float) + sizeof(int)) bytes.
hipError_t launch_argmax(hipStream_t s, const void* logits, int32_t* ids, uint32_t rows,
                         uint32_t vocab, int act, void* scratch) {
    if (rows == 0) return hipSuccess;
    if (!scratch) {
        LSSM_DISPATCH_ACT(act, T,
                          argmax_partial_kernel<T, 1024><<<dim3(1, rows), 1024, 0, s>>>(
                              (const T*)logits, vocab, nullptr, nullptr, ids));
        return hipGetLastError();
    }
    const uint32_t nblk = 128;
    float* pv = (float*)scratch;
    int* pi = (int*)(pv + (size_t)rows * nblk);
    LSSM_DISPATCH_ACT(act, T,
                      argmax_partial_kernel<T, 256><<<dim3(nblk, rows), 256, 0, s>>>(
                          (const T*)logits, vocab, pv, pi, ids));
    argmax_final_kernel<<<rows, 256, 0, s>>>(pv, pi, nblk, nullptr, ids);
    return hipGetLastError();
}

hipError_t launch_argmax_final(hipStream_t s, const float* pv, const int* pi, const uint32_t* nblk,
                               int32_t* ids) {
    argmax_final_kernel<<<1, 256, 0, s>>>(pv, pi, 0u, nblk, ids);
    return hipGetLastError();
}

hipError_t launch_id_log(hipStream_t s, const int32_t* next, uint32_t B, int32_t* log, uint32_t cap,
                         uint32_t* pos) {
    if (B == 0 || B > 64) return hipErrorInvalidValue;
    id_log_kernel<<<1, 64, 0, s>>>(next, B, log, cap, pos);
    return hipGetLastError();
}

}  // namespace lssm

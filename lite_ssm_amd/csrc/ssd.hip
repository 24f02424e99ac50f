// ssd.hip — Mamba-2 SSD: single-token step (decode) and chunked scan (prefill).
//
// Step (ssd_step.metal:33-77):  s = e^{A dt} s + dt B x  (fp32 state, in place);
//                               y = r(C.s + D x)
// Chunk (ssd_chunked.metal:82-297), per (sequence, head), chunks in order:
//   DT = clamp(softplus(dt_raw + dt_bias)),  Lcum = inclusive cumsum(A DT)
//   M[t,j] = r((C_t.B_j) e^{Lcum_t - Lcum_j} DT_j)   (j <= t)
//   y[t,p] = r(sum_j M[t,j] X[j,p] + e^{Lcum_t} C_t.S_p + D x[t,p])
//   S[p,n] = r(e^{L_end} S[p,n] + sum_j e^{L_end - Lcum_j} DT_j B[j,n] X[j,p])
// with S held in the activation dtype between chunks (the reference keeps it
// in `half` threadgroup memory) and written back as fp32.
#include <algorithm>
#include <cfloat>
#include <cstdlib>

#include "common.hpp"
#include "internal.hpp"

namespace lssm {

namespace {

// ---------------------------------------------------------------------------
// Decode step.  Block (h * PS + ps, b), one wave, owns 8 rows p of one head's
// (P, N) fp32 state: 8 lanes per row, each streaming F = N / 32 float4 of
// state.  Every load is issued first and unconditionally (state, the lane's B
// and C vectors, then the per-row / per-head scalars as raw bits), so nothing
// waits before the math; the 8 lanes of a row reduce C.s with shuffles.
// 2.7B at batch 1: 640 one-wave blocks (every CU streams part of the state;
// 256-thread blocks left 96 CUs idle and took 4.96 us instead of 4.08 us),
// 4 x 16-byte state loads per thread.
// ---------------------------------------------------------------------------
constexpr int ST_NV = 8;                              // lanes per state row
constexpr int ST_NT = 64;                             // threads per block (one wave)
constexpr int ST_RB = ST_NT / ST_NV;                  // rows per block

template <typename T> __device__ __forceinline__ uint32_t raw_of(const T* p) {
    if constexpr (sizeof(T) == 2) return *reinterpret_cast<const uint16_t*>(p);
    else return *reinterpret_cast<const uint32_t*>(p);
}
template <typename T> __device__ __forceinline__ float f_of(uint32_t r) {
    if constexpr (sizeof(T) == 2) return to_f(__builtin_bit_cast(T, (uint16_t)r));
    else return __uint_as_float(r);
}

// FRAG (bf16, gate; the decode batches whose out_proj normalises on load):
// blocks of four waves own 32 consecutive rows j = h P + p of the flattened
// (H, P) (H P a multiple of 128), write r(y w) (w = a.ynorm_w, the norm
// weight in front of out_proj) in the single-pass MFMA GEMV's fragment order
// (a.yfrag) and the 32 values' sum of squares of y to a.ypart[b][blockIdx.x].
template <typename T, int F, bool GATE, bool FRAG = false>
__global__ __launch_bounds__(FRAG ? 4 * ST_NT : ST_NT) void ssd_step_kernel(SsdArgs a) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint32_t P = a.P, N = a.N;
    const uint32_t b = blockIdx.y;
    uint32_t h, p;
    if constexpr (FRAG) {
        const uint32_t j = blockIdx.x * (4 * ST_RB) + threadIdx.x / ST_NV;
        h = j / P;
        p = j % P;
    } else {
        const uint32_t PS = (P + ST_RB - 1) / ST_RB;
        h = blockIdx.x / PS;
        p = (blockIdx.x % PS) * ST_RB + threadIdx.x / ST_NV;
        if (p >= P) return;                           // whole 8-lane row groups exit together
    }
    const uint32_t g = h / (a.H / a.G);
    const uint32_t lr = threadIdx.x % ST_NV;
    f32x4* S = reinterpret_cast<f32x4*>(a.state + (((size_t)b * a.H + h) * P + p) * N);
    const T4* B4 = reinterpret_cast<const T4*>((const T*)a.B + (size_t)b * a.b_stride + (size_t)g * N);
    const T4* C4 = reinterpret_cast<const T4*>((const T*)a.C + (size_t)b * a.c_stride + (size_t)g * N);
    f32x4 s[F];
    T4 bv[F], cv[F];
#pragma unroll
    for (int f = 0; f < F; ++f) s[f] = __builtin_nontemporal_load(&S[lr + ST_NV * f]);   // streamed once
#pragma unroll
    for (int f = 0; f < F; ++f) {
        bv[f] = B4[lr + ST_NV * f];
        cv[f] = C4[lr + ST_NV * f];
    }
    const T* Xp = (const T*)a.X + (size_t)b * a.x_stride + (size_t)h * P + p;
    const uint32_t xr = raw_of(Xp);
    const uint32_t zr = GATE ? raw_of((const T*)a.z + (size_t)b * a.z_stride + (size_t)h * P + p) : 0u;
    const uint32_t alr = raw_of((const T*)a.A_log + h);
    const uint32_t dtr = raw_of((const T*)a.dt + (size_t)b * a.dt_stride + h);
    const uint32_t dbr = raw_of((const T*)a.dt_bias + h);
    const uint32_t dr = raw_of(a.has_D ? (const T*)a.D + h : Xp);   // value unused without D
    [[maybe_unused]] const uint32_t nwr = FRAG ? raw_of((const T*)a.ynorm_w + h * P + p) : 0u;

    // dt = clamp(softplus(dt_raw + dt_bias)), decay = e^{A dt} (ssd_step.metal:55-66)
    const float xv = f_of<T>(xr);
    const float A_h = -expf(f_of<T>(alr));
    float dt = softplus_f(f_of<T>(dtr) + f_of<T>(dbr));
    dt = fminf(fmaxf(dt, a.dt_min), a.dt_max);
    const float decay = expf(A_h * dt);
    float ys = 0.0f;
#pragma unroll
    for (int f = 0; f < F; ++f) {
        // s = decay*s + (dt*B)*x  (ssd_step.metal:68-69)
        // the fused multiply-adds are spelled out: the batch-1 decode launch
        // that also runs this step (gemv.hip) must round identically
        f32x4 t = s[f];
        t.x = fmaf(decay, t.x, dt * to_f(bv[f].x) * xv);
        t.y = fmaf(decay, t.y, dt * to_f(bv[f].y) * xv);
        t.z = fmaf(decay, t.z, dt * to_f(bv[f].z) * xv);
        t.w = fmaf(decay, t.w, dt * to_f(bv[f].w) * xv);
        __builtin_nontemporal_store(t, &S[lr + ST_NV * f]);
        ys += fmaf(to_f(cv[f].w), t.w, fmaf(to_f(cv[f].z), t.z, fmaf(to_f(cv[f].x), t.x, to_f(cv[f].y) * t.y)));
    }
    ys = group_sum<ST_NV>(ys);
    float q = 0.0f;
    if (lr == 0) {
        float y = rnd<T>(fmaf(a.has_D ? f_of<T>(dr) : 0.0f, xv, ys));
        if constexpr (GATE) y = silu_fast(f_of<T>(zr)) * y;
        const T yr = from_f<T>(y);
        ((T*)a.Y)[(size_t)b * a.y_stride + (size_t)h * P + p] = yr;
        if constexpr (FRAG) {
            const float yv = to_f(yr);
            const float wv = f_of<T>(nwr);
            static_cast<T*>(a.yfrag)[frag_half(b, h * P + p, a.H * P / 128)] = from_f<T>(yv * wv);
            q = yv * yv;
        }
    }
    if constexpr (FRAG) {
        // the wave's 8 rows (lanes 8 i), then the 4 waves in order
        __shared__ float red[4];
        q += __shfl_xor(q, 8);
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        if (threadIdx.x % WAVE == 0) red[threadIdx.x / WAVE] = q;
        __syncthreads();
        if (threadIdx.x == 0) a.ypart[(size_t)b * gridDim.x + blockIdx.x] = red[0] + red[1] + red[2] + red[3];
    }
}

// Generic step for any N (one thread per (h, p), ssd_step.metal layout).
template <typename T, bool GATE>
__global__ void ssd_step_generic_kernel(SsdArgs a) {
    const uint32_t h = blockIdx.x, b = blockIdx.y, p = threadIdx.x;
    if (p >= a.P) return;
    const uint32_t P = a.P, N = a.N;
    const uint32_t hpg = (a.H / a.G) > 0 ? a.H / a.G : 1;
    const uint32_t g = h / hpg;
    const T* Bv = (const T*)a.B + (size_t)b * a.b_stride + (size_t)g * N;
    const T* Cv = (const T*)a.C + (size_t)b * a.c_stride + (size_t)g * N;
    const float A_h = -expf(to_f(((const T*)a.A_log)[h]));
    float dt = softplus_f(to_f(((const T*)a.dt)[(size_t)b * a.dt_stride + h]) + to_f(((const T*)a.dt_bias)[h]));
    dt = fminf(fmaxf(dt, a.dt_min), a.dt_max);
    const float decay = expf(A_h * dt);
    const float D_h = a.has_D ? to_f(((const T*)a.D)[h]) : 0.0f;
    const float xv = to_f(((const T*)a.X)[(size_t)b * a.x_stride + (size_t)h * P + p]);
    float* S = a.state + (((size_t)b * a.H + h) * P + p) * N;
    float ys = 0.0f;
    for (uint32_t n = 0; n < N; ++n) {
        const float s = decay * S[n] + dt * to_f(Bv[n]) * xv;
        S[n] = s;
        ys += to_f(Cv[n]) * s;
    }
    float y = rnd<T>(ys + D_h * xv);
    if constexpr (GATE) {
        const T* Z = (const T*)a.z + (size_t)b * a.z_stride + (size_t)h * P;
        y = silu_f(to_f(Z[p])) * y;
    }
    ((T*)a.Y)[(size_t)b * a.y_stride + (size_t)h * P + p] = from_f<T>(y);
}

// ---------------------------------------------------------------------------
// Chunked scan, scalar VALU version (any dtype; used for fp32 activations).
// Block (h * nPB + pb, b): one head, PB columns of P, all N.  LDS holds the
// rounded state S[PB][N], the chunk's M[CK][CK], DT and Lcum; B/C/X are read
// from global memory (L2-resident within a chunk), as the reference does.
// ---------------------------------------------------------------------------
constexpr int SC_NT = 256;
constexpr int SC_PB = 16;
constexpr int SC_MAXCK = 64;
constexpr int SC_MAXN = 256;

template <typename T>
__global__ __launch_bounds__(SC_NT) void ssd_chunk_scalar_kernel(SsdArgs a) {
    __shared__ float S[SC_PB * SC_MAXN];
    __shared__ float M[SC_MAXCK * SC_MAXCK];
    __shared__ float DT[SC_MAXCK], Lc[SC_MAXCK];
    const uint32_t P = a.P, N = a.N, H = a.H, L = a.L, CK = a.chunk;
    const uint32_t npb = (P + SC_PB - 1) / SC_PB;
    const uint32_t h = blockIdx.x / npb, pb = blockIdx.x % npb, b = blockIdx.y;
    const uint32_t p0 = pb * SC_PB;
    const uint32_t pn = min((uint32_t)SC_PB, P - p0);
    const uint32_t hpg = (H / a.G) > 0 ? H / a.G : 1;
    const uint32_t g = h / hpg;
    const T* X = (const T*)a.X + (size_t)b * L * a.x_stride + (size_t)h * P + p0;
    const T* Bv = (const T*)a.B + (size_t)b * L * a.b_stride + (size_t)g * N;
    const T* Cv = (const T*)a.C + (size_t)b * L * a.c_stride + (size_t)g * N;
    const T* dtr = (const T*)a.dt + (size_t)b * L * a.dt_stride + h;
    T* Y = (T*)a.Y + (size_t)b * L * a.y_stride + (size_t)h * P + p0;
    float* st = a.state + (((size_t)b * H + h) * P + p0) * N;
    const float A_h = -expf(to_f(((const T*)a.A_log)[h]));
    const float dt_b = to_f(((const T*)a.dt_bias)[h]);
    const float D_h = a.has_D ? to_f(((const T*)a.D)[h]) : 0.0f;
    const int tid = threadIdx.x;

    for (uint32_t i = tid; i < pn * N; i += SC_NT) S[i] = rnd<T>(st[i]);
    __syncthreads();

    for (uint32_t t0 = 0; t0 < L; t0 += CK) {
        const uint32_t tl = min(CK, L - t0);
        if (tid < WAVE) {
            float v = 0.0f;
            if ((uint32_t)tid < tl) {
                float dv = softplus_f(to_f(dtr[(size_t)(t0 + tid) * a.dt_stride]) + dt_b);
                dv = fminf(fmaxf(dv, a.dt_min), a.dt_max);
                DT[tid] = dv;
                v = A_h * dv;
            }
#pragma unroll
            for (int off = 1; off < WAVE; off <<= 1) {
                const float o = __shfl_up(v, off, WAVE);
                if (tid >= off) v += o;
            }
            if ((uint32_t)tid < tl) Lc[tid] = v;
        }
        __syncthreads();
        const float L_end = Lc[tl - 1];
        for (uint32_t idx = tid; idx < tl * tl; idx += SC_NT) {
            const uint32_t t = idx / tl, j = idx % tl;
            float m = 0.0f;
            if (j <= t) {
                float cb = 0.0f;
                const T* cr = Cv + (size_t)(t0 + t) * a.c_stride;
                const T* br = Bv + (size_t)(t0 + j) * a.b_stride;
                for (uint32_t n = 0; n < N; ++n) cb += to_f(cr[n]) * to_f(br[n]);
                m = rnd<T>(cb * expf(Lc[t] - Lc[j]) * DT[j]);
            }
            M[t * SC_MAXCK + j] = m;
        }
        __syncthreads();
        for (uint32_t idx = tid; idx < tl * pn; idx += SC_NT) {
            const uint32_t t = idx / pn, p = idx % pn;
            float yi = 0.0f;
            for (uint32_t j = 0; j <= t; ++j) yi += M[t * SC_MAXCK + j] * to_f(X[(size_t)(t0 + j) * a.x_stride + p]);
            float yo = 0.0f;
            const T* cr = Cv + (size_t)(t0 + t) * a.c_stride;
            for (uint32_t n = 0; n < N; ++n) yo += to_f(cr[n]) * S[p * N + n];
            const float xc = to_f(X[(size_t)(t0 + t) * a.x_stride + p]);
            Y[(size_t)(t0 + t) * a.y_stride + p] = from_f<T>(yi + yo * expf(Lc[t]) + D_h * xc);
        }
        __syncthreads();
        const float dch = expf(L_end);
        for (uint32_t idx = tid; idx < pn * N; idx += SC_NT) {
            const uint32_t p = idx / N, n = idx % N;
            float acc = dch * S[idx];
            for (uint32_t j = 0; j < tl; ++j)
                acc += expf(L_end - Lc[j]) * DT[j] * to_f(Bv[(size_t)(t0 + j) * a.b_stride + n]) *
                       to_f(X[(size_t)(t0 + j) * a.x_stride + p]);
            S[idx] = rnd<T>(acc);
        }
        __syncthreads();
    }
    for (uint32_t i = tid; i < pn * N; i += SC_NT) st[i] = S[i];
}

// ---------------------------------------------------------------------------
// Chunked scan on MFMA (fp16 / bf16), chunk Q = 64, N = 128, P % (16 NW) == 0.
// Block (h * P/(16 NW) + pb, b), NW waves; wave w owns the 16 state columns
// p = 16 w .. +16 of the block's slice.  v_mfma_f32_16x16x32 operand lanes:
// lane l = 16 q + i supplies row/column i and k = 8 q .. 8 q + 7; the result
// holds rows 4 q .. 4 q + 3 of column i.  All products put the token index on
// k, so token-major tiles (B, X) are read with the gfx950 LDS transpose load
// (ds_read_b64_tr_b16: lane i of each 16-lane group gets column i of the
// four rows read by lane blocks 0..3).  Per chunk:
//   G^T[j][t] = B_j . C_t                    (10 lower tiles, shared by the waves)
//   M[t][j]   = r(G^T e^{Lc_t - Lc_j} DT_j)  -> LDS, token-major
//   Y^T[p][t] = X^T M^T + e^{Lc_t} (S . C_t) + D x      (wave: 16 p x 64 t)
//   S^T[n][p] = r(e^{L_end} S^T + B^T (w o X)),  w_j = e^{L_end - Lc_j} DT_j
// S^T lives in registers as fp32 (the rounded values), laid out so that its
// tiles are directly the k = n operand of S . C_t.  The next chunk's B, C, X
// and dt are prefetched into registers during the current chunk; two
// barriers per chunk.
// ---------------------------------------------------------------------------
// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its global loads and stores (a __syncthreads would also
// wait for the register prefetch of later chunks and for the Y stores).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int CQ = 64;            // chunk
constexpr int CN = 128;           // state size
constexpr int SPAD = CN + 8;      // B / C row pitch (elements)
constexpr int MPAD = CQ + 8;      // M row pitch

typedef short s4v __attribute__((ext_vector_type(4)));
typedef short s8v __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ floatx4 mma16(s8v a, s8v b, floatx4 c) {
    if constexpr (__is_same(T, bf16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                      __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Transposed 64-bit LDS load (see above); p must be 8-byte aligned.
__device__ __forceinline__ s4v ld_tr(const void* p) {
    typedef __attribute__((address_space(3))) s4v lds_s4v;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v*)(const_cast<void*>(p)));
}

template <typename T> __device__ __forceinline__ short bits_of(float v) {
    return __builtin_bit_cast(short, from_f<T>(v));
}
template <typename T> __device__ __forceinline__ float val_of(short v) {
    return to_f(__builtin_bit_cast(T, v));
}
typedef float f32x2s __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2s __attribute__((ext_vector_type(2)));
typedef short s2v __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ s4v pack4(floatx4 v) {
    if constexpr (__is_same(T, bf16)) {
        // two v_cvt_pk_bf16_f32 (round to nearest even, as each value alone)
        typedef uint32_t u32x2s __attribute__((ext_vector_type(2)));
        const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2s{v[0], v[1]}, bf16x2s));
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2s{v[2], v[3]}, bf16x2s));
        return __builtin_bit_cast(s4v, u32x2s{lo, hi});
    } else {
        s4v r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = bits_of<T>(v[e]);
        return r;
    }
}
__device__ __forceinline__ s8v cat8(s4v lo, s4v hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <typename T> __device__ __forceinline__ floatx4 unpack4(s4v v) {
    floatx4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = val_of<T>(v[e]);
    return r;
}

// The chunks' Gram tiles G[t][j] = C_t . B_j (fp32, t, j < 64), which depend
// only on the sequence, the chunk and the group: computed once here and read
// by every head of the group (and P slice) in ssd_chunk_mfma_kernel instead of
// being recomputed there.  Block (chunk, group, sequence), four waves; the ten
// tiles with J <= T (16-token blocks) only, on the same MFMA with the same
// operands as the in-kernel computation, so the values are identical.  The
// operands are read straight from global memory: both have k = n contiguous.
// Tokens past the end of the last chunk re-read token t0 (their entries are
// masked by the scan).
template <typename T>
__global__ __launch_bounds__(256) void ssd_gram_kernel(SsdArgs a) {
    const uint32_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const uint32_t L = a.L, nch = (L + CQ - 1) / CQ, t0 = c * CQ;
    const uint32_t tl = min((uint32_t)CQ, L - t0);
    const int lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const int li = lane % 16, lq = lane / 16;
    const T* Bv = (const T*)a.B + ((size_t)b * L + t0) * a.b_stride + (size_t)g * CN;
    const T* Cv = (const T*)a.C + ((size_t)b * L + t0) * a.c_stride + (size_t)g * CN;
    float* out = a.gram + (((size_t)b * nch + c) * a.G + g) * (CQ * CQ);
    // (J, T) of the ten lower tiles, 2 + 2 bits each
    constexpr uint64_t JT = 0x0ull | 0x4ull << 4 | 0x5ull << 8 | 0x8ull << 12 | 0x9ull << 16 | 0xAull << 20 |
                            0xCull << 24 | 0xDull << 28 | 0xEull << 32 | 0xFull << 36;
    for (int kt = w; kt < 10; kt += 4) {
        const int jt = (int)(JT >> (4 * kt)) & 15;
        const int J = jt & 3, Tt = jt >> 2;
        const uint32_t j = 16 * J + li, t = 16 * Tt + li;
        const T* br = Bv + (size_t)(j < tl ? j : 0) * a.b_stride + 8 * lq;
        const T* cr = Cv + (size_t)(t < tl ? t : 0) * a.c_stride + 8 * lq;
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < CN / 32; ++ks)
            acc = mma16<T>(*reinterpret_cast<const s8v*>(br + 32 * ks), *reinterpret_cast<const s8v*>(cr + 32 * ks), acc);
        // acc[r] = B_{16J + 4lq + r} . C_t  ->  G[t][16J + 4lq .. + 3]
        *reinterpret_cast<floatx4*>(out + (size_t)t * CQ + 16 * J + 4 * lq) = acc;
    }
}

// SPL = 2: two waves per 16-column slice.  Wave (slice cs, half hh) computes
// the output token tiles 2 hh, 2 hh + 1 and updates state tiles n = 64 hh ..
// + 63 (it keeps the whole state of its columns, the k = n operand of C . S);
// the halves trade their updated state tiles through LDS at the mid-chunk
// barrier.  The serial chain per chunk is then about half as long, and a CU
// holds twice the waves.
// (four-wave blocks are held to 256 registers, two blocks per CU: a grid
// slightly larger than the CU count runs in one round)
template <typename T, int NW, bool GP, int SPL>
__global__ __launch_bounds__(64 * NW * SPL) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 2 : 1)))
void ssd_chunk_mfma_kernel(SsdArgs a) {
    constexpr int NWV = NW * SPL;         // waves
    constexpr int NT = 64 * NWV;          // threads
    constexpr int PB = 16 * NW;           // state columns p per block
    constexpr int NTT = 4 / SPL;          // output token tiles per wave
    constexpr int NST = 8 / SPL;          // state n-tiles a wave updates
    constexpr int XP = PB + 8;            // X row pitch
    constexpr int BV = CQ * CN / 8 / NT;  // 16-byte pieces of B (and of C) per thread
    constexpr int XV = CQ * PB / 8 / NT;  // 16-byte pieces of X per thread (= 2)
    constexpr int BR = NT / 16;           // B / C rows per load round
    constexpr int XR = NT / (PB / 8);     // X rows per load round
    __shared__ __attribute__((aligned(16))) T Bs[CQ * SPAD];
    __shared__ __attribute__((aligned(16))) T Cs[CQ * SPAD];
    __shared__ __attribute__((aligned(16))) T Xs[CQ * XP];
    __shared__ __attribute__((aligned(16))) T Ms[CQ * MPAD];
    // per-token chunk scalars, double-buffered: wave 0 computes chunk c + 1's
    // while the block works on chunk c
    __shared__ __attribute__((aligned(16))) float LCb[2][CQ], DTb[2][CQ], ELb[2][CQ], Wb[2][CQ];
    // the masked decay factored per 16-token block T (r = 16 T):
    // e^{Lc_t - Lc_j} DT_j = AFb[t] * BFb[T][j], AFb[t] = e^{Lc_t - Lc_r} (t in
    // block T), BFb[T][j] = e^{Lc_r - Lc_j} DT_j (j < r + 16); SFb bit T set when
    // block T's own decay is small enough for its diagonal tile to use them
    __shared__ __attribute__((aligned(16))) float AFb[2][CQ], BFb[2][4][CQ];
    __shared__ uint32_t SFb[2];
    // gated epilogue (a.gpart): each column slice's per-token sums of g^2,
    // double-buffered by chunk parity
    __shared__ __attribute__((aligned(16))) float GQ[2][NW][CQ];
    // SPL = 2: each wave's updated state tiles for its partner
    __shared__ __attribute__((aligned(16))) s4v Sx[SPL == 2 ? NWV * NST * 64 : 1];

    const uint32_t P = a.P, H = a.H, L = a.L;
    const uint32_t npb = P / PB;
    // (grouping one sequence's walks on one or two XCDs, so that its B, C and
    // Gram tiles are read through fewer L2s, measured 2 % slower at 4 x 4096)
    const uint32_t h = blockIdx.x / npb, pb = blockIdx.x % npb, b = blockIdx.y;
    const uint32_t p0 = pb * PB;
    const uint32_t hpg = (H / a.G) > 0 ? H / a.G : 1;
    const uint32_t g = h / hpg;
    const T* X = (const T*)a.X + (size_t)b * L * a.x_stride + (size_t)h * P + p0;
    const T* Bv = (const T*)a.B + (size_t)b * L * a.b_stride + (size_t)g * CN;
    const T* Cv = (const T*)a.C + (size_t)b * L * a.c_stride + (size_t)g * CN;
    const T* dtr = (const T*)a.dt + (size_t)b * L * a.dt_stride + h;
    T* Y = (T*)a.Y + (size_t)b * L * a.y_stride + (size_t)h * P + p0;
    const bool gate = a.gpart != nullptr;
    const T* Z = gate ? (const T*)a.z + (size_t)b * L * a.z_stride + (size_t)h * P + p0 : nullptr;
    // gpart is [part][batch L]: a block's 64 per-token sums of a chunk are
    // one contiguous 256-byte store
    float* gcol = gate ? a.gpart + ((size_t)h * npb + pb) * ((size_t)a.batch * L) + (size_t)b * L : nullptr;
    float* st = a.state + (((size_t)b * H + h) * P + p0) * CN;
    // segment blockIdx.z of a.nseg: chunks cb .. ce - 1, starting from the
    // state the segment pass left in the workspace; only the last segment
    // writes the final state
    const uint32_t sg = blockIdx.z, nchs = (L + CQ - 1) / CQ;
    const uint32_t cb = sg * a.seg_chunks, ce = min(nchs, cb + a.seg_chunks);
    const bool last_seg = sg + 1 == a.nseg;
    const float* st_in = a.nseg > 1 ? a.seg + ((((size_t)b * a.nseg + sg) * H + h) * P + p0) * CN : st;
    const float A_h = -expf(to_f(((const T*)a.A_log)[h]));
    const float dt_b = to_f(((const T*)a.dt_bias)[h]);
    const float D_h = a.has_D ? to_f(((const T*)a.D)[h]) : 0.0f;

    const int tid = threadIdx.x;
    const int lane = tid % WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int li = lane % 16, lq = lane / 16;
    const int tk = li / 4, tc = li % 4;    // transpose-load row block / column piece
    const int cs = w % NW, hh = SPL == 1 ? 0 : w / NW;   // column slice, half (SPL = 2)
    const int pw = 16 * cs;                // this wave's columns within the block

    // S^T tiles, rounded to T and packed: sp[nt][r] = S[p = pw + li][n = 16 nt + 4 lq + r]
    s4v sp[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
        sp[nt] = pack4<T>(*reinterpret_cast<const floatx4*>(st_in + (size_t)(pw + li) * CN + 16 * nt + 4 * lq));

    // D x as one more MFMA: X^T times the diagonal tile D I (exact in T).
    // Token tile Tt lies in k-slice Tt / 2, where column t = 16 Tt + li has its
    // diagonal at slot e = 16 (Tt % 2) + li - 8 lq.
    s8v dfr[2];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
        for (int e = 0; e < 8; ++e) dfr[par][e] = (e == 16 * par + li - 8 * lq) ? bits_of<T>(D_h) : (short)0;

    // ---- register prefetch of one chunk through buffer loads: a resource
    // per tensor and chunk (base = the chunk's first row, range = its tl
    // rows), a fixed 32-bit per-thread offset and a uniform offset per row
    // group, so no per-lane address arithmetic.  Rows past L (last chunk)
    // fall outside the range and read 0: they only meet M entries that are
    // masked and state weights w = 0. ----
    const uint32_t brow = tid / 16, bcol = (tid % 16) * 8;
    const uint32_t xrow = tid / (PB / 8), xcol = (tid % (PB / 8)) * 8;
    const uint32_t boff = (brow * a.b_stride + bcol) * sizeof(T), coff = (brow * a.c_stride + bcol) * sizeof(T);
    const uint32_t xoff = (xrow * a.x_stride + xcol) * sizeof(T);
    const uint32_t bstep = BR * a.b_stride * sizeof(T), cstep = BR * a.c_stride * sizeof(T);
    const uint32_t xstep = XR * a.x_stride * sizeof(T);
    auto rsrc = [](const void* p, uint32_t bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
    };
    u32x4 rb[BV], rc[BV], rx[XV];   // (vector types: a struct uint4 copies
                                    // through memory and stays in scratch)
    uint32_t rdt = 0;
    // Gram tiles of this wave's M positions (GP): next chunk's in flight,
    // current chunk's in use
    constexpr int NTL = (12 + NWV - 1) / NWV;
    constexpr uint64_t JT = 0x1ull | 0x0ull << 4 | 0x4ull << 8 | 0x5ull << 12 | 0xBull << 16 |
                            0x8ull << 20 | 0x9ull << 24 | 0xAull << 28 | 0xCull << 32 |
                            0xDull << 36 | 0xEull << 40 | 0xFull << 44;
    floatx4 rgn[GP ? NTL : 1], rgc[GP ? NTL : 1];
    const uint32_t nchk = (L + CQ - 1) / CQ;
    auto fetch = [&](uint32_t t0) {
        const uint32_t tl = min((uint32_t)CQ, L - t0);
        if constexpr (GP) {
            const auto rg = rsrc(a.gram + (((size_t)b * nchk + t0 / CQ) * a.G + g) * (CQ * CQ), CQ * CQ * 4);
#pragma unroll
            for (int i = 0; i < NTL; ++i) {
                const int kt = w + NWV * i;
                const int jt = (int)(JT >> (4 * kt)) & 15;
                const int J = jt & 3, Tt = jt >> 2;
                if (kt < 12 && kt != 0 && kt != 4)
                    rgn[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                        rg, (uint32_t)(((16 * Tt + li) * CQ + 16 * J + 4 * lq) * 4), 0, 0));
            }
        }
        const auto rB = rsrc(Bv + (size_t)t0 * a.b_stride, ((tl - 1) * a.b_stride + CN) * sizeof(T));
        const auto rC = rsrc(Cv + (size_t)t0 * a.c_stride, ((tl - 1) * a.c_stride + CN) * sizeof(T));
        const auto rX = rsrc(X + (size_t)t0 * a.x_stride, ((tl - 1) * a.x_stride + PB) * sizeof(T));
#pragma unroll
        for (int v = 0; v < BV; ++v) {
            rb[v] = __builtin_amdgcn_raw_buffer_load_b128(rB, boff, v * bstep, 0);
            rc[v] = __builtin_amdgcn_raw_buffer_load_b128(rC, coff, v * cstep, 0);
        }
#pragma unroll
        for (int v = 0; v < XV; ++v) rx[v] = __builtin_amdgcn_raw_buffer_load_b128(rX, xoff, v * xstep, 0);
        const auto rD = rsrc(dtr + (size_t)t0 * a.dt_stride, ((tl - 1) * a.dt_stride + 1) * sizeof(T));
        rdt = __builtin_amdgcn_raw_buffer_load_b16(rD, (uint32_t)lane * a.dt_stride * (uint32_t)sizeof(T), 0, 0);
    };
    auto stage = [&]() {
        if constexpr (GP) {
#pragma unroll
            for (int i = 0; i < NTL; ++i) rgc[i] = rgn[i];
        }
#pragma unroll
        for (int v = 0; v < BV; ++v) {
            *reinterpret_cast<u32x4*>(Bs + (brow + BR * v) * SPAD + bcol) = rb[v];
            *reinterpret_cast<u32x4*>(Cs + (brow + BR * v) * SPAD + bcol) = rc[v];
        }
#pragma unroll
        for (int v = 0; v < XV; ++v) *reinterpret_cast<u32x4*>(Xs + (xrow + XR * v) * XP + xcol) = rx[v];
    };
    // DT, Lcum, e^{Lcum}, the state weights w and the masked-decay factors of
    // the chunk at t0 into buffer `buf` (tokens past tl get DT = 0, so they
    // drop out).  Every wave forms DT and Lcum (a few instructions and a DPP
    // prefix sum) and writes one part of the outputs, so the exponentials are
    // spread over the waves: part 0 Lcum, DT and the block flags; 1 e^{Lcum}
    // and w; 2 the row factors and the first column factors; 3 the others.
    auto scan = [&](uint32_t t0, int buf, int part) {
        const uint32_t tl = min((uint32_t)CQ, L - t0);
        float dv = 0.0f;
        if ((uint32_t)lane < tl) {
            dv = softplus_fast(f_of<T>(rdt) + dt_b);
            dv = fminf(fmaxf(dv, a.dt_min), a.dt_max);
        }
        const float v = wave_prefix_sum(A_h * dv);
        // factors of the masked decay.  Off-diagonal tiles (j < r <= t): both
        // exponents <= 0, so a <= 1 and b <= DT.  Diagonal tiles (r <= j, t <
        // r + 16): b >= DT grows with the block's decay, bounded by e^60 DT
        // where the flag is set; tokens past tl have a = b = 0 (DT = 0).
        if (part == 0) {
            LCb[buf][lane] = v;
            DTb[buf][lane] = dv;
            const float lc_q = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x15F, 0xF, 0xF, false));
            const float lc_r = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150, 0xF, 0xF, false));
            const uint64_t ok = __ballot(lc_r - lc_q <= 60.0f);   // decay over the lane's block
            if (lane == 0) {
                uint32_t bits = 0;
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) bits |= ((ok >> (16 * tb)) & 1ull) ? (1u << tb) : 0u;
                SFb[buf] = bits;
            }
        } else if (part == 1) {
            ELb[buf][lane] = __expf(v);
            Wb[buf][lane] = __expf(readlane_f(v, WAVE - 1) - v) * dv;
        } else if (part == 2) {
            const float lc_r = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150, 0xF, 0xF, false));
            AFb[buf][lane] = (uint32_t)lane < tl ? __expf(v - lc_r) : 0.0f;
            BFb[buf][0][lane] = lane < 16 ? __expf(readlane_f(v, 0) - v) * dv : 0.0f;
        } else {
#pragma unroll
            for (int tb = 1; tb < 4; ++tb)
                BFb[buf][tb][lane] = lane < 16 * tb + 16 ? __expf(readlane_f(v, 16 * tb) - v) * dv : 0.0f;
        }
    };
    // the parts of the scan this wave writes
    auto scan_parts = [&](uint32_t t0, int buf) {
        if constexpr (NWV >= 4) {
            if (w < 4) scan(t0, buf, w);
        } else {
            scan(t0, buf, w);
            scan(t0, buf, w + 2);
        }
    };

    // Prefetches past the segment's last chunk re-read that chunk: loads
    // issued on every iteration keep the registers they fill out of
    // conditional merges (which the compiler resolves with copies that wait
    // for the loads just issued).
    const uint32_t t_last = (ce - 1) * CQ;
    // gated epilogue: the norm weights of this lane's four columns, and z of
    // the wave's token tiles, requested at the start of each chunk (a phase
    // ahead of their use in the Y stores)
    floatx4 gw = {0.0f, 0.0f, 0.0f, 0.0f};
    if (gate) gw = unpack4<T>(*reinterpret_cast<const s4v*>((const T*)a.gnorm_w + (size_t)h * P + p0 + pw + 4 * lq));
    typedef uint32_t u32x2z __attribute__((ext_vector_type(2)));
    u32x2z zr[4];
    auto fetch_z = [&](uint32_t t0) {
        const uint32_t tl = min((uint32_t)CQ, L - t0);
        const auto rZ = rsrc(Z + (size_t)t0 * a.z_stride, ((tl - 1) * a.z_stride + PB) * sizeof(T));
        const uint32_t zo = (li * a.z_stride + pw + 4 * lq) * sizeof(T);
#pragma unroll
        for (int Tt = 0; Tt < 4; ++Tt)
            if (Tt / NTT == hh)
                zr[Tt] = __builtin_amdgcn_raw_buffer_load_b64(rZ, zo, Tt * 16 * a.z_stride * sizeof(T), 0);
    };
    // wave 0: the block's per-token sums of chunk cp (parity pp) to gpart
    auto flush_gq = [&](uint32_t cp, uint32_t pp) {
        const uint32_t tp0 = cp * CQ, tlp = min((uint32_t)CQ, L - tp0);
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < NW; ++k) v += GQ[pp][k][lane];
        if ((uint32_t)lane < tlp) gcol[tp0 + lane] = v;
    };
    fetch(cb * CQ);
    stage();
    scan_parts(cb * CQ, 0);
    fetch(min((cb + 1) * CQ, t_last));
    lds_barrier();

    for (uint32_t c = cb; c < ce; ++c) {
        const uint32_t par = (c - cb) & 1;   // buffer of this chunk's scalars
        const uint32_t t0 = c * CQ;
        const uint32_t tl = min((uint32_t)CQ, L - t0);

        const float* LCs = LCb[par];
        const float* ELs = ELb[par];
        const float* Ws = Wb[par];
        if (gate) {
            fetch_z(t0);
            if (w == 0 && c > cb) flush_gq(c - 1, par ^ 1);
        }

        // ---- G^T tiles (J <= T) -> M.  Twelve tiles, wave w takes positions
        // w, w + NW, ...; positions 0 and 4 are the zero upper halves (1,0)
        // and (3,2) of the k = 32 slices Y reads, which leaves wave 0 time
        // for the next chunk's dt scan.  (J, T) per position as 2 + 2 bits of
        // an immediate (an indexed array would be a memory load whose wait
        // would also wait for the prefetch). ----
        {
            const float* DTs = DTb[par];
            const uint32_t safe = SFb[par];
#pragma unroll
            for (int i = 0; i < NTL; ++i) {
                const int kt = w + NWV * i;
                if (kt >= 12) break;
                const int jt = (int)(JT >> (4 * kt)) & 15;
                const int J = jt & 3, Tt = jt >> 2;
                const int t = 16 * Tt + li;
                s4v m4 = {0, 0, 0, 0};
                if (kt != 0 && kt != 4) {
                    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (GP) {
                        acc = rgc[i];
                    } else {
#pragma unroll
                        for (int ks = 0; ks < CN / 32; ++ks) {
                            const s8v af = *reinterpret_cast<const s8v*>(Bs + (16 * J + li) * SPAD + 32 * ks + 8 * lq);
                            const s8v bf = *reinterpret_cast<const s8v*>(Cs + t * SPAD + 32 * ks + 8 * lq);
                            acc = mma16<T>(af, bf, acc);
                        }
                    }
                    floatx4 m;
                    if (J < Tt || ((safe >> Tt) & 1u)) {
                        // factored decay (wave-uniform branch): two products
                        const float at = AFb[par][t];
                        const floatx4 bj = *reinterpret_cast<const floatx4*>(&BFb[par][Tt][16 * J + 4 * lq]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float mv = acc[r] * at * bj[r];
                            m[r] = (J < Tt || 16 * J + 4 * lq + r <= t) ? mv : 0.0f;
                        }
                    } else {
                        const float lct = LCs[t];
                        const floatx4 lcj = *reinterpret_cast<const floatx4*>(LCs + 16 * J + 4 * lq);
                        const floatx4 dtj = *reinterpret_cast<const floatx4*>(DTs + 16 * J + 4 * lq);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int j = 16 * J + 4 * lq + r;
                            // Lcum is non-increasing, so the exponent is <= 0 on
                            // the kept entries; the clamp keeps the others finite
                            float mv = acc[r] * __expf(fminf(lct - lcj[r], 0.0f)) * dtj[r];
                            asm volatile("" : "+v"(mv));   // compute, then select (no branch)
                            m[r] = (j <= t && (uint32_t)t < tl) ? mv : 0.0f;
                        }
                    }
                    m4 = pack4<T>(m);
                }
                *reinterpret_cast<s4v*>(Ms + t * MPAD + 16 * J + 4 * lq) = m4;
            }
        }

        // ---- X^T slices of this wave's columns (k = token) ----
        s8v xf[2];
#pragma unroll
        for (int ka = 0; ka < 2; ++ka) {
            const T* xp = Xs + (32 * ka + 8 * lq + tk) * XP + pw + 4 * tc;
            xf[ka] = cat8(ld_tr(xp), ld_tr(xp + 4 * XP));
        }

        // ---- e^{Lcum_t} (S_p . C_t) for the 4 token tiles; S is the
        // k = n operand as it lies in registers ----
        // (register arrays are indexed by unrolled constants only: the wave's
        // half hh selects tiles by a wave-uniform branch)
        floatx4 yacc[4];
#pragma unroll
        for (int Tt = 0; Tt < 4; ++Tt) {
            if (Tt / NTT != hh) continue;
            const int t = 16 * Tt + li;
            floatx4 yo = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const T* cp = Cs + t * SPAD + 32 * ks + 4 * lq;
                const s8v cf = cat8(*reinterpret_cast<const s4v*>(cp), *reinterpret_cast<const s4v*>(cp + 16));
                yo = mma16<T>(cat8(sp[2 * ks], sp[2 * ks + 1]), cf, yo);
            }
            const float el = ELs[t];
#pragma unroll
            for (int r = 0; r < 4; ++r) yacc[Tt][r] = yo[r] * el;
        }

        // ---- S^T = r(e^{L_end} S^T + B^T (w o X)) ----
        {
            const float dch = __expf(LCs[CQ - 1]);
            s8v wx[2];
#pragma unroll
            for (int ka = 0; ka < 2; ++ka) {
                const floatx4 w0 = *reinterpret_cast<const floatx4*>(Ws + 32 * ka + 8 * lq);
                const floatx4 w1 = *reinterpret_cast<const floatx4*>(Ws + 32 * ka + 8 * lq + 4);
                floatx4 p0, p1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    p0[e] = w0[e] * val_of<T>(xf[ka][e]);
                    p1[e] = w1[e] * val_of<T>(xf[ka][e + 4]);
                }
                wx[ka] = cat8(pack4<T>(p0), pack4<T>(p1));
            }
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                if (nt / NST != hh) continue;
                floatx4 acc = unpack4<T>(sp[nt]);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] *= dch;
#pragma unroll
                for (int ka = 0; ka < 2; ++ka) {
                    const T* bp = Bs + (32 * ka + 8 * lq + tk) * SPAD + 16 * nt + 4 * tc;
                    const s8v bt = cat8(ld_tr(bp), ld_tr(bp + 4 * SPAD));
                    acc = mma16<T>(bt, wx[ka], acc);
                }
                sp[nt] = pack4<T>(acc);
                if constexpr (SPL == 2) Sx[(w * NST + nt % NST) * 64 + lane] = sp[nt];
            }
        }
        lds_barrier();   // M complete; staging no longer read; state halves posted
        if constexpr (SPL == 2) {
            const int pw2 = (w + NW) % NWV;                 // the partner wave
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
                if (nt / NST != hh) sp[nt] = Sx[(pw2 * NST + nt % NST) * 64 + lane];
        }

        // Stage the next chunk first: its loads were issued a chunk ago, and
        // waiting for them before the Y stores below keeps those stores out
        // of the wait.
        if (c + 1 < ce) stage();
        // the next chunk's scalars (their buffer was last read in the previous
        // chunk; dt arrived with the prefetch a chunk ago)
        if (c + 1 < ce) scan_parts(t0 + CQ, par ^ 1);

        // ---- Y^T += X^T M^T + X^T (D I), store ----
#pragma unroll
        for (int Tt = 0; Tt < 4; ++Tt) {
            if (Tt / NTT != hh) continue;
            const int t = 16 * Tt + li;
#pragma unroll
            for (int ka = 0; ka < 2; ++ka) {
                if (ka == 1 && Tt < 2) continue;
                const s8v mf = *reinterpret_cast<const s8v*>(Ms + t * MPAD + 32 * ka + 8 * lq);
                yacc[Tt] = mma16<T>(xf[ka], mf, yacc[Tt]);
            }
            if (a.has_D) yacc[Tt] = mma16<T>(xf[Tt / 2], dfr[Tt % 2], yacc[Tt]);
            if (gate) {
                // the gated RMSNorm's front half (gated_rmsnorm: g =
                // r(silu(z) r(y)), then g w): r(g w) stored, sum of g^2 kept
                // (the projection GEMM stored r(silu(z)) as z)
                const floatx4 zf = unpack4<T>(__builtin_bit_cast(s4v, zr[Tt]));
                floatx4 o;
                float sq = 0.0f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float g = rnd<T>(zf[r] * rnd<T>(yacc[Tt][r]));
                    o[r] = g * gw[r];
                    sq = fmaf(g, g, sq);
                }
                sq = swap_add32(swap_add16(sq));   // the token's 16 columns
                if (lq == 0) GQ[par][cs][t] = sq;
                if ((uint32_t)t < tl)
                    *reinterpret_cast<s4v*>(Y + (size_t)(t0 + t) * a.y_stride + pw + 4 * lq) = pack4<T>(o);
            } else if ((uint32_t)t < tl) {
                *reinterpret_cast<s4v*>(Y + (size_t)(t0 + t) * a.y_stride + pw + 4 * lq) = pack4<T>(yacc[Tt]);
            }
        }
        fetch(min(t0 + 2 * CQ, t_last));
        lds_barrier();
    }
    if (gate && w == 0) flush_gq(ce - 1, (ce - 1 - cb) & 1);
    if (!last_seg) return;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
        if (nt / NST == hh)
            *reinterpret_cast<floatx4*>(st + (size_t)(pw + li) * CN + 16 * nt + 4 * lq) = unpack4<T>(sp[nt]);
}


// ---------------------------------------------------------------------------
// Segmented chunked scan.  When a grid of (sequence, head, column block)
// walks would leave CUs idle, each sequence's chunks are split into a.nseg
// segments of a.seg_chunks chunks, run in three launches:
//   1. ssd_seg_state_kernel, segments 0 .. nseg - 2 in parallel: the state
//      the segment's chunks leave when it starts from zero,
//        S_s = sum_c e^{sum of L_end after c} B_c^T (w_c o X_c)   (fp32),
//      by the walk's state update without its rounding, and the segment's
//      log-decay sum_c L_end(c);
//   2. ssd_seg_scan_kernel: the state entering every segment,
//        S_in(0) = S_init,  S_in(s + 1) = e^{decay(s)} S_in(s) + S_s,
//      in place over the workspace (an exact recurrence over nseg terms);
//   3. the walk, all segments at once, segment s from S_in(s) (rounded to
//      the activation type as the walk holds its state); the last segment
//      writes the final state.
// The walk rounds its state after every chunk as ssd_chunked.metal does;
// across a segment boundary the entering state is the fp32 recurrence
// instead of the chain of rounded states, so results agree with the
// unsegmented scan to within that rounding.
// ---------------------------------------------------------------------------
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW) void ssd_seg_state_kernel(SsdArgs a) {
    constexpr int NT = 64 * NW;
    constexpr int PB = 16 * NW;           // state columns p per block
    constexpr int XP = PB + 8;            // X row pitch
    constexpr int BV = CQ * CN / 8 / NT;  // 16-byte pieces of B per thread
    constexpr int XV = CQ * PB / 8 / NT;  // 16-byte pieces of X per thread
    constexpr int BR = NT / 16, XR = NT / (PB / 8);
    // double-buffered: chunk c + 1 is staged while chunk c is in use, so one
    // barrier per chunk
    __shared__ __attribute__((aligned(16))) T Bs[2][CQ * SPAD];
    __shared__ __attribute__((aligned(16))) T Xs[2][CQ * XP];
    __shared__ __attribute__((aligned(16))) float Wb[2][CQ];
    __shared__ float LEb[2];

    const uint32_t P = a.P, H = a.H, L = a.L;
    const uint32_t npb = P / PB;
    const uint32_t h = blockIdx.x / npb, pb = blockIdx.x % npb, b = blockIdx.y, sg = blockIdx.z;
    const uint32_t p0 = pb * PB;
    const uint32_t hpg = (H / a.G) > 0 ? H / a.G : 1;
    const uint32_t g = h / hpg;
    const uint32_t nch = (L + CQ - 1) / CQ;
    const uint32_t cb = sg * a.seg_chunks, ce = min(nch, cb + a.seg_chunks);
    const T* X = (const T*)a.X + (size_t)b * L * a.x_stride + (size_t)h * P + p0;
    const T* Bv = (const T*)a.B + (size_t)b * L * a.b_stride + (size_t)g * CN;
    const T* dtr = (const T*)a.dt + (size_t)b * L * a.dt_stride + h;
    const float A_h = -expf(to_f(((const T*)a.A_log)[h]));
    const float dt_b = to_f(((const T*)a.dt_bias)[h]);

    const int tid = threadIdx.x;
    const int lane = tid % WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int li = lane % 16, lq = lane / 16;
    const int tk = li / 4, tc = li % 4;
    const int pw = 16 * w;

    const uint32_t brow = tid / 16, bcol = (tid % 16) * 8;
    const uint32_t xrow = tid / (PB / 8), xcol = (tid % (PB / 8)) * 8;
    u32x4 rb[BV], rx[XV];
    uint32_t rdt = 0;
    // rows past L (last chunk) re-read row t0; their state weight is 0
    auto fetch = [&](uint32_t t0) {
        const uint32_t tl = min((uint32_t)CQ, L - t0);
#pragma unroll
        for (int v = 0; v < BV; ++v) {
            const uint32_t t = brow + BR * v, tt = t0 + (t < tl ? t : 0);
            rb[v] = *reinterpret_cast<const u32x4*>(Bv + (size_t)tt * a.b_stride + bcol);
        }
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            const uint32_t t = xrow + XR * v, tt = t0 + (t < tl ? t : 0);
            rx[v] = *reinterpret_cast<const u32x4*>(X + (size_t)tt * a.x_stride + xcol);
        }
        if (w == 0) rdt = raw_of(dtr + (size_t)(t0 + min((uint32_t)lane, tl - 1)) * a.dt_stride);
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int v = 0; v < BV; ++v) *reinterpret_cast<u32x4*>(Bs[buf] + (brow + BR * v) * SPAD + bcol) = rb[v];
#pragma unroll
        for (int v = 0; v < XV; ++v) *reinterpret_cast<u32x4*>(Xs[buf] + (xrow + XR * v) * XP + xcol) = rx[v];
    };
    // wave 0: the state weights w and L_end of the chunk at t0, as the walk's
    // scan computes them
    auto scan = [&](uint32_t t0, int buf) {
        const uint32_t tl = min((uint32_t)CQ, L - t0);
        float dv = 0.0f;
        if ((uint32_t)lane < tl) {
            dv = softplus_fast(f_of<T>(rdt) + dt_b);
            dv = fminf(fmaxf(dv, a.dt_min), a.dt_max);
        }
        const float v = wave_prefix_sum(A_h * dv);
        const float l_end = readlane_f(v, WAVE - 1);
        Wb[buf][lane] = __expf(l_end - v) * dv;
        if (lane == 0) LEb[buf] = l_end;
    };

    floatx4 sf[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) sf[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float lseg = 0.0f;
    fetch(cb * CQ);
    for (uint32_t c = cb; c < ce; ++c) {
        const int buf = (c - cb) & 1;
        stage(buf);
        if (w == 0) scan(c * CQ, buf);
        __syncthreads();
        if (c + 1 < ce) fetch((c + 1) * CQ);
        const float le = LEb[buf];
        lseg += le;
        const float dch = __expf(le);
        s8v xf[2], wx[2];
#pragma unroll
        for (int ka = 0; ka < 2; ++ka) {
            const T* xp = Xs[buf] + (32 * ka + 8 * lq + tk) * XP + pw + 4 * tc;
            xf[ka] = cat8(ld_tr(xp), ld_tr(xp + 4 * XP));
            const floatx4 w0 = *reinterpret_cast<const floatx4*>(Wb[buf] + 32 * ka + 8 * lq);
            const floatx4 w1 = *reinterpret_cast<const floatx4*>(Wb[buf] + 32 * ka + 8 * lq + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wx[ka][e] = bits_of<T>(w0[e] * val_of<T>(xf[ka][e]));
                wx[ka][e + 4] = bits_of<T>(w1[e] * val_of<T>(xf[ka][e + 4]));
            }
        }
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
            floatx4 acc = sf[nt];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] *= dch;
#pragma unroll
            for (int ka = 0; ka < 2; ++ka) {
                const T* bp = Bs[buf] + (32 * ka + 8 * lq + tk) * SPAD + 16 * nt + 4 * tc;
                acc = mma16<T>(cat8(ld_tr(bp), ld_tr(bp + 4 * SPAD)), wx[ka], acc);
            }
            sf[nt] = acc;
        }
    }
    float* out = a.seg + ((((size_t)b * a.nseg + sg) * H + h) * P + p0) * CN;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
        *reinterpret_cast<floatx4*>(out + (size_t)(pw + li) * CN + 16 * nt + 4 * lq) = sf[nt];
    if (pb == 0 && tid == 0)
        a.seg[(size_t)a.batch * a.nseg * H * P * CN + ((size_t)b * a.nseg + sg) * H + h] = lseg;
}

// S_in(s) for every segment, in place over the workspace (thread: 4
// consecutive state entries of one sequence).  Slot s holds S_s from the
// segment pass (s < nseg - 1) and receives S_in(s).
__global__ __launch_bounds__(256) void ssd_seg_scan_kernel(SsdArgs a) {
    const size_t per_b = (size_t)a.H * a.P * CN;
    const size_t i = 4 * ((size_t)blockIdx.x * 256 + threadIdx.x);
    if (i >= (size_t)a.batch * per_b) return;
    const uint32_t b = (uint32_t)(i / per_b);
    const size_t r = i % per_b;
    const uint32_t h = (uint32_t)(r / ((size_t)a.P * CN));
    const uint32_t ns = a.nseg;
    const float* dec = a.seg + (size_t)a.batch * ns * per_b;
    floatx4 v = *reinterpret_cast<const floatx4*>(a.state + i);
    for (uint32_t s = 0; s < ns; ++s) {
        floatx4* slot = reinterpret_cast<floatx4*>(a.seg + ((size_t)b * ns + s) * per_b + r);
        if (s + 1 < ns) {
            const floatx4 loc = *slot;
            *slot = v;
            const float d = __expf(dec[((size_t)b * ns + s) * a.H + h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = d * v[e] + loc[e];
        } else {
            *slot = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Chunked scan for fp32 activations on v_mfma_f32_16x16x4_f32 (chunk 64,
// N = 128, P % 64 == 0).  No rounding between the steps (the activation dtype
// is fp32), so this is ssd_chunked.metal's arithmetic in fp32 throughout.
// Block (h * P / 64 + pb, b), four waves, wave w owns state columns
// p = 16 w .. + 16.  Per chunk, B, C and X are staged in LDS, wave 0 scans DT
// and Lcum, the waves split the ten lower tiles of G = C B^T into
// M[t][j] = G e^{Lc_t - Lc_j} DT_j (LDS), then each wave computes
//   Y^T[p][t] = e^{Lc_t} (S C^T)[p][t] + (X^T M^T)[p][t] + D x[t][p]
//   S^T[n][p] = e^{L_end} S^T[n][p] + (B^T (w o X))[n][p]
// with its state tiles S^T in registers, laid out exactly as the S update's
// MFMA writes them.  16x16x4 operands: lane l supplies A[l % 16][k = l / 16]
// and B[k = l / 16][l % 16]; D[4 (l / 16) + r][l % 16] comes back in element
// r.  The k order inside a product is free as long as both operands follow
// it, so it is chosen per product to keep the LDS reads conflict-free: state
// row i = 4 q + r of tile nt is n = 64 (nt / 4) + 16 q + 4 (nt % 4) + r.  LDS
// pitches (floats): C 129 (= 1 mod 64 banks), B 132 (= 4), X 80 (= 16),
// M 68 (= 4).
// ---------------------------------------------------------------------------
constexpr int F_CP = 129, F_BP = 132, F_XP = 80, F_MP = 68;

__device__ __forceinline__ int f_srow(int nt, int i) {   // state row (n) of tile nt, row i
    return 64 * (nt / 4) + 16 * (i / 4) + 4 * (nt % 4) + (i % 4);
}
__device__ __forceinline__ floatx4 mma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LOCAL: the segment pass of the segmented scan (state from zero, no Y).
template <bool LOCAL>
__global__ __launch_bounds__(256) void ssd_chunk_f32_mfma_kernel(SsdArgs a) {
    __shared__ float Cs[CQ * F_CP];
    __shared__ float Bs[CQ * F_BP];
    __shared__ float Xs[CQ * F_XP];
    __shared__ float Ms[CQ * F_MP];
    __shared__ float LCs[CQ], DTs[CQ], ELs[CQ], Ws[CQ];

    const uint32_t P = a.P, H = a.H, L = a.L;
    const uint32_t npb = P / 64;
    const uint32_t h = blockIdx.x / npb, pb = blockIdx.x % npb, b = blockIdx.y;
    const uint32_t p0 = pb * 64;
    const uint32_t hpg = (H / a.G) > 0 ? H / a.G : 1;
    const uint32_t g = h / hpg;
    const float* X = (const float*)a.X + (size_t)b * L * a.x_stride + (size_t)h * P + p0;
    const float* Bv = (const float*)a.B + (size_t)b * L * a.b_stride + (size_t)g * CN;
    const float* Cv = (const float*)a.C + (size_t)b * L * a.c_stride + (size_t)g * CN;
    const float* dtr = (const float*)a.dt + (size_t)b * L * a.dt_stride + h;
    float* Y = (float*)a.Y + (size_t)b * L * a.y_stride + (size_t)h * P + p0;
    float* st = a.state + (((size_t)b * H + h) * P + p0) * CN;
    // segment blockIdx.z: chunks cb .. ce - 1 (one segment: all chunks)
    const uint32_t sg = blockIdx.z, nch = (L + CQ - 1) / CQ;
    const uint32_t cb = sg * a.seg_chunks, ce = min(nch, cb + a.seg_chunks);
    float* seg_slot = a.nseg > 1 ? a.seg + ((((size_t)b * a.nseg + sg) * H + h) * P + p0) * CN : nullptr;
    const float A_h = -expf(((const float*)a.A_log)[h]);
    const float dt_b = ((const float*)a.dt_bias)[h];
    const float D_h = a.has_D ? ((const float*)a.D)[h] : 0.0f;

    const int tid = threadIdx.x, lane = tid % WAVE;
    const int w = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int li = lane % 16, lq = lane / 16;
    const int pw = 16 * w;

    // S^T tiles: sT[nt][r] = S[p = pw + li][n = f_srow(nt, 4 lq + r)] (4 consecutive n)
    floatx4 sT[8];
    const float* st_in = seg_slot ? seg_slot : st;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
        sT[nt] = LOCAL ? floatx4{0.0f, 0.0f, 0.0f, 0.0f}
                       : *reinterpret_cast<const floatx4*>(st_in + (size_t)(pw + li) * CN + f_srow(nt, 4 * lq));
    float lseg = 0.0f;

    for (uint32_t c = cb; c < ce; ++c) {
        const uint32_t t0 = c * CQ, tl = min((uint32_t)CQ, L - t0);
        // ---- stage the chunk (rows past tl as zeros) and scan DT / Lcum ----
        for (uint32_t i = tid; i < CQ * CN; i += 256) {
            const uint32_t t = i / CN, n = i % CN;
            if (!LOCAL) Cs[t * F_CP + n] = t < tl ? Cv[(size_t)(t0 + t) * a.c_stride + n] : 0.0f;
            Bs[t * F_BP + n] = t < tl ? Bv[(size_t)(t0 + t) * a.b_stride + n] : 0.0f;
        }
        for (uint32_t i = tid; i < CQ * 64; i += 256) {
            const uint32_t t = i / 64, pp = i % 64;
            Xs[t * F_XP + pp] = t < tl ? X[(size_t)(t0 + t) * a.x_stride + pp] : 0.0f;
        }
        if (w == 0) {
            float dv = 0.0f;
            if ((uint32_t)lane < tl) {
                dv = softplus_fast(dtr[(size_t)(t0 + lane) * a.dt_stride] + dt_b);
                dv = fminf(fmaxf(dv, a.dt_min), a.dt_max);
            }
            const float v = wave_prefix_sum(A_h * dv);
            const float l_end = readlane_f(v, WAVE - 1);
            LCs[lane] = v;
            DTs[lane] = dv;
            ELs[lane] = expf(v);
            Ws[lane] = expf(l_end - v) * dv;
        }
        __syncthreads();
        if (LOCAL) lseg += LCs[CQ - 1];
        // ---- M = G e^{Lc_t - Lc_j} DT_j on the ten lower tiles (J <= T) ----
        for (int kt = w; kt < (LOCAL ? 0 : 10); kt += 4) {
            constexpr uint64_t JT = 0x0ull | 0x4ull << 4 | 0x5ull << 8 | 0x8ull << 12 | 0x9ull << 16 |
                                    0xAull << 20 | 0xCull << 24 | 0xDull << 28 | 0xEull << 32 | 0xFull << 36;
            const int jt = (int)(JT >> (4 * kt)) & 15;
            const int J = jt & 3, Tt = jt >> 2;
            floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            // A = C rows t, B = B^T columns j; k = n = 16 q + ks % 16 + 64 (ks / 16)
            const float* cr = Cs + (16 * Tt + li) * F_CP + 16 * lq;
            const float* br = Bs + (16 * J + li) * F_BP + 16 * lq;
#pragma unroll
            for (int ks = 0; ks < 32; ++ks) {
                const int n = (ks % 16) + 64 * (ks / 16);
                acc = mma4(cr[n], br[n], acc);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * Tt + 4 * lq + r, j = 16 * J + li;
                const float mv = acc[r] * expf(fminf(LCs[t] - LCs[j], 0.0f)) * DTs[j];
                Ms[t * F_MP + j] = (j <= t && (uint32_t)t < tl) ? mv : 0.0f;
            }
        }
        if (!LOCAL) __syncthreads();   // (token tile Tt reads M columns j < 16 (Tt + 1) only)
        // ---- Y^T for this wave's columns ----
#pragma unroll
        for (int Tt = 0; Tt < (LOCAL ? 0 : 4); ++Tt) {
            floatx4 yo = {0.0f, 0.0f, 0.0f, 0.0f};
            const float* cr = Cs + (16 * Tt + li) * F_CP;
#pragma unroll
            for (int ks = 0; ks < 32; ++ks) {
                const int nt = ks / 4, r = ks % 4;
                yo = mma4(sT[nt][r], cr[f_srow(nt, 4 * lq + r)], yo);
            }
            const float el = ELs[16 * Tt + li];
            floatx4 y;
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] = yo[r] * el;
            // + X^T M^T over j <= 16 Tt + 15
            for (int kk = 0; kk < 4 * (Tt + 1); ++kk)
                y = mma4(Xs[(4 * kk + lq) * F_XP + pw + li], Ms[(16 * Tt + li) * F_MP + 4 * kk + lq], y);
            const int t = 16 * Tt + li;
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] += D_h * Xs[t * F_XP + pw + 4 * lq + r];
            if ((uint32_t)t < tl)
                *reinterpret_cast<floatx4*>(Y + (size_t)(t0 + t) * a.y_stride + pw + 4 * lq) = y;
        }
        // ---- S^T = e^{L_end} S^T + B^T (w o X) ----
        {
            const float dch = expf(LCs[CQ - 1]);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                floatx4 acc = sT[nt];
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] *= dch;
                const int n = f_srow(nt, li);
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const int j = 4 * kk + lq;
                    acc = mma4(Bs[j * F_BP + n], Ws[j] * Xs[j * F_XP + pw + li], acc);
                }
                sT[nt] = acc;
            }
        }
        __syncthreads();   // staging and M no longer read
    }
    if (LOCAL) {
        if (pb == 0 && tid == 0)
            a.seg[(size_t)a.batch * a.nseg * H * P * CN + ((size_t)b * a.nseg + sg) * H + h] = lseg;
    } else if (sg + 1 != a.nseg) {
        return;
    }
    float* out = LOCAL ? seg_slot : st;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
        *reinterpret_cast<floatx4*>(out + (size_t)(pw + li) * CN + f_srow(nt, 4 * lq)) = sT[nt];
}

template <typename T, bool GATE>
hipError_t step_go(hipStream_t s, const SsdArgs& a) {
    // vector path: 4-element B / C vectors aligned, fp32 state 16-byte aligned
    const size_t v4 = 4 * sizeof(T);
    const bool vec = ((uintptr_t)a.state % 16 == 0) && ((uintptr_t)a.B % v4 == 0) &&
                     ((uintptr_t)a.C % v4 == 0) && (a.b_stride % 4 == 0) && (a.c_stride % 4 == 0);
    if (a.yfrag) {
        if constexpr (__is_same(T, bf16) && GATE) {
            if (!vec || ssd_step_parts(a.H, a.P, a.N, a.act) == 0 || !a.ypart || !a.ynorm_w ||
                (uintptr_t)a.yfrag % 16)
                return hipErrorInvalidValue;
            const dim3 gf(a.H * a.P / (4 * ST_RB), a.batch);
            if (a.N == 128) ssd_step_kernel<T, 4, GATE, true><<<gf, 4 * ST_NT, 0, s>>>(a);
            else if (a.N == 64) ssd_step_kernel<T, 2, GATE, true><<<gf, 4 * ST_NT, 0, s>>>(a);
            else if (a.N == 256) ssd_step_kernel<T, 8, GATE, true><<<gf, 4 * ST_NT, 0, s>>>(a);
            else ssd_step_kernel<T, 1, GATE, true><<<gf, 4 * ST_NT, 0, s>>>(a);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    const dim3 grid(a.H * ((a.P + ST_RB - 1) / ST_RB), a.batch);
    if (vec && a.N == 128) ssd_step_kernel<T, 4, GATE><<<grid, ST_NT, 0, s>>>(a);
    else if (vec && a.N == 64) ssd_step_kernel<T, 2, GATE><<<grid, ST_NT, 0, s>>>(a);
    else if (vec && a.N == 256) ssd_step_kernel<T, 8, GATE><<<grid, ST_NT, 0, s>>>(a);
    else if (vec && a.N == 32) ssd_step_kernel<T, 1, GATE><<<grid, ST_NT, 0, s>>>(a);
    else ssd_step_generic_kernel<T, GATE><<<dim3(a.H, a.batch), ((a.P + 63) / 64) * 64, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

uint32_t ssd_step_parts(uint32_t H, uint32_t P, uint32_t N, int act) {
    const uint32_t HP = H * P;
    const bool n_ok = N == 32 || N == 64 || N == 128 || N == 256;
    return act == LSSM_BF16 && n_ok && HP % 128 == 0 && HP / 32 <= GEMV_MAX_XPARTS ? HP / 32 : 0;
}

hipError_t launch_ssd_step(hipStream_t s, const SsdArgs& a) {
    if (a.batch == 0 || a.H == 0) return hipSuccess;
    const bool gate = a.z != nullptr;
    if (a.act == LSSM_F16) return gate ? step_go<f16, true>(s, a) : step_go<f16, false>(s, a);
    if (a.act == LSSM_BF16) return gate ? step_go<bf16, true>(s, a) : step_go<bf16, false>(s, a);
    return gate ? step_go<float, true>(s, a) : step_go<float, false>(s, a);
}

// Segments per sequence of the chunked scan: enough for about two blocks per
// CU when the (sequence, head, column block) walks alone would leave CUs
// idle, as many as the workspace holds, none without a workspace.
// LSSM_SSD_SEGMENTS overrides the count (read once).
static uint32_t pick_segments(const SsdArgs& a, size_t nblk0) {
    const uint32_t nch = (a.L + CQ - 1) / CQ;
    if (!a.seg || nch < 2) return 1;
    static const int env = [] {
        const char* e = getenv("LSSM_SSD_SEGMENTS");
        return e ? atoi(e) : 0;
    }();
    const size_t cus = num_cus();
    size_t ns = env > 0 ? (size_t)env : (nblk0 >= cus ? 1 : (2 * cus + nblk0 - 1) / nblk0);
    ns = std::min(ns, (size_t)nch);
    const size_t per = (size_t)a.batch * a.H * a.P * CN;   // floats of one segment slot, all sequences
    while (ns > 1 && (ns * per > SSD_SEG_STATE_FLOATS || ns * a.batch * a.H > SSD_SEG_DECAY_FLOATS)) --ns;
    if (ns <= 1) return 1;
    const uint32_t K = (nch + (uint32_t)ns - 1) / (uint32_t)ns;
    return (nch + K - 1) / K;                              // no empty segment
}

namespace {
// A single partial chunk (L < 64, chunk == L) has the same rounding points as
// chunk 64, so it also takes the MFMA path.
bool chunk_ok(const SsdArgs& a) { return a.chunk == CQ || (a.chunk == a.L && a.L < CQ); }
bool mfma_ok(const SsdArgs& a) {
    return (a.act != LSSM_F32) && chunk_ok(a) && a.N == CN && (a.P % 32) == 0 && (a.x_stride % 8 == 0) &&
           (a.b_stride % 8 == 0) && (a.c_stride % 8 == 0) && (a.y_stride % 4 == 0) &&
           ((uintptr_t)a.X % 16 == 0) && ((uintptr_t)a.B % 16 == 0) && ((uintptr_t)a.C % 16 == 0) &&
           ((uintptr_t)a.Y % 8 == 0) && ((uintptr_t)a.state % 16 == 0);
}
// Four waves (64 columns of P) per block when that still gives a block per
// CU, or when segments make up the count; otherwise two, for more blocks.
bool walk_nw4(const SsdArgs& a, size_t cus) {
    const uint32_t nch = (a.L + CQ - 1) / CQ;
    const size_t nb64 = (size_t)a.batch * a.H * (a.P / 64);
    return (a.P % 64) == 0 && (nb64 >= cus || (a.seg && nch >= 2));
}

// rs[row] = 1 / sqrt(sum_k part[k][row] / dim + eps).  A block takes 64 rows;
// wave w adds parts w, w + 4, ... of its lane's row (each load instruction
// reads 256 consecutive bytes), then the four waves' sums meet in LDS in a
// fixed order.
__global__ __launch_bounds__(256) void rms_from_parts_kernel(const float* __restrict__ part, uint32_t nparts,
                                                             uint32_t rows, float inv_dim, float eps,
                                                             float* __restrict__ rs) {
    __shared__ float red[4][64];
    const uint32_t lane = threadIdx.x % WAVE, w = threadIdx.x / WAVE;
    const uint32_t row = blockIdx.x * 64 + lane;
    float v = 0.0f;
    if (row < rows) {
        // eight loads in flight, added in the order of k
        const float* p = part + row;
        uint32_t k = w;
        for (; k + 28 < nparts; k += 32) {
            float a[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = __builtin_nontemporal_load(p + (size_t)(k + 4 * u) * rows);
#pragma unroll
            for (int u = 0; u < 8; ++u) v += a[u];
        }
        for (; k < nparts; k += 4) v += __builtin_nontemporal_load(p + (size_t)k * rows);
    }
    red[w][lane] = v;
    __syncthreads();
    if (w == 0 && row < rows)
        rs[row] = 1.0f / sqrtf(((red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane])) * inv_dim + eps);
}
}  // namespace

uint32_t ssd_chunked_gate_parts(const SsdArgs& a) {
    if (a.batch == 0 || a.H == 0 || a.L == 0 || !mfma_ok(a) || !a.z_silu) return 0;
    if (!a.z || !a.gnorm_w || a.z_stride % 4 != 0 || (uintptr_t)a.z % 8 != 0 ||
        (uintptr_t)a.gnorm_w % 8 != 0)
        return 0;
    return a.H * (a.P / (walk_nw4(a, num_cus()) ? 64u : 32u));
}

hipError_t launch_rms_from_parts(hipStream_t s, const float* part, uint32_t nparts, uint32_t rows,
                                 uint32_t dim, float eps, float* rs) {
    if (rows == 0) return hipSuccess;
    rms_from_parts_kernel<<<(rows + 63) / 64, 256, 0, s>>>(part, nparts, rows, 1.0f / (float)dim, eps, rs);
    return hipGetLastError();
}

hipError_t launch_ssd_chunked(hipStream_t s, const SsdArgs& a0) {
    if (a0.batch == 0 || a0.H == 0 || a0.L == 0) return hipSuccess;
    SsdArgs a = a0;
    const uint32_t nch = (a.L + CQ - 1) / CQ;
    a.nseg = 1;
    a.seg_chunks = nch;
    const size_t cus = num_cus();
    if (a.gpart && ssd_chunked_gate_parts(a) == 0) return hipErrorInvalidValue;
    // segment pass + the scan of the segments' states (a.nseg > 1)
    auto seg_scan = [&]() {
        const size_t n4 = (size_t)a.batch * a.H * a.P * CN / 4;
        ssd_seg_scan_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, s>>>(a);
    };
    if (mfma_ok(a)) {
        const bool p64 = (a.P % 64) == 0;
        const bool nw4 = walk_nw4(a, cus);
        const uint32_t pbw = nw4 ? 64 : 32;
        a.nseg = pick_segments(a, (size_t)a.batch * a.H * (a.P / pbw));
        a.seg_chunks = (nch + a.nseg - 1) / a.nseg;
        const bool gp = a.gram != nullptr;
        auto go = [&](auto tag) {
            using T = decltype(tag);
            if (gp) {
                const dim3 gg(nch, a.G, a.batch);
                ssd_gram_kernel<T><<<gg, 256, 0, s>>>(a);
            }
            if (a.nseg > 1) {
                if (p64) ssd_seg_state_kernel<T, 4><<<dim3(a.H * (a.P / 64), a.batch, a.nseg - 1), 256, 0, s>>>(a);
                else ssd_seg_state_kernel<T, 2><<<dim3(a.H * (a.P / 32), a.batch, a.nseg - 1), 128, 0, s>>>(a);
                seg_scan();
            }
            // two waves per 16-column slice (SPL = 2) when the grid does not
            // fill the chip anyway (then every block has a CU to itself and
            // the shorter chain wins; with more blocks than CUs the larger
            // register footprint of SPL = 2 costs a second round of blocks)
            const size_t nblk = (size_t)a.batch * a.H * (a.P / pbw) * a.nseg;
            const bool split = nblk <= cus;
            const dim3 grid(a.H * (a.P / pbw), a.batch, a.nseg);
            if (nw4) {
                if (split) {
                    if (gp) ssd_chunk_mfma_kernel<T, 4, true, 2><<<grid, 512, 0, s>>>(a);
                    else ssd_chunk_mfma_kernel<T, 4, false, 2><<<grid, 512, 0, s>>>(a);
                } else {
                    if (gp) ssd_chunk_mfma_kernel<T, 4, true, 1><<<grid, 256, 0, s>>>(a);
                    else ssd_chunk_mfma_kernel<T, 4, false, 1><<<grid, 256, 0, s>>>(a);
                }
            } else {
                if (split) {
                    if (gp) ssd_chunk_mfma_kernel<T, 2, true, 2><<<grid, 256, 0, s>>>(a);
                    else ssd_chunk_mfma_kernel<T, 2, false, 2><<<grid, 256, 0, s>>>(a);
                } else {
                    if (gp) ssd_chunk_mfma_kernel<T, 2, true, 1><<<grid, 128, 0, s>>>(a);
                    else ssd_chunk_mfma_kernel<T, 2, false, 1><<<grid, 128, 0, s>>>(a);
                }
            }
        };
        if (a.act == LSSM_F16) go(f16{});
        else go(bf16{});
        return hipGetLastError();
    }
    if (a.act == LSSM_F32 && chunk_ok(a) && a.N == CN && (a.P % 64) == 0 && ((uintptr_t)a.state % 16 == 0) &&
        ((uintptr_t)a.Y % 16 == 0) && (a.y_stride % 4 == 0)) {
        a.nseg = pick_segments(a, (size_t)a.batch * a.H * (a.P / 64));
        a.seg_chunks = (nch + a.nseg - 1) / a.nseg;
        if (a.nseg > 1) {
            ssd_chunk_f32_mfma_kernel<true><<<dim3(a.H * (a.P / 64), a.batch, a.nseg - 1), 256, 0, s>>>(a);
            seg_scan();
        }
        ssd_chunk_f32_mfma_kernel<false><<<dim3(a.H * (a.P / 64), a.batch, a.nseg), 256, 0, s>>>(a);
        return hipGetLastError();
    }
    if (a.chunk > (uint32_t)SC_MAXCK || a.N > (uint32_t)SC_MAXN) return hipErrorInvalidValue;
    dim3 grid(a.H * ((a.P + SC_PB - 1) / SC_PB), a.batch);
    if (a.act == LSSM_F16) ssd_chunk_scalar_kernel<f16><<<grid, SC_NT, 0, s>>>(a);
    else if (a.act == LSSM_BF16) ssd_chunk_scalar_kernel<bf16><<<grid, SC_NT, 0, s>>>(a);
    else ssd_chunk_scalar_kernel<float><<<grid, SC_NT, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace lssm

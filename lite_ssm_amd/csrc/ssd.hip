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
#include <cfloat>

#include "common.cuh"
#include "internal.hpp"

namespace lssm {

namespace {

// ---------------------------------------------------------------------------
// Decode step.  Block (h * PS + ps, b), 256 threads, owns 32 rows p of one
// head's (P, N) fp32 state: 8 lanes per row, each streaming F = N / 32 float4
// of state.  Every load is issued first and unconditionally (state, the
// lane's B and C vectors, then the per-row / per-head scalars as raw bits), so
// nothing waits before the math; the 8 lanes of a row reduce C.s with
// shuffles.  2.7B at batch 1: 160 blocks, 4 x 16-byte state loads per thread.
// ---------------------------------------------------------------------------
constexpr int ST_NV = 8;                              // lanes per state row
constexpr int ST_RB = 256 / ST_NV;                    // rows per block

template <typename T> __device__ __forceinline__ uint32_t raw_of(const T* p) {
    if constexpr (sizeof(T) == 2) return *reinterpret_cast<const uint16_t*>(p);
    else return *reinterpret_cast<const uint32_t*>(p);
}
template <typename T> __device__ __forceinline__ float f_of(uint32_t r) {
    if constexpr (sizeof(T) == 2) return to_f(__builtin_bit_cast(T, (uint16_t)r));
    else return __uint_as_float(r);
}

template <typename T, int F, bool GATE>
__global__ __launch_bounds__(256) void ssd_step_kernel(SsdArgs a) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const uint32_t P = a.P, N = a.N;
    const uint32_t PS = (P + ST_RB - 1) / ST_RB;
    const uint32_t h = blockIdx.x / PS, ps = blockIdx.x % PS, b = blockIdx.y;
    const uint32_t p = ps * ST_RB + threadIdx.x / ST_NV;
    if (p >= P) return;                               // whole 8-lane row groups exit together
    const uint32_t g = h / (a.H / a.G);
    const uint32_t lr = threadIdx.x % ST_NV;
    f32x4* S = reinterpret_cast<f32x4*>(a.state + (((size_t)b * a.H + h) * P + p) * N);
    const T4* B4 = reinterpret_cast<const T4*>((const T*)a.B + (size_t)b * a.b_stride + (size_t)g * N);
    const T4* C4 = reinterpret_cast<const T4*>((const T*)a.C + (size_t)b * a.c_stride + (size_t)g * N);
    f32x4 s[F];
    T4 bv[F], cv[F];
#pragma unroll
    for (int f = 0; f < F; ++f) s[f] = S[lr + ST_NV * f];
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
        f32x4 t = s[f];
        t.x = decay * t.x + dt * to_f(bv[f].x) * xv;
        t.y = decay * t.y + dt * to_f(bv[f].y) * xv;
        t.z = decay * t.z + dt * to_f(bv[f].z) * xv;
        t.w = decay * t.w + dt * to_f(bv[f].w) * xv;
        S[lr + ST_NV * f] = t;
        ys += to_f(cv[f].x) * t.x + to_f(cv[f].y) * t.y + to_f(cv[f].z) * t.z + to_f(cv[f].w) * t.w;
    }
    ys = group_sum<ST_NV>(ys);
    if (lr == 0) {
        float y = rnd<T>(ys + (a.has_D ? f_of<T>(dr) : 0.0f) * xv);
        if constexpr (GATE) y = silu_fast(f_of<T>(zr)) * y;
        ((T*)a.Y)[(size_t)b * a.y_stride + (size_t)h * P + p] = from_f<T>(y);
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
// Chunked scan on MFMA (fp16 / bf16), chunk = 64, N = 128, P % 32 == 0.
// Block (h * P/32 + pb, b), 256 threads = 4 waves, owns 32 columns of P.
// Per chunk, with v_mfma_f32_16x16x32 (lane l: A row l%16 / B column l%16,
// k = (l/16)*8 .. +8; D element r at row (l/16)*4 + r, column l%16):
//   G  = C_c . B_c^T          [64 x 64]  K = 128   (wave w: rows 16w..16w+15)
//   M  = r(G o decay o DT) -> LDS
//   Y  = M . X_c + e^{Lcum} (C_c . S^T) + D x     [64 x 32]
//   S  = r(e^{L_end} S + (X_c o w)^T . B_c)        [32 x 128], fp32 in registers
// The rounded S is also kept in LDS as the B operand of the next C_c . S^T.
// ---------------------------------------------------------------------------
constexpr int MF_NT = 256;
constexpr int MF_Q = 64;      // chunk
constexpr int MF_N = 128;     // state size
constexpr int MF_PB = 32;     // P columns per block
constexpr int NPAD = MF_N + 8;
constexpr int QPAD = MF_Q + 8;

template <typename T> struct Mfma16;
template <> struct Mfma16<f16> {
    using frag = half8;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma16<bf16> {
    using frag = bf16x8;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <typename T>
__global__ __launch_bounds__(MF_NT) void ssd_chunk_mfma_kernel(SsdArgs a) {
    __shared__ __attribute__((aligned(16))) T Cc[MF_Q * NPAD];
    __shared__ __attribute__((aligned(16))) T Bc[MF_Q * NPAD];
    __shared__ __attribute__((aligned(16))) T Sl[MF_PB * NPAD];
    __shared__ __attribute__((aligned(16))) T Xt[MF_PB * QPAD];
    __shared__ __attribute__((aligned(16))) T Ml[MF_Q * QPAD];
    __shared__ float DT[MF_Q], Lc[MF_Q];
    using Op = Mfma16<T>;
    using frag = typename Op::frag;

    const uint32_t P = a.P, H = a.H, L = a.L;
    const uint32_t npb = P / MF_PB;
    const uint32_t h = blockIdx.x / npb, pb = blockIdx.x % npb, b = blockIdx.y;
    const uint32_t p0 = pb * MF_PB;
    const uint32_t hpg = (H / a.G) > 0 ? H / a.G : 1;
    const uint32_t g = h / hpg;
    const T* X = (const T*)a.X + (size_t)b * L * a.x_stride + (size_t)h * P + p0;
    const T* Bv = (const T*)a.B + (size_t)b * L * a.b_stride + (size_t)g * MF_N;
    const T* Cv = (const T*)a.C + (size_t)b * L * a.c_stride + (size_t)g * MF_N;
    const T* dtr = (const T*)a.dt + (size_t)b * L * a.dt_stride + h;
    T* Y = (T*)a.Y + (size_t)b * L * a.y_stride + (size_t)h * P + p0;
    float* st = a.state + (((size_t)b * H + h) * P + p0) * MF_N;
    const float A_h = -expf(to_f(((const T*)a.A_log)[h]));
    const float dt_b = to_f(((const T*)a.dt_bias)[h]);
    const float D_h = a.has_D ? to_f(((const T*)a.D)[h]) : 0.0f;

    const int tid = threadIdx.x;
    const int lane = tid % WAVE;
    const int w = tid / WAVE;
    const int l16 = lane % 16, kq = (lane / 16) * 8;

    // State tiles owned by wave w: S rows (p) 16*(w%2) .. +16, columns (n)
    // 64*(w/2) .. +64 = 4 tiles of 16 x 16.
    const int sp0 = 16 * (w % 2);
    const int sn0 = 64 * (w / 2);
    floatx4 sacc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = sp0 + (lane / 16) * 4 + r;
            const int n = sn0 + 16 * j + l16;
            const float v = rnd<T>(st[(size_t)p * MF_N + n]);
            sacc[j][r] = v;
            Sl[p * NPAD + n] = from_f<T>(v);
        }

    for (uint32_t t0 = 0; t0 < L; t0 += MF_Q) {
        const uint32_t tl = min((uint32_t)MF_Q, L - t0);
        __syncthreads();
        // ---- stage B_c, C_c [64 x 128] and X_c^T [32 x 64]; zero past tl ----
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = tid + MF_NT * i;          // 1024 chunks of 8 elements
            const int t = id / 16, c8 = (id % 16) * 8;
            uint4 bv = make_uint4(0, 0, 0, 0), cv = make_uint4(0, 0, 0, 0);
            if ((uint32_t)t < tl) {
                bv = *reinterpret_cast<const uint4*>(Bv + (size_t)(t0 + t) * a.b_stride + c8);
                cv = *reinterpret_cast<const uint4*>(Cv + (size_t)(t0 + t) * a.c_stride + c8);
            }
            *reinterpret_cast<uint4*>(Bc + t * NPAD + c8) = bv;
            *reinterpret_cast<uint4*>(Cc + t * NPAD + c8) = cv;
        }
        {
            const int t = tid / 4, c8 = (tid % 4) * 8;   // 256 chunks: 64 tokens x 4
            uint4 xv = make_uint4(0, 0, 0, 0);
            if ((uint32_t)t < tl) xv = *reinterpret_cast<const uint4*>(X + (size_t)(t0 + t) * a.x_stride + c8);
            const T* xe = reinterpret_cast<const T*>(&xv);
#pragma unroll
            for (int e = 0; e < 8; ++e) Xt[(c8 + e) * QPAD + t] = xe[e];
        }
        if (w == 0) {
            float v = 0.0f, dv = 0.0f;
            if ((uint32_t)lane < tl) {
                dv = softplus_f(to_f(dtr[(size_t)(t0 + lane) * a.dt_stride]) + dt_b);
                dv = fminf(fmaxf(dv, a.dt_min), a.dt_max);
                v = A_h * dv;
            }
#pragma unroll
            for (int off = 1; off < WAVE; off <<= 1) {
                const float o = __shfl_up(v, off, WAVE);
                if (lane >= off) v += o;
            }
            DT[lane] = dv;
            Lc[lane] = v;
        }
        __syncthreads();
        const float L_end = Lc[tl - 1];

        // ---- G = C_c . B_c^T, M = r(G o e^{Lc_t - Lc_j} o DT_j) (j <= t) ----
        {
            const int t_base = 16 * w;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                floatx4 gacc = {0.0f, 0.0f, 0.0f, 0.0f};
                if (jt * 16 <= t_base + 15) {
#pragma unroll
                    for (int ks = 0; ks < MF_N / 32; ++ks) {
                        const frag af = *reinterpret_cast<const frag*>(Cc + (t_base + l16) * NPAD + ks * 32 + kq);
                        const frag bf = *reinterpret_cast<const frag*>(Bc + (jt * 16 + l16) * NPAD + ks * 32 + kq);
                        gacc = Op::mma(af, bf, gacc);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = t_base + (lane / 16) * 4 + r;
                    const int j = jt * 16 + l16;
                    float m = 0.0f;
                    if (j <= t && (uint32_t)t < tl) m = gacc[r] * expf(Lc[t] - Lc[j]) * DT[j];
                    Ml[t * QPAD + j] = from_f<T>(m);
                }
            }
        }
        __syncthreads();

        // ---- Y tiles: wave w owns rows 16w..16w+15 x the 2 column tiles of PB ----
        {
            const int t_base = 16 * w;
#pragma unroll
            for (int pt = 0; pt < MF_PB / 16; ++pt) {
                floatx4 yi = {0.0f, 0.0f, 0.0f, 0.0f}, yo = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < MF_Q / 32; ++ks) {
                    const frag af = *reinterpret_cast<const frag*>(Ml + (t_base + l16) * QPAD + ks * 32 + kq);
                    const frag bf = *reinterpret_cast<const frag*>(Xt + (pt * 16 + l16) * QPAD + ks * 32 + kq);
                    yi = Op::mma(af, bf, yi);
                }
#pragma unroll
                for (int ks = 0; ks < MF_N / 32; ++ks) {
                    const frag af = *reinterpret_cast<const frag*>(Cc + (t_base + l16) * NPAD + ks * 32 + kq);
                    const frag bf = *reinterpret_cast<const frag*>(Sl + (pt * 16 + l16) * NPAD + ks * 32 + kq);
                    yo = Op::mma(af, bf, yo);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = t_base + (lane / 16) * 4 + r;
                    const int p = pt * 16 + l16;
                    if ((uint32_t)t < tl) {
                        const float xc = to_f(Xt[p * QPAD + t]);
                        const float y = yi[r] + yo[r] * expf(Lc[t]) + D_h * xc;
                        Y[(size_t)(t0 + t) * a.y_stride + p] = from_f<T>(y);
                    }
                }
            }
        }
        __syncthreads();

        // ---- S = r(e^{L_end} S + (X_c o w)^T . B_c), w_j = e^{L_end - Lc_j} DT_j ----
        {
            const float dch = expf(L_end);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) sacc[j][r] *= dch;
#pragma unroll
            for (int ks = 0; ks < MF_Q / 32; ++ks) {
                // A[p][j] = w_j X[j][p], rounded to T (one extra rounding vs the
                // fp32 sum of the reference)
                frag af;
                const int jb = ks * 32 + kq;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int jj = jb + e;
                    const float wj = ((uint32_t)jj < tl) ? expf(L_end - Lc[jj]) * DT[jj] : 0.0f;
                    af[e] = from_f<T>(wj * to_f(Xt[(sp0 + l16) * QPAD + jj]));
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    frag bf;
                    const int n = sn0 + 16 * j + l16;
#pragma unroll
                    for (int e = 0; e < 8; ++e) bf[e] = Bc[(jb + e) * NPAD + n];
                    sacc[j] = Op::mma(af, bf, sacc[j]);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = rnd<T>(sacc[j][r]);
                    sacc[j][r] = v;
                    Sl[(sp0 + (lane / 16) * 4 + r) * NPAD + sn0 + 16 * j + l16] = from_f<T>(v);
                }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            st[(size_t)(sp0 + (lane / 16) * 4 + r) * MF_N + sn0 + 16 * j + l16] = sacc[j][r];
}

template <typename T, bool GATE>
hipError_t step_go(hipStream_t s, const SsdArgs& a) {
    // vector path: 4-element B / C vectors aligned, fp32 state 16-byte aligned
    const size_t v4 = 4 * sizeof(T);
    const bool vec = ((uintptr_t)a.state % 16 == 0) && ((uintptr_t)a.B % v4 == 0) &&
                     ((uintptr_t)a.C % v4 == 0) && (a.b_stride % 4 == 0) && (a.c_stride % 4 == 0);
    const dim3 grid(a.H * ((a.P + ST_RB - 1) / ST_RB), a.batch);
    if (vec && a.N == 128) ssd_step_kernel<T, 4, GATE><<<grid, 256, 0, s>>>(a);
    else if (vec && a.N == 64) ssd_step_kernel<T, 2, GATE><<<grid, 256, 0, s>>>(a);
    else if (vec && a.N == 256) ssd_step_kernel<T, 8, GATE><<<grid, 256, 0, s>>>(a);
    else if (vec && a.N == 32) ssd_step_kernel<T, 1, GATE><<<grid, 256, 0, s>>>(a);
    else ssd_step_generic_kernel<T, GATE><<<dim3(a.H, a.batch), ((a.P + 63) / 64) * 64, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_ssd_step(hipStream_t s, const SsdArgs& a) {
    if (a.batch == 0 || a.H == 0) return hipSuccess;
    const bool gate = a.z != nullptr;
    if (a.act == LSSM_F16) return gate ? step_go<f16, true>(s, a) : step_go<f16, false>(s, a);
    if (a.act == LSSM_BF16) return gate ? step_go<bf16, true>(s, a) : step_go<bf16, false>(s, a);
    return gate ? step_go<float, true>(s, a) : step_go<float, false>(s, a);
}

hipError_t launch_ssd_chunked(hipStream_t s, const SsdArgs& a) {
    if (a.batch == 0 || a.H == 0 || a.L == 0) return hipSuccess;
    // A single partial chunk (L < 64, chunk == L) has the same rounding points
    // as chunk 64, so it also takes the MFMA path.
    const bool chunk_ok = a.chunk == MF_Q || (a.chunk == a.L && a.L < MF_Q);
    const bool mfma_ok = (a.act != LSSM_F32) && chunk_ok && a.N == MF_N && (a.P % MF_PB) == 0 &&
                         (a.x_stride % 8 == 0) && (a.b_stride % 8 == 0) && (a.c_stride % 8 == 0) &&
                         ((uintptr_t)a.X % 16 == 0) && ((uintptr_t)a.B % 16 == 0) &&
                         ((uintptr_t)a.C % 16 == 0);
    if (mfma_ok) {
        dim3 grid(a.H * (a.P / MF_PB), a.batch);
        if (a.act == LSSM_F16) ssd_chunk_mfma_kernel<f16><<<grid, MF_NT, 0, s>>>(a);
        else ssd_chunk_mfma_kernel<bf16><<<grid, MF_NT, 0, s>>>(a);
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

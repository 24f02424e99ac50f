// gemv.hip — dequantize-in-register GEMV for decode (M <= 4 rows of x).
//
// Y[m, n] = epi( sum_k deq(W)[n, k] * x[m, k] ), W row-major [N, K] in one of
// the formats of lssm_wfmt.  Restates linear.metal:440-474 (int4 GEMV: exact
// fp32 dequant float(q) * float(scale), fp32 accumulation, one rounding at the
// store) and linear.metal:82-109 (dense fp16 GEMV).
//
// Mapping (MI355X): 256-thread blocks = 4 waves; 16 lanes per weight row, so a
// wave streams 4 rows and a block 16 rows.  Each lane owns 16-byte chunks of
// its row (32 int4 / 16 int8 / 8 dense weights) strided by 16 chunks, issues
// up to U chunk loads back to back, and only then dequantizes: every weight
// byte is read from HBM exactly once with 16-byte vector loads.  The x rows are
// staged once per block in LDS as fp32 (optionally through a fused RMSNorm
// prologue), and the 16 partial sums of a row are combined with cross-lane
// shuffles.
#include "common.cuh"
#include "internal.hpp"

namespace lssm {

namespace {

constexpr int GV_NT = 256;
constexpr int GV_LPR = 16;                       // lanes per weight row
constexpr int GV_ROWS = GV_NT / GV_LPR;          // rows per block
constexpr int GV_U = 4;                          // chunks in flight per lane
constexpr size_t GV_LDS_MAX = GEMV_LDS_BYTES;

struct GemvCore {
    const void* x;
    uint32_t x_stride;
    const uint8_t* w;
    const uint16_t* s;
    const void* norm_w;
    float eps;
    uint32_t N, K;
};

template <int FMT, typename T> struct Fmt;
template <typename T> struct Fmt<LSSM_W_Q4_B32, T> {
    static constexpr int WPC = 32, G = 32;       // weights per 16-byte chunk, group size
    static __device__ __forceinline__ size_t row_bytes(uint32_t K) { return K / 2; }
};
template <typename T> struct Fmt<LSSM_W_Q4_G64, T> {
    static constexpr int WPC = 32, G = 64;
    static __device__ __forceinline__ size_t row_bytes(uint32_t K) { return K / 2; }
};
template <typename T> struct Fmt<LSSM_W_Q8_G32, T> {
    static constexpr int WPC = 16, G = 32;
    static __device__ __forceinline__ size_t row_bytes(uint32_t K) { return K; }
};
template <typename T> struct Fmt<LSSM_W_DENSE, T> {
    static constexpr int WPC = 16 / (int)sizeof(T), G = 0;
    static __device__ __forceinline__ size_t row_bytes(uint32_t K) { return (size_t)K * sizeof(T); }
};

// Dot of one 16-byte weight chunk with WPC fp32 x values (x points into LDS).
template <int FMT, typename T>
__device__ __forceinline__ float chunk_dot(const uint4 wv, const float* __restrict__ xr) {
    const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
    float acc = 0.0f;
    if constexpr (FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64) {
        // nibble j of dword i is weight 8*i + j (low nibble = even k, linear.metal:47-61)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int q = ((int)(d[i] << (28 - 4 * j))) >> 28;   // sign-extended nibble
                acc += (float)q * xr[8 * i + j];
            }
        }
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int q = ((int)(d[i] << (24 - 8 * j))) >> 24;
                acc += (float)q * xr[4 * i + j];
            }
        }
    } else {
        const T* wt = reinterpret_cast<const T*>(d);
#pragma unroll
        for (int i = 0; i < 16 / (int)sizeof(T); ++i) acc += to_f(wt[i]) * xr[i];
    }
    return acc;
}

// Epilogue: y[m, n] = r(acc) / r(silu(acc)) / r(res + r(acc)).
template <typename T, int EPI> struct EpiPlain {
    T* y;
    uint32_t y_stride;
    const T* res;
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc) const {
        const size_t i = (size_t)m * y_stride + n;
        float v = acc;
        if (EPI == LSSM_EPI_SILU) v = silu_f(acc);
        if (EPI == LSSM_EPI_ADD) v = to_f(res[i]) + rnd<T>(acc);
        y[i] = from_f<T>(v);
    }
};

// Engine decode in_proj epilogue: rows [0, d_inner) -> z, rows of xBC ->
// depthwise conv update (conv1d.metal:108-137) + SiLU (activations.metal:49-73)
// -> xbc_act, remaining rows -> dt.  The pre-conv xBC value is r(acc), the conv
// output is rounded once more before SiLU, as in the unfused op sequence.
template <typename T> struct EpiInproj {
    uint32_t d_inner, xbc, H, dconv;
    T* conv_state;
    const T* conv_w;
    const T* conv_b;
    T* z;
    T* xbc_act;
    T* dt;
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc) const {
        const T v = from_f<T>(acc);
        if (n < d_inner) {
            z[(size_t)m * d_inner + n] = v;
        } else if (n < d_inner + xbc) {
            const uint32_t c = n - d_inner;
            T* sd = conv_state + ((size_t)m * xbc + c) * dconv;
            const T* wd = conv_w + (size_t)c * dconv;
            float a = to_f(conv_b[c]);
            for (uint32_t k = 0; k + 1 < dconv; ++k) {
                const T sk = sd[k + 1];
                sd[k] = sk;
                a += to_f(sk) * to_f(wd[k]);
            }
            sd[dconv - 1] = v;
            a += to_f(v) * to_f(wd[dconv - 1]);
            xbc_act[(size_t)m * xbc + c] = from_f<T>(silu_f(rnd<T>(a)));
        } else {
            dt[(size_t)m * H + (n - d_inner - xbc)] = v;
        }
    }
};

template <int FMT, typename T, int MR, bool NORM, class Epi>
__global__ __launch_bounds__(GV_NT) void gemv_kernel(GemvCore c, Epi epi) {
    extern __shared__ float xs[];                 // [MR][K] fp32
    __shared__ float red[GV_NT / WAVE];
    using F = Fmt<FMT, T>;
    const uint32_t K = c.K;
    const T* x = reinterpret_cast<const T*>(c.x);

    // ---- stage x (optionally RMSNorm'ed, norm.metal:52-79) into LDS ----
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const T* xr = x + (size_t)m * c.x_stride;
        if constexpr (NORM) {
            const T* nw = reinterpret_cast<const T*>(c.norm_w);
            float ss = 0.0f;
            for (uint32_t k = threadIdx.x; k < K; k += GV_NT) {
                const float v = to_f(xr[k]);
                ss += v * v;
            }
            ss = block_sum<GV_NT>(ss, red);
            const float rrms = 1.0f / sqrtf(ss / (float)K + c.eps);
            for (uint32_t k = threadIdx.x; k < K; k += GV_NT)
                xs[m * K + k] = rnd<T>(to_f(xr[k]) * to_f(nw[k]) * rrms);
        } else {
            for (uint32_t k = threadIdx.x; k < K; k += GV_NT) xs[m * K + k] = to_f(xr[k]);
        }
    }
    __syncthreads();

    const int lane = threadIdx.x % WAVE;
    const int wv = threadIdx.x / WAVE;
    const int lr = lane % GV_LPR;                       // lane within row
    const uint32_t n = blockIdx.x * GV_ROWS + wv * (WAVE / GV_LPR) + lane / GV_LPR;
    const bool live = n < c.N;
    const uint32_t cpr = K / F::WPC;                     // chunks per row
    const uint8_t* wrow = c.w + (size_t)(live ? n : 0) * F::row_bytes(K);
    const uint32_t gpr = F::G ? K / F::G : 0;

    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;

    if (live) {
        for (uint32_t c0 = lr; c0 < cpr; c0 += GV_LPR * GV_U) {
            uint4 wq[GV_U];
            float sc[GV_U];
#pragma unroll
            for (int u = 0; u < GV_U; ++u) {
                const uint32_t ch = c0 + u * GV_LPR;
                if (ch < cpr) {
                    wq[u] = *reinterpret_cast<const uint4*>(wrow + (size_t)ch * 16);
                    if constexpr (F::G > 0)
                        sc[u] = fp16_bits_to_f(c.s[(size_t)n * gpr + (ch * F::WPC) / F::G]);
                    else
                        sc[u] = 1.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < GV_U; ++u) {
                const uint32_t ch = c0 + u * GV_LPR;
                if (ch < cpr) {
#pragma unroll
                    for (int m = 0; m < MR; ++m)
                        acc[m] += chunk_dot<FMT, T>(wq[u], xs + m * K + ch * F::WPC) * sc[u];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = group_sum<GV_LPR>(acc[m]);
    if (live && lr == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) epi(m, n, acc[m]);
    }
}

template <int FMT, typename T, int MR, bool NORM, class Epi>
hipError_t launch_one(hipStream_t s, const GemvCore& c, const Epi& e) {
    const size_t lds = (size_t)MR * c.K * sizeof(float);
    auto kern = gemv_kernel<FMT, T, MR, NORM, Epi>;
    // opt in to the full 64 KiB of dynamic LDS once per instantiation (a host
    // attribute, done before any graph capture reaches this launch)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)GV_LDS_MAX);
    if (attr != hipSuccess) return attr;
    dim3 grid((c.N + GV_ROWS - 1) / GV_ROWS);
    kern<<<grid, GV_NT, lds, s>>>(c, e);
    return hipGetLastError();
}

template <int FMT, typename T, bool NORM, class Epi>
hipError_t launch_mr(hipStream_t s, const GemvCore& c, const Epi& e, int mr) {
    switch (mr) {
        case 1: return launch_one<FMT, T, 1, NORM, Epi>(s, c, e);
        case 2: return launch_one<FMT, T, 2, NORM, Epi>(s, c, e);
        case 3: return launch_one<FMT, T, 3, NORM, Epi>(s, c, e);
        default: return launch_one<FMT, T, 4, NORM, Epi>(s, c, e);
    }
}

template <typename T, bool NORM, class Epi>
hipError_t launch_fmt(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int wfmt) {
    switch (wfmt) {
        case LSSM_W_Q4_B32: return launch_mr<LSSM_W_Q4_B32, T, NORM, Epi>(s, c, e, mr);
        case LSSM_W_Q4_G64: return launch_mr<LSSM_W_Q4_G64, T, NORM, Epi>(s, c, e, mr);
        case LSSM_W_Q8_G32: return launch_mr<LSSM_W_Q8_G32, T, NORM, Epi>(s, c, e, mr);
        default: return launch_mr<LSSM_W_DENSE, T, NORM, Epi>(s, c, e, mr);
    }
}

// Largest number of x rows per launch whose fp32 LDS staging fits.
inline int max_rows(uint32_t K) {
    int mr = (int)(GV_LDS_MAX / ((size_t)K * sizeof(float)));
    return mr > 4 ? 4 : mr;
}

template <typename T, int EPI>
hipError_t gemv_plain(hipStream_t s, const GemvArgs& a) {
    const size_t es = sizeof(T);
    const int mrmax = max_rows(a.K);
    if (mrmax < 1) return hipErrorInvalidValue;
    for (uint32_t m0 = 0; m0 < a.M; m0 += (uint32_t)mrmax) {
        const int mr = (int)((a.M - m0) < (uint32_t)mrmax ? (a.M - m0) : (uint32_t)mrmax);
        GemvCore c{(const char*)a.x + (size_t)m0 * a.x_stride * es, a.x_stride,
                   (const uint8_t*)a.w, (const uint16_t*)a.s, a.norm_w, a.eps, a.N, a.K};
        EpiPlain<T, EPI> e{(T*)a.y + (size_t)m0 * a.y_stride, a.y_stride,
                           a.res ? (const T*)a.res + (size_t)m0 * a.y_stride : nullptr};
        hipError_t err = a.norm_w ? launch_fmt<T, true>(s, c, e, mr, a.wfmt)
                                  : launch_fmt<T, false>(s, c, e, mr, a.wfmt);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

template <typename T>
hipError_t gemv_epi(hipStream_t s, const GemvArgs& a) {
    switch (a.epi) {
        case LSSM_EPI_SILU: return gemv_plain<T, LSSM_EPI_SILU>(s, a);
        case LSSM_EPI_ADD: return gemv_plain<T, LSSM_EPI_ADD>(s, a);
        default: return gemv_plain<T, LSSM_EPI_NONE>(s, a);
    }
}

// Bit-exact dequantization: out[n, k] = float(q) * float(scale).
template <int FMT>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, const uint16_t* __restrict__ s,
                               float* __restrict__ out, uint32_t N, uint32_t K) {
    using F = Fmt<FMT, f16>;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const uint32_t n = (uint32_t)(i / K), k = (uint32_t)(i % K);
    int q;
    if constexpr (FMT == LSSM_W_Q8_G32) {
        q = (int)(int8_t)w[(size_t)n * K + k];
    } else {
        const uint8_t b = w[(size_t)n * (K / 2) + k / 2];
        const uint32_t nib = (k & 1u) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0fu);
        q = nib < 8u ? (int)nib : (int)nib - 16;
    }
    out[i] = (float)q * fp16_bits_to_f(s[(size_t)n * (K / F::G) + k / F::G]);
}

}  // namespace

hipError_t launch_gemv(hipStream_t s, const GemvArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.act == LSSM_F16) return gemv_epi<f16>(s, a);
    if (a.act == LSSM_BF16) return gemv_epi<bf16>(s, a);
    return gemv_epi<float>(s, a);
}

hipError_t launch_inproj_decode(hipStream_t s, const InprojDecodeArgs& a) {
    const GemvArgs& g = a.g;
    if (g.M == 0) return hipSuccess;
    if ((int)g.M > max_rows(g.K)) return hipErrorInvalidValue;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K};
    auto go = [&](auto tag) -> hipError_t {
        using T = decltype(tag);
        EpiInproj<T> e{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state, (const T*)a.conv_w,
                       (const T*)a.conv_b, (T*)a.z, (T*)a.xbc_act, (T*)a.dt};
        return g.norm_w ? launch_fmt<T, true>(s, c, e, (int)g.M, g.wfmt)
                        : launch_fmt<T, false>(s, c, e, (int)g.M, g.wfmt);
    };
    if (g.act == LSSM_F16) return go(f16{});
    if (g.act == LSSM_BF16) return go(bf16{});
    return go(float{});
}

hipError_t launch_dequant(hipStream_t s, const void* w, const void* sc, float* out, uint32_t N,
                          uint32_t K, int wfmt) {
    const size_t n = (size_t)N * K;
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    switch (wfmt) {
        case LSSM_W_Q4_B32:
            dequant_kernel<LSSM_W_Q4_B32><<<blocks, 256, 0, s>>>((const uint8_t*)w, (const uint16_t*)sc, out, N, K);
            break;
        case LSSM_W_Q4_G64:
            dequant_kernel<LSSM_W_Q4_G64><<<blocks, 256, 0, s>>>((const uint8_t*)w, (const uint16_t*)sc, out, N, K);
            break;
        case LSSM_W_Q8_G32:
            dequant_kernel<LSSM_W_Q8_G32><<<blocks, 256, 0, s>>>((const uint8_t*)w, (const uint16_t*)sc, out, N, K);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lssm

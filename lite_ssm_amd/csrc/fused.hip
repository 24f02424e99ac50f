// fused.hip — the reference's fused in_proj + conv1d + SiLU split for short
// prefills (fused.metal:43-165), kept for drop-in completeness.
//
// One block per 32 projection columns (as the reference); the L x 32 fp32
// projection tile stays in LDS and the depthwise conv reads it UNROUNDED
// (fused.metal:140-149), so this op's rounding differs from the unfused chain.
#include "common.hpp"
#include "internal.hpp"

namespace lssm {

namespace {

constexpr int FT_N = 32, FT_M = 16, FT_NT = 256;

template <typename T>
__global__ __launch_bounds__(FT_NT) void inproj_fused_kernel(const T* __restrict__ normed,
                                                             const T* __restrict__ W,
                                                             const T* __restrict__ Wc,
                                                             const T* __restrict__ cb, T* pz, T* sx,
                                                             T* sB, T* sC, T* pdt, T* pxbc,
                                                             lssm_fused_inproj_dims p) {
    __shared__ float Cmm[FT_M * FT_N];
    const uint32_t col0 = blockIdx.x * FT_N;
    const uint32_t cw = min((uint32_t)FT_N, p.proj_dim - col0);
    const uint32_t L = p.L, K = p.d_model, d_inner = p.d_inner;
    const uint32_t GN = p.n_groups * p.d_state;
    const uint32_t xbc = d_inner + 2u * GN;
    const int lane = threadIdx.x % WAVE, wv = threadIdx.x / WAVE;
    // each wave computes 8 columns; lanes split K and reduce
    for (uint32_t cc = wv; cc < cw; cc += FT_NT / WAVE) {
        const T* wr = W + (size_t)(col0 + cc) * K;
        for (uint32_t m = 0; m < L; ++m) {
            float a = 0.0f;
            for (uint32_t k = lane; k < K; k += WAVE) a += to_f(normed[(size_t)m * K + k]) * to_f(wr[k]);
            a = wave_sum(a);
            if (lane == 0) Cmm[m * FT_N + cc] = a;
        }
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < L * cw; t += FT_NT) {
        const uint32_t m = t / cw, c = t % cw, gc = col0 + c;
        const float v = Cmm[m * FT_N + c];
        if (gc < d_inner) {
            pz[(size_t)m * d_inner + gc] = from_f<T>(v);
        } else if (gc < d_inner + xbc) {
            const uint32_t xc = gc - d_inner;
            pxbc[(size_t)m * xbc + xc] = from_f<T>(v);
            float sum = to_f(cb[xc]);
            for (uint32_t kk = 0; kk < p.d_conv; ++kk) {
                const int sm = (int)m - (int)(p.d_conv - 1 - kk);
                if (sm >= 0) sum += to_f(Wc[(size_t)xc * p.d_conv + kk]) * Cmm[sm * FT_N + c];
            }
            const T sv = from_f<T>(silu_f(sum));
            if (xc < d_inner) sx[(size_t)m * d_inner + xc] = sv;
            else if (xc < d_inner + GN) sB[(size_t)m * GN + (xc - d_inner)] = sv;
            else sC[(size_t)m * GN + (xc - d_inner - GN)] = sv;
        } else {
            pdt[(size_t)m * p.n_heads + (gc - d_inner - xbc)] = from_f<T>(v);
        }
    }
}

}  // namespace

hipError_t launch_inproj_fused(hipStream_t s, const void* normed, const void* W_in,
                               const void* W_conv, const void* conv_b, void* proj_z, void* ssd_x,
                               void* ssd_B, void* ssd_C, void* proj_dt, void* proj_xBC,
                               lssm_fused_inproj_dims d) {
    if (d.L == 0 || d.proj_dim == 0) return hipSuccess;
    dim3 grid((d.proj_dim + FT_N - 1) / FT_N);
    inproj_fused_kernel<f16><<<grid, FT_NT, 0, s>>>(
        (const f16*)normed, (const f16*)W_in, (const f16*)W_conv, (const f16*)conv_b, (f16*)proj_z,
        (f16*)ssd_x, (f16*)ssd_B, (f16*)ssd_C, (f16*)proj_dt, (f16*)proj_xBC, d);
    return hipGetLastError();
}

}  // namespace lssm

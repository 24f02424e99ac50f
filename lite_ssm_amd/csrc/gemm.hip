// gemm.hip — MFMA GEMM for prefill and batched decode (M > 4).
//
// Y[M, N] = epi( X[M, K] . deq(W)[N, K]^T ).  Restates linear.metal:492-574
// (int4 GEMM: the dequantized weight is rounded to the activation dtype before
// the matrix product, :538) and linear.metal:253-343 (dense fp16 GEMM), with
// fp32 accumulation and one rounding at the store.
//
// gfx950 mapping: 256-thread blocks (4 waves in a 2 x 2 grid) own a 128 x 128
// output tile; each wave owns 64 x 64 = 2 x 2 tiles of v_mfma_f32_32x32x16
// (f16 or bf16 operands, fp32 accumulators in registers).  Per 64-wide K step
// the block stages X[128 x 64] and the dequantized W[128 x 64] in LDS (rows
// padded to 72 elements so the 16-byte fragment reads of 8 consecutive rows
// hit distinct banks); the global loads of step k+1 are issued before the
// MFMAs of step k.
#include "common.cuh"
#include "internal.hpp"

namespace lssm {

namespace {

constexpr int BM = 128, BN = 128, BK = 64, PAD = 72, NT = 256;

template <typename T> struct MfmaOp;
template <> struct MfmaOp<f16> {
    using frag = half8;
    static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct MfmaOp<bf16> {
    using frag = bf16x8;
    static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// Per-thread register staging of one K step.
template <int FMT> struct BStage {
    static constexpr int NCH = (FMT == LSSM_W_DENSE) ? 4 : (FMT == LSSM_W_Q8_G32 ? 2 : 1);
    uint4 w[NCH];
    float s[NCH];
};

template <int FMT, typename T>
__device__ __forceinline__ void load_b(BStage<FMT>& st, const GemmArgs& a, uint32_t n0, uint32_t k0) {
    const int t = threadIdx.x;
    const uint32_t K = a.K;
#pragma unroll
    for (int i = 0; i < BStage<FMT>::NCH; ++i) {
        uint32_t row, koff;  // koff = first k of the chunk within the step
        if constexpr (FMT == LSSM_W_DENSE) {
            const int id = t + NT * i;
            row = id / 8;
            koff = (id % 8) * 8;
        } else if constexpr (FMT == LSSM_W_Q8_G32) {
            const int id = t + NT * i;
            row = id / 4;
            koff = (id % 4) * 16;
        } else {
            row = t / 2;
            koff = (t % 2) * 32;
        }
        const uint32_t n = n0 + row;
        if (n < a.N) {
            const uint8_t* w = (const uint8_t*)a.w;
            const uint16_t* s = (const uint16_t*)a.s;
            if constexpr (FMT == LSSM_W_DENSE) {
                st.w[i] = *reinterpret_cast<const uint4*>(w + ((size_t)n * K + k0 + koff) * sizeof(T));
                st.s[i] = 1.0f;
            } else if constexpr (FMT == LSSM_W_Q8_G32) {
                st.w[i] = *reinterpret_cast<const uint4*>(w + (size_t)n * K + k0 + koff);
                st.s[i] = fp16_bits_to_f(s[(size_t)n * (K / 32) + (k0 + koff) / 32]);
            } else if constexpr (FMT == LSSM_W_Q4_G64) {
                st.w[i] = *reinterpret_cast<const uint4*>(w + (size_t)n * (K / 2) + (k0 + koff) / 2);
                st.s[i] = fp16_bits_to_f(s[(size_t)n * (K / 64) + k0 / 64]);
            } else {
                st.w[i] = *reinterpret_cast<const uint4*>(w + (size_t)n * (K / 2) + (k0 + koff) / 2);
                st.s[i] = fp16_bits_to_f(s[(size_t)n * (K / 32) + (k0 + koff) / 32]);
            }
        } else {
            st.w[i] = make_uint4(0, 0, 0, 0);
            st.s[i] = 0.0f;
        }
    }
}

// Dequantize the staged chunk(s) and write them to LDS Bs[row][k] as T.
template <int FMT, typename T>
__device__ __forceinline__ void store_b(const BStage<FMT>& st, T* Bs) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < BStage<FMT>::NCH; ++i) {
        const uint32_t d[4] = {st.w[i].x, st.w[i].y, st.w[i].z, st.w[i].w};
        if constexpr (FMT == LSSM_W_DENSE) {
            const int id = t + NT * i;
            *reinterpret_cast<uint4*>(Bs + (id / 8) * PAD + (id % 8) * 8) = st.w[i];
        } else if constexpr (FMT == LSSM_W_Q8_G32) {
            const int id = t + NT * i;
            T* dst = Bs + (id / 4) * PAD + (id % 4) * 16;
            T v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int q = ((int)(d[e / 4] << (24 - 8 * (e % 4)))) >> 24;
                v[e] = from_f<T>((float)q * st.s[i]);
            }
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(&v[0]);
            *reinterpret_cast<uint4*>(dst + 8) = *reinterpret_cast<const uint4*>(&v[8]);
        } else {
            T* dst = Bs + (t / 2) * PAD + (t % 2) * 32;
            T v[32];
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const int q = ((int)(d[e / 8] << (28 - 4 * (e % 8)))) >> 28;
                v[e] = from_f<T>((float)q * st.s[i]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<uint4*>(dst + 8 * j) = *reinterpret_cast<const uint4*>(&v[8 * j]);
        }
    }
}

template <int FMT, typename T, int EPI>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) T As[BM * PAD];
    __shared__ __attribute__((aligned(16))) T Bs[BN * PAD];
    using Op = MfmaOp<T>;
    using frag = typename Op::frag;

    const int t = threadIdx.x;
    const int lane = t % WAVE;
    const int wv = t / WAVE;
    const int wm = wv / 2, wn = wv % 2;
    const uint32_t m0 = blockIdx.y * BM;
    const uint32_t n0 = blockIdx.x * BN;
    const T* X = (const T*)a.x;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    uint4 areg[4];
    BStage<FMT> breg;
    auto load_a = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = t + NT * i;
            const uint32_t m = m0 + id / 8;
            if (m < a.M)
                areg[i] = *reinterpret_cast<const uint4*>(X + (size_t)m * a.x_stride + k0 + (id % 8) * 8);
            else
                areg[i] = make_uint4(0, 0, 0, 0);
        }
    };

    const uint32_t KT = a.K / BK;
    load_a(0);
    load_b<FMT, T>(breg, a, n0, 0);
    for (uint32_t kt = 0; kt < KT; ++kt) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = t + NT * i;
            *reinterpret_cast<uint4*>(As + (id / 8) * PAD + (id % 8) * 8) = areg[i];
        }
        store_b<FMT, T>(breg, Bs);
        __syncthreads();
        if (kt + 1 < KT) {
            load_a((kt + 1) * BK);
            load_b<FMT, T>(breg, a, n0, (kt + 1) * BK);
        }
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kk = ks * 16 + (lane / 32) * 8;
            frag af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const frag*>(As + (wm * 64 + i * 32 + lane % 32) * PAD + kk);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = *reinterpret_cast<const frag*>(Bs + (wn * 64 + j * 32 + lane % 32) * PAD + kk);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = Op::mma(af[i], bfr[j], acc[i][j]);
        }
    }

    // D layout of v_mfma_f32_32x32x*: element r of lane l is
    // row (r/4)*8 + (l/32)*4 + r%4, column l%32.
    T* Y = (T*)a.y;
    const T* R = (const T*)a.res;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + lane % 32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 64 + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + r % 4;
                if (m < a.M && n < a.N) {
                    const size_t yi = (size_t)m * a.y_stride + n;
                    float v = acc[i][j][r];
                    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
                    if (EPI == LSSM_EPI_ADD) v = to_f(R[yi]) + rnd<T>(v);
                    Y[yi] = from_f<T>(v);
                }
            }
        }
    }
}

// Plain per-output kernel for fp32 activations and unaligned shapes: one
// thread per output; the dequantized weight is rounded to the activation dtype
// when round_dequant != 0 (GEMM semantics) and exact otherwise (GEMV).
template <typename T, int EPI>
__global__ void gemm_simple_kernel(GemmArgs a) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m = blockIdx.y;
    if (n >= a.N) return;
    const T* X = (const T*)a.x + (size_t)m * a.x_stride;
    float acc = 0.0f;
    const uint32_t K = a.K;
    if (a.wfmt == LSSM_W_DENSE) {
        const T* W = (const T*)a.w + (size_t)n * K;
        for (uint32_t k = 0; k < K; ++k) acc += to_f(W[k]) * to_f(X[k]);
    } else {
        const uint8_t* w = (const uint8_t*)a.w;
        const uint16_t* s = (const uint16_t*)a.s;
        const uint32_t G = a.wfmt == LSSM_W_Q4_G64 ? 64 : 32;
        for (uint32_t k = 0; k < K; ++k) {
            int q;
            if (a.wfmt == LSSM_W_Q8_G32) {
                q = (int)(int8_t)w[(size_t)n * K + k];
            } else {
                const uint8_t b = w[(size_t)n * (K / 2) + k / 2];
                const uint32_t nib = (k & 1u) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0xfu);
                q = nib < 8u ? (int)nib : (int)nib - 16;
            }
            float wv = (float)q * fp16_bits_to_f(s[(size_t)n * (K / G) + k / G]);
            if (a.round_dequant) wv = rnd<T>(wv);
            acc += wv * to_f(X[k]);
        }
    }
    const size_t yi = (size_t)m * a.y_stride + n;
    float v = acc;
    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
    if (EPI == LSSM_EPI_ADD) v = to_f(((const T*)a.res)[yi]) + rnd<T>(v);
    ((T*)a.y)[yi] = from_f<T>(v);
}

template <int FMT, typename T>
hipError_t go_epi(hipStream_t s, const GemmArgs& a) {
    dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
    switch (a.epi) {
        case LSSM_EPI_SILU: gemm_kernel<FMT, T, LSSM_EPI_SILU><<<grid, NT, 0, s>>>(a); break;
        case LSSM_EPI_ADD: gemm_kernel<FMT, T, LSSM_EPI_ADD><<<grid, NT, 0, s>>>(a); break;
        default: gemm_kernel<FMT, T, LSSM_EPI_NONE><<<grid, NT, 0, s>>>(a); break;
    }
    return hipGetLastError();
}

template <typename T>
hipError_t go_fmt(hipStream_t s, const GemmArgs& a) {
    switch (a.wfmt) {
        case LSSM_W_Q4_B32: return go_epi<LSSM_W_Q4_B32, T>(s, a);
        case LSSM_W_Q4_G64: return go_epi<LSSM_W_Q4_G64, T>(s, a);
        case LSSM_W_Q8_G32: return go_epi<LSSM_W_Q8_G32, T>(s, a);
        default: return go_epi<LSSM_W_DENSE, T>(s, a);
    }
}

}  // namespace

hipError_t launch_gemm(hipStream_t s, const GemmArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.act == LSSM_F16) return go_fmt<f16>(s, a);
    if (a.act == LSSM_BF16) return go_fmt<bf16>(s, a);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_simple(hipStream_t s, const GemmArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    dim3 grid((a.N + 255) / 256, a.M);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        switch (a.epi) {
            case LSSM_EPI_SILU: gemm_simple_kernel<T, LSSM_EPI_SILU><<<grid, 256, 0, s>>>(a); break;
            case LSSM_EPI_ADD: gemm_simple_kernel<T, LSSM_EPI_ADD><<<grid, 256, 0, s>>>(a); break;
            default: gemm_simple_kernel<T, LSSM_EPI_NONE><<<grid, 256, 0, s>>>(a); break;
        }
    };
    if (a.act == LSSM_F16) go(f16{});
    else if (a.act == LSSM_BF16) go(bf16{});
    else go(float{});
    return hipGetLastError();
}

}  // namespace lssm

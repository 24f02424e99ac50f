// gemv.hip — dequantize-in-register GEMV for decode (M <= 4 rows of x).
//
// Y[m, n] = epi( sum_k deq(W)[n, k] * x[m, k] ), W row-major [N, K] in one of
// the formats of lssm_wfmt.  Restates linear.metal:440-474 (int4 GEMV: exact
// dequantization float(q) * float(scale), fp32 accumulation, one rounding at
// the store) and linear.metal:82-109 (dense fp16 GEMV).
//
// Two kernels, both reading every weight byte from HBM exactly once with
// 16-byte loads (a "chunk": 32 int4 / 16 int8 / 8 dense weights of one row):
//
//  * gemv1 (M == 1, fp16 / bf16): LPR lanes own one row; lane l owns chunks
//    l, l + LPR, ... (CPL of them), so the LPR lanes of a row cover all of K.
//    The first row's weight chunks (and the epilogue's inputs) are issued
//    before anything else; meanwhile the 512-thread block loads x once (one
//    round of 16-byte loads of x and of the norm weight), RMSNorms it when
//    fused, and stages it in LDS as packed pairs in the order the unpacked
//    weights come out, with each chunk's sum(x) in the padding.  Waves then
//    walk rows with the next row's chunks in flight while the current row is
//    reduced.  Int4 / int8 are unpacked with mask-and-or "magic" constants into
//    packed fp16 / bf16 pairs and multiplied with v_dot2 (exact products, fp32
//    sums):
//      fp16: ((q ^ 8) | 0x6400) = 1032 + q, then v_pk_add_f16 -1032 (exact);
//      bf16: ((q ^ 8) | 0x4300) = 136 + q; 136 * sum(x) of the chunk is
//            subtracted once per chunk.
//
//  * gemv_lds (M <= 4, any dtype): x rows staged once per block in LDS as
//    fp32, padded by 4 floats per chunk so that the 16-byte reads of the 16
//    lanes of a row fall in distinct banks; 16 lanes per row.
#include "common.cuh"
#include "internal.hpp"

namespace lssm {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GV_NT = 256;
constexpr int G1_NT = 512;                       // gemv1 block: 8 waves share one x staging
constexpr size_t GV_LDS_MAX = GEMV_LDS_BYTES;
// LDS dwords per staged x chunk in gemv1: <= 16 packed pairs, the chunk's
// sum(x), padding to 20 so that 16 lanes' 16-byte reads hit distinct banks.
constexpr int GV_XS = 20;

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

inline uint32_t wpc_of(int wfmt, int act) {
    switch (wfmt) {
        case LSSM_W_Q4_B32:
        case LSSM_W_Q4_G64: return 32;
        case LSSM_W_Q8_G32: return 16;
        default: return 16 / (uint32_t)dtype_size(act);
    }
}

// ---------------------------------------------------------------------------
// Epilogues (called by one lane per output element)
// ---------------------------------------------------------------------------
// Each epilogue has prefetch(m, n), issued together with the row's weight
// loads, whose result is handed to operator() once the row's sum is ready.
//
// y[m, n] = r(acc) / r(silu(acc)) / r(res + r(acc))
template <typename T> struct EpiPlain {
    T* y;
    uint32_t y_stride;
    const T* res;
    int epi;
    struct Pre {
        float r;
    };
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const {
        Pre p{0.0f};
        if (epi == LSSM_EPI_ADD) p.r = to_f(res[(size_t)m * y_stride + n]);
        return p;
    }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const size_t i = (size_t)m * y_stride + n;
        float v = acc;
        if (epi == LSSM_EPI_SILU) v = silu_f(acc);
        else if (epi == LSSM_EPI_ADD) v = p.r + rnd<T>(acc);
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
    // the 4-tap window, weights and bias of an xBC row (2-byte T, d_conv == 4)
    struct Pre {
        uint2 s, w;
        float b;
    };
    static constexpr bool kVec = sizeof(T) == 2;
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const {
        Pre p{make_uint2(0, 0), make_uint2(0, 0), 0.0f};
        if (kVec && dconv == 4 && n >= d_inner && n < d_inner + xbc) {
            const uint32_t c = n - d_inner;
            p.s = *reinterpret_cast<const uint2*>(conv_state + ((size_t)m * xbc + c) * 4);
            p.w = *reinterpret_cast<const uint2*>(conv_w + (size_t)c * 4);
            p.b = to_f(conv_b[c]);
        }
        return p;
    }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const T v = from_f<T>(acc);
        if (n < d_inner) {
            z[(size_t)m * d_inner + n] = v;
        } else if (n < d_inner + xbc) {
            const uint32_t c = n - d_inner;
            T* sd = conv_state + ((size_t)m * xbc + c) * dconv;
            float a = 0.0f;
            bool done = false;
            if constexpr (kVec) {
                if (dconv == 4) {
                    const T* s = reinterpret_cast<const T*>(&p.s);
                    const T* w = reinterpret_cast<const T*>(&p.w);
                    // window shift (conv1d.metal:127-130): taps 1..3 move down, x lands in 3
                    a = p.b + to_f(s[1]) * to_f(w[0]) + to_f(s[2]) * to_f(w[1]) + to_f(s[3]) * to_f(w[2]) +
                        to_f(v) * to_f(w[3]);
                    uint2 ns;
                    ns.x = p.s.x >> 16 | p.s.y << 16;                                     // (s1, s2)
                    ns.y = p.s.y >> 16 | (uint32_t)__builtin_bit_cast(uint16_t, v) << 16;  // (s3, x)
                    *reinterpret_cast<uint2*>(sd) = ns;
                    done = true;
                }
            }
            if (!done) {
                const T* wd = conv_w + (size_t)c * dconv;
                a = to_f(conv_b[c]);
                for (uint32_t k = 0; k + 1 < dconv; ++k) {
                    const T sk = sd[k + 1];
                    sd[k] = sk;
                    a += to_f(sk) * to_f(wd[k]);
                }
                sd[dconv - 1] = v;
                a += to_f(v) * to_f(wd[dconv - 1]);
            }
            xbc_act[(size_t)m * xbc + c] = from_f<T>(silu_f(rnd<T>(a)));
        } else {
            dt[(size_t)m * H + (n - d_inner - xbc)] = v;
        }
    }
};

// ---------------------------------------------------------------------------
// gemv1: M == 1, x in registers
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ uint32_t bits16(T v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, v);
}
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return bits16(from_f<T>(a)) | (bits16(from_f<T>(b)) << 16);
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c, f16) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c, false);
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c, bf16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a), __builtin_bit_cast(bf16x2v, b), c,
                                           false);
}
__device__ __forceinline__ uint32_t pk_add_f16(uint32_t a, float c) {
    const half2v r = __builtin_bit_cast(half2v, a) + half2v{(f16)c, (f16)c};
    return __builtin_bit_cast(uint32_t, r);
}

// Position (within the chunk) of the two x values paired with packed pair p.
// Q4: dword i, pair j (shift 4j) holds weights 8i+j and 8i+j+4.
// Q8: dword i holds weights 4i..4i+3; pair 0 = (4i, 4i+2), pair 1 = (4i+1, 4i+3).
// Dense: natural pairs (2p, 2p+1).
template <int FMT> __device__ __forceinline__ void pair_pos(int p, int& a, int& b) {
    if constexpr (FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64) {
        a = 8 * (p / 4) + (p % 4);
        b = a + 4;
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
        a = 4 * (p / 2) + (p % 2);
        b = a + 2;
    } else {
        a = 2 * p;
        b = a + 1;
    }
}

// sum_pairs dot of one weight chunk with the packed x pairs xp[0..WPC/2).
template <int FMT, typename T>
__device__ __forceinline__ float chunk_dot2(const uint4 wv, const uint32_t* xp) {
    const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
    float acc = 0.0f;
    if constexpr (FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = d[i] ^ 0x88888888u;            // nibble -> q + 8
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t m = (u >> (4 * j)) & 0x000F000Fu;
                if constexpr (sizeof(T) == 2 && __is_same(T, f16)) {
                    const uint32_t h = pk_add_f16(m | 0x64006400u, -1032.0f);   // exact q
                    acc = dot2(h, xp[4 * i + j], acc, f16{});
                } else {
                    acc = dot2(m | 0x43004300u, xp[4 * i + j], acc, bf16{});    // q + 136
                }
            }
        }
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = d[i] ^ 0x80808080u;            // byte -> q + 128
            const uint32_t h0 = pk_add_f16((u & 0x00FF00FFu) | 0x64006400u, -1152.0f);
            const uint32_t h1 = pk_add_f16(((u >> 8) & 0x00FF00FFu) | 0x64006400u, -1152.0f);
            acc = dot2(h0, xp[2 * i], acc, f16{});
            acc = dot2(h1, xp[2 * i + 1], acc, f16{});
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = dot2(d[i], xp[i], acc, T{});
    }
    return acc;
}

template <int FMT, typename T, int LPR, int CPL, bool NORM, class Epi>
__global__ __launch_bounds__(G1_NT) void gemv1_kernel(GemvCore c, Epi epi) {
    using F = Fmt<FMT, T>;
    constexpr int WPC = F::WPC;
    constexpr int NP = WPC / 2;                      // packed pairs per chunk
    constexpr int RPW = WAVE / LPR;                  // rows per wave per step
    constexpr bool BIAS136 = (FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64) && !__is_same(T, f16);
    extern __shared__ uint32_t xl[];                 // [cpr][XS]: NP packed pairs, sum(x), pad
    __shared__ float red[G1_NT / WAVE];
    const int lane = threadIdx.x % WAVE;
    const int lr = lane % LPR;
    const uint32_t K = c.K;
    const uint32_t nwaves = gridDim.x * (G1_NT / WAVE);
    const uint32_t ngroups = (c.N + RPW - 1) / RPW;
    const size_t rb = F::row_bytes(K);
    constexpr uint32_t GD = F::G ? F::G : 1;
    const uint32_t gpr = K / GD;

    auto load = [&](uint32_t n, uint4* wq, float* sc) {
        if (n < c.N) {
            const uint8_t* wr = c.w + (size_t)n * rb;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t ch = lr + LPR * j;
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (size_t)ch * 16));
                wq[j] = make_uint4(v[0], v[1], v[2], v[3]);
                if constexpr (F::G > 0) sc[j] = fp16_bits_to_f(c.s[(size_t)n * gpr + (ch * WPC) / GD]);
                else sc[j] = 1.0f;
            }
        }
    };

    // ---- 1. the first row's weight chunks (and epilogue inputs) go out first ----
    uint32_t rg = blockIdx.x * (G1_NT / WAVE) + threadIdx.x / WAVE;
    uint32_t n = rg * RPW + lane / LPR;
    uint4 wq[CPL];
    float sc[CPL];
    typename Epi::Pre pre{};
    if (rg < ngroups) {
        load(n, wq, sc);
        if (lr == 0 && n < c.N) pre = epi.prefetch(0, n);
    }

    // ---- 2. stage x (RMSNorm'ed when fused, norm.metal:52-79) as packed pairs ----
    // Thread t owns octets (8 consecutive x) t, t + NT, ...: one round of 16-byte
    // loads of x and of the norm weight, a block reduction, then packing.
    constexpr int OCT = 4;                           // octets per thread: K <= 8 * NT * OCT
    const uint4* x4 = reinterpret_cast<const uint4*>(c.x);
    const uint4* nw4 = reinterpret_cast<const uint4*>(c.norm_w);
    const uint32_t noct = K / 8;
    uint4 xo[OCT], wo[OCT];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < OCT; ++i) {
        const uint32_t o = threadIdx.x + G1_NT * i;
        if (o < noct) {
            xo[i] = x4[o];
            if constexpr (NORM) wo[i] = nw4[o];
            const T* t = reinterpret_cast<const T*>(&xo[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = to_f(t[e]);
                ss += v * v;
            }
        }
    }
    float rrms = 1.0f;
    if constexpr (NORM) {
        ss = block_sum<G1_NT>(ss, red);
        rrms = 1.0f / sqrtf(ss / (float)K + c.eps);
    }
#pragma unroll
    for (int i = 0; i < OCT; ++i) {
        const uint32_t o = threadIdx.x + G1_NT * i;       // uniform in i across a wave's lanes
        if (G1_NT * i >= noct) break;
        float v[8];
        float s = 0.0f;
        if (o < noct) {
            const T* t = reinterpret_cast<const T*>(&xo[i]);
            const T* tw = reinterpret_cast<const T*>(&wo[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = to_f(t[e]);
                if constexpr (NORM) v[e] = rnd<T>(v[e] * to_f(tw[e]) * rrms);
                s += v[e];
            }
            const uint32_t k0 = o * 8, ch = k0 / WPC, off = k0 % WPC;
            uint32_t* dst = xl + (size_t)ch * GV_XS;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int a, b;
                pair_pos<FMT>((int)(off / 2) + q, a, b);
                dst[off / 2 + q] = pack2<T>(v[a - (int)off], v[b - (int)off]);
            }
        }
        // sum(x) of a chunk: its WPC/8 octets sit in consecutive lanes
        s = group_sum<WPC / 8>(s);
        if (o < noct && (o % (WPC / 8)) == 0) xl[(size_t)(o * 8 / WPC) * GV_XS + NP] = __float_as_uint(s);
    }
    __syncthreads();
    if (rg >= ngroups) return;

    // ---- 3. rows: next row's chunks in flight while this one is reduced ----
    for (;;) {
        const uint32_t rg_next = rg + nwaves;
        const bool more = rg_next < ngroups;
        const uint32_t n_next = rg_next * RPW + lane / LPR;
        uint4 wq2[CPL];
        float sc2[CPL];
        typename Epi::Pre pre2{};
        if (more) {
            load(n_next, wq2, sc2);
            if (lr == 0 && n_next < c.N) pre2 = epi.prefetch(0, n_next);
        }
        float acc = 0.0f;
        if (n < c.N) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t* src = xl + (size_t)(lr + LPR * j) * GV_XS;
                uint32_t xp[NP];
#pragma unroll
                for (int q = 0; q < NP / 4; ++q) {
                    const uint4 v = *reinterpret_cast<const uint4*>(src + 4 * q);
                    xp[4 * q] = v.x;
                    xp[4 * q + 1] = v.y;
                    xp[4 * q + 2] = v.z;
                    xp[4 * q + 3] = v.w;
                }
                float d = chunk_dot2<FMT, T>(wq[j], xp);
                if constexpr (BIAS136) d -= 136.0f * __uint_as_float(src[NP]);
                acc += d * sc[j];
            }
        }
        acc = group_sum<LPR>(acc);
        if (lr == 0 && n < c.N) epi(0, n, acc, pre);
        if (!more) break;
        rg = rg_next;
        n = n_next;
        pre = pre2;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            wq[j] = wq2[j];
            sc[j] = sc2[j];
        }
    }
}


template <int FMT, typename T, int LPR, int CPL, class Epi>
hipError_t go1(hipStream_t s, const GemvCore& c, const Epi& e, int norm) {
    constexpr int RPW = WAVE / LPR;
    const uint32_t ngroups = (c.N + RPW - 1) / RPW;
    uint32_t waves = ngroups < 3072u ? ngroups : 3072u;     // ~3 resident waves per SIMD
    const uint32_t blocks = (waves + (G1_NT / WAVE) - 1) / (G1_NT / WAVE);
    const size_t lds = (size_t)(c.K / Fmt<FMT, T>::WPC) * GV_XS * sizeof(uint32_t);
    if (norm) gemv1_kernel<FMT, T, LPR, CPL, true, Epi><<<blocks, G1_NT, lds, s>>>(c, e);
    else gemv1_kernel<FMT, T, LPR, CPL, false, Epi><<<blocks, G1_NT, lds, s>>>(c, e);
    return hipGetLastError();
}

// (lanes per row, chunks per lane) for the chunk counts of the model shapes.
template <int FMT, typename T, class Epi>
hipError_t launch_gemv1(hipStream_t s, const GemvCore& c, const Epi& e, int norm, bool& done) {
    done = true;
    const uint32_t cpr = c.K / Fmt<FMT, T>::WPC;
    switch (cpr) {
        case 48: return go1<FMT, T, 16, 3, Epi>(s, c, e, norm);
        case 64: return go1<FMT, T, 16, 4, Epi>(s, c, e, norm);
        case 80: return go1<FMT, T, 16, 5, Epi>(s, c, e, norm);
        case 96: return go1<FMT, T, 32, 3, Epi>(s, c, e, norm);
        case 128: return go1<FMT, T, 32, 4, Epi>(s, c, e, norm);
        case 160: return go1<FMT, T, 32, 5, Epi>(s, c, e, norm);
        case 192: return go1<FMT, T, 64, 3, Epi>(s, c, e, norm);
        case 256: return go1<FMT, T, 64, 4, Epi>(s, c, e, norm);
        case 320: return go1<FMT, T, 64, 5, Epi>(s, c, e, norm);
        case 512: return go1<FMT, T, 64, 8, Epi>(s, c, e, norm);
        default: done = false; return hipSuccess;
    }
}

// ---------------------------------------------------------------------------
// gemv_lds: M <= 4, x staged in padded LDS
// ---------------------------------------------------------------------------
template <int FMT, typename T>
__device__ __forceinline__ float chunk_dot_f32(const uint4 wv, const float* __restrict__ xr) {
    const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
    float acc = 0.0f;
    if constexpr (FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64) {
        // nibble j of dword i is weight 8*i + j (low nibble = even k, linear.metal:47-61)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc += (float)(((int)(d[i] << (28 - 4 * j))) >> 28) * xr[8 * i + j];
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc += (float)(((int)(d[i] << (24 - 8 * j))) >> 24) * xr[4 * i + j];
    } else {
        const T* wt = reinterpret_cast<const T*>(d);
#pragma unroll
        for (int i = 0; i < 16 / (int)sizeof(T); ++i) acc += to_f(wt[i]) * xr[i];
    }
    return acc;
}

constexpr int LDS_LPR = 16;
constexpr int LDS_ROWS = GV_NT / LDS_LPR;
constexpr int LDS_U = 4;

// padded LDS length of one x row: WPC + 4 floats per chunk
__host__ __device__ inline uint32_t padded_len(uint32_t K, uint32_t wpc) { return K / wpc * (wpc + 4); }

template <int FMT, typename T, int MR, class Epi>
__global__ __launch_bounds__(GV_NT) void gemv_lds_kernel(GemvCore c, Epi epi, int norm) {
    extern __shared__ float xs[];                 // [MR][K/WPC][WPC + 4] fp32
    __shared__ float red[GV_NT / WAVE];
    using F = Fmt<FMT, T>;
    constexpr int WPC = F::WPC, CS = WPC + 4;
    const uint32_t K = c.K;
    const uint32_t KP = padded_len(K, WPC);
    const T* x = reinterpret_cast<const T*>(c.x);

#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const T* xr = x + (size_t)m * c.x_stride;
        float rrms = 1.0f;
        if (norm) {
            float ss = 0.0f;
            for (uint32_t k = threadIdx.x; k < K; k += GV_NT) {
                const float v = to_f(xr[k]);
                ss += v * v;
            }
            ss = block_sum<GV_NT>(ss, red);
            rrms = 1.0f / sqrtf(ss / (float)K + c.eps);
        }
        const T* nw = reinterpret_cast<const T*>(c.norm_w);
        for (uint32_t k = threadIdx.x; k < K; k += GV_NT) {
            float v = to_f(xr[k]);
            if (norm) v = rnd<T>(v * to_f(nw[k]) * rrms);
            xs[m * KP + (k / WPC) * CS + k % WPC] = v;
        }
    }
    __syncthreads();

    const int lane = threadIdx.x % WAVE;
    const int wv = threadIdx.x / WAVE;
    const int lr = lane % LDS_LPR;
    const uint32_t n = blockIdx.x * LDS_ROWS + wv * (WAVE / LDS_LPR) + lane / LDS_LPR;
    const bool live = n < c.N;
    const uint32_t cpr = K / WPC;
    const uint8_t* wrow = c.w + (size_t)(live ? n : 0) * F::row_bytes(K);
    constexpr uint32_t GD = F::G ? F::G : 1;
    const uint32_t gpr = K / GD;

    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    if (live) {
        for (uint32_t c0 = lr; c0 < cpr; c0 += LDS_LPR * LDS_U) {
            uint4 wq[LDS_U];
            float sc[LDS_U];
#pragma unroll
            for (int u = 0; u < LDS_U; ++u) {
                const uint32_t ch = c0 + u * LDS_LPR;
                if (ch < cpr) {
                    wq[u] = *reinterpret_cast<const uint4*>(wrow + (size_t)ch * 16);
                    sc[u] = F::G > 0 ? fp16_bits_to_f(c.s[(size_t)n * gpr + (ch * WPC) / GD]) : 1.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < LDS_U; ++u) {
                const uint32_t ch = c0 + u * LDS_LPR;
                if (ch < cpr) {
#pragma unroll
                    for (int m = 0; m < MR; ++m)
                        acc[m] += chunk_dot_f32<FMT, T>(wq[u], xs + m * KP + ch * CS) * sc[u];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = group_sum<LDS_LPR>(acc[m]);
    if (live && lr == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) epi(m, n, acc[m], epi.prefetch(m, n));
    }
}

template <int FMT, typename T, int MR, class Epi>
hipError_t launch_lds_one(hipStream_t s, const GemvCore& c, const Epi& e, int norm) {
    const size_t lds = (size_t)MR * padded_len(c.K, Fmt<FMT, T>::WPC) * sizeof(float);
    auto kern = gemv_lds_kernel<FMT, T, MR, Epi>;
    // opt in to the full dynamic LDS once per instantiation (a host attribute)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)GV_LDS_MAX);
    if (attr != hipSuccess) return attr;
    dim3 grid((c.N + LDS_ROWS - 1) / LDS_ROWS);
    kern<<<grid, GV_NT, lds, s>>>(c, e, norm);
    return hipGetLastError();
}

template <int FMT, typename T, class Epi>
hipError_t launch_lds_mr(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int norm) {
    switch (mr) {
        case 1: return launch_lds_one<FMT, T, 1, Epi>(s, c, e, norm);
        case 2: return launch_lds_one<FMT, T, 2, Epi>(s, c, e, norm);
        case 3: return launch_lds_one<FMT, T, 3, Epi>(s, c, e, norm);
        default: return launch_lds_one<FMT, T, 4, Epi>(s, c, e, norm);
    }
}

// Format dispatch: M == 1 on fp16/bf16 tries gemv1 first.
template <typename T, class Epi>
hipError_t launch_fmt(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int wfmt, int norm) {
    const bool aligned = ((uintptr_t)c.x % 16 == 0) && (!norm || (uintptr_t)c.norm_w % 16 == 0) &&
                         ((uintptr_t)c.w % 16 == 0);
    if constexpr (!__is_same(T, float)) {
      if (mr == 1 && aligned) {
        bool done = false;
        hipError_t err = hipSuccess;
        switch (wfmt) {
            case LSSM_W_Q4_B32: err = launch_gemv1<LSSM_W_Q4_B32, T, Epi>(s, c, e, norm, done); break;
            case LSSM_W_Q4_G64: err = launch_gemv1<LSSM_W_Q4_G64, T, Epi>(s, c, e, norm, done); break;
            case LSSM_W_Q8_G32:
                if constexpr (__is_same(T, f16)) err = launch_gemv1<LSSM_W_Q8_G32, T, Epi>(s, c, e, norm, done);
                break;
            default: err = launch_gemv1<LSSM_W_DENSE, T, Epi>(s, c, e, norm, done); break;
        }
        if (done) return err;
      }
    }
    switch (wfmt) {
        case LSSM_W_Q4_B32: return launch_lds_mr<LSSM_W_Q4_B32, T, Epi>(s, c, e, mr, norm);
        case LSSM_W_Q4_G64: return launch_lds_mr<LSSM_W_Q4_G64, T, Epi>(s, c, e, mr, norm);
        case LSSM_W_Q8_G32: return launch_lds_mr<LSSM_W_Q8_G32, T, Epi>(s, c, e, mr, norm);
        default: return launch_lds_mr<LSSM_W_DENSE, T, Epi>(s, c, e, mr, norm);
    }
}

// Largest number of x rows per launch whose padded fp32 LDS staging fits.
inline int max_rows(uint32_t K, int wfmt, int act) {
    const uint32_t wpc = wpc_of(wfmt, act);
    int mr = (int)(GV_LDS_MAX / ((size_t)padded_len(K, wpc) * sizeof(float)));
    return mr > 4 ? 4 : mr;
}

template <typename T>
hipError_t gemv_plain(hipStream_t s, const GemvArgs& a) {
    const size_t es = sizeof(T);
    const int mrmax = max_rows(a.K, a.wfmt, a.act);
    if (mrmax < 1) return hipErrorInvalidValue;
    for (uint32_t m0 = 0; m0 < a.M; m0 += (uint32_t)mrmax) {
        const int mr = (int)((a.M - m0) < (uint32_t)mrmax ? (a.M - m0) : (uint32_t)mrmax);
        GemvCore c{(const char*)a.x + (size_t)m0 * a.x_stride * es, a.x_stride,
                   (const uint8_t*)a.w, (const uint16_t*)a.s, a.norm_w, a.eps, a.N, a.K};
        EpiPlain<T> e{(T*)a.y + (size_t)m0 * a.y_stride, a.y_stride,
                      a.res ? (const T*)a.res + (size_t)m0 * a.y_stride : nullptr, a.epi};
        hipError_t err = launch_fmt<T>(s, c, e, mr, a.wfmt, a.norm_w ? 1 : 0);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
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

int gemv_max_rows(uint32_t K, int wfmt, int act) { return max_rows(K, wfmt, act); }

hipError_t launch_gemv(hipStream_t s, const GemvArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.act == LSSM_F16) return gemv_plain<f16>(s, a);
    if (a.act == LSSM_BF16) return gemv_plain<bf16>(s, a);
    return gemv_plain<float>(s, a);
}

hipError_t launch_inproj_decode(hipStream_t s, const InprojDecodeArgs& a) {
    const GemvArgs& g = a.g;
    if (g.M == 0) return hipSuccess;
    if ((int)g.M > max_rows(g.K, g.wfmt, g.act)) return hipErrorInvalidValue;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K};
    auto go = [&](auto tag) -> hipError_t {
        using T = decltype(tag);
        EpiInproj<T> e{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state, (const T*)a.conv_w,
                       (const T*)a.conv_b, (T*)a.z, (T*)a.xbc_act, (T*)a.dt};
        return launch_fmt<T>(s, c, e, (int)g.M, g.wfmt, g.norm_w ? 1 : 0);
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

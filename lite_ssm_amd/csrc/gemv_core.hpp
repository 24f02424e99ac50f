// gemv_core.hpp — pieces shared by the decode GEMV kernels (gemv.hip: one
// to four x rows on VALU; gemv_mma.hip: decode batches on MFMA): the weight
// formats, the int4 / int8 unpack into packed fp16 / bf16 pairs and the order
// of those pairs, and the per-row epilogues.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace lssm {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GV_NT = 256;
constexpr int G1_NT = 256;                       // smallest gemv1 block (4 waves)
constexpr size_t GV_LDS_MAX = GEMV_LDS_BYTES;

struct GemvCore {
    const void* x;
    uint32_t x_stride;
    const uint8_t* w;
    const uint16_t* s;
    const void* norm_w;
    float eps;
    uint32_t N, K;
    float inv_k;                                     // 1 / K (the RMSNorm mean)
    // the MFMA decode GEMV only: x already normalised and packed in its
    // staging order ([M][K / 2] dwords, launch_mma_pack), or null
    const uint32_t* xp = nullptr;
    // gemv_mmx only, with xp: when part is set, xp holds the rows raw (not
    // normalised) in fragment order, their sums of squares are the `nparts`
    // partial sums of each row in part ([rows][nparts], added in order) and
    // the norm weight is norm_w
    const float* part = nullptr;
    uint32_t nparts = 0;
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
// prefetch() loads unconditionally (clamped / substitute addresses) and keeps
// raw bits: a conversion or a branch around a load would make the compiler
// wait for it, and with it for every weight load issued before it.
template <typename T> __device__ __forceinline__ uint32_t raw_at(const T* p) {
    if constexpr (sizeof(T) == 2) return *reinterpret_cast<const uint16_t*>(p);
    else return *reinterpret_cast<const uint32_t*>(p);
}
template <typename T> __device__ __forceinline__ float f_of_raw(uint32_t r) {
    if constexpr (sizeof(T) == 2) return to_f(__builtin_bit_cast(T, (uint16_t)r));
    else return __uint_as_float(r);
}

// Read a kernel argument into a register now (an empty asm that uses it):
// pinned at kernel entry, no argument load is left for after the weight loads,
// where it would queue behind the weight traffic.
template <typename V> __device__ __forceinline__ void pin_arg(const V& v) {
    if constexpr (sizeof(V) == 8) asm volatile("" ::"s"(v));
    else asm volatile("" ::"s"(v));
}

// y[m, n] = r(acc) / r(silu(acc)) / r(res + r(acc))
template <typename T> struct EpiPlain {
    static constexpr bool kNormOptional = true;
    static constexpr bool kTail = false;             // no block-level work after the rows
    T* y;
    uint32_t y_stride;
    const T* res;
    int epi;
    struct Pre {
        uint32_t r;
    };
    __device__ __forceinline__ void pin() const {
        pin_arg(y);
        pin_arg(y_stride);
        pin_arg(res);
        pin_arg(epi);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const {
        const T* src = (epi == LSSM_EPI_ADD) ? res : y;   // y: a valid address, value unused
        return Pre{raw_at(src + ((uint32_t)m * y_stride + n))};
    }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const size_t i = (size_t)m * y_stride + n;
        float v = acc;
        if (epi == LSSM_EPI_SILU) v = silu_f(acc);
        else if (epi == LSSM_EPI_ADD) v = f_of_raw<T>(p.r) + rnd<T>(acc);
        y[i] = from_f<T>(v);
    }
    // four rows m[0..3] of one column n (the MFMA decode kernel's lane share)
    struct Pre4 {
        uint32_t r[4];
    };
    __device__ __forceinline__ Pre4 prefetch4(const uint32_t (&m)[4], uint32_t n) const {
        Pre4 p;
#pragma unroll
        for (int r = 0; r < 4; ++r) p.r[r] = prefetch((int)m[r], n).r;
        return p;
    }
    __device__ __forceinline__ void store4(const uint32_t (&m)[4], uint32_t n, const float (&acc)[4], const Pre4& p,
                                           uint32_t live) const {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (live & (1u << r)) (*this)((int)m[r], n, acc[r], Pre{p.r[r]});
    }
};

// Engine decode in_proj epilogue: rows [0, d_inner) -> z, rows of xBC ->
// depthwise conv update (conv1d.metal:108-137) + SiLU (activations.metal:49-73)
// -> xbc_act, remaining rows -> dt.  The pre-conv xBC value is r(acc), the conv
// output is rounded once more before SiLU, as in the unfused op sequence.
template <typename T> struct EpiInproj {
    static constexpr bool kNormOptional = false;           // always behind the layer RMSNorm
    static constexpr bool kTail = false;
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
        uint32_t b;
    };
    static constexpr bool kVec = sizeof(T) == 2;
    __device__ __forceinline__ void pin() const {
        pin_arg(d_inner);
        pin_arg(xbc);
        pin_arg(H);
        pin_arg(dconv);
        pin_arg(conv_state);
        pin_arg(conv_w);
        pin_arg(conv_b);
        pin_arg(z);
        pin_arg(xbc_act);
        pin_arg(dt);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const {
        Pre p{make_uint2(0, 0), make_uint2(0, 0), 0u};
        if constexpr (kVec) {
            // clamped channel; element 0 when the window is not 4 wide (value unused)
            uint32_t c = n < d_inner ? 0u : n - d_inner;
            c = c < xbc ? c : xbc - 1;
            c = dconv == 4 ? c : 0u;
            // 32-bit offsets: 64-bit multiply-adds here get register pairs whose
            // high half is a pending load, which forces a wait for every load
            const uint32_t so = ((uint32_t)m * xbc + c) * dconv, wo = c * dconv;
            p.s = *reinterpret_cast<const uint2*>(conv_state + so);
            p.w = *reinterpret_cast<const uint2*>(conv_w + wo);
            p.b = raw_at(conv_b + c);
        }
        return p;
    }
    // The value row n takes: r(acc) for z and dt rows; for an xBC row the
    // conv window is shifted (and written back) and silu(r(conv)) returned.
    __device__ __forceinline__ T value(int m, uint32_t n, float acc, const Pre& p) const {
        const T v = from_f<T>(acc);
        if (n < d_inner || n >= d_inner + xbc) return v;
        const uint32_t c = n - d_inner;
        T* sd = conv_state + ((size_t)m * xbc + c) * dconv;
        float a = 0.0f;
        bool done = false;
        if constexpr (kVec) {
            if (dconv == 4) {
                // taps and weights by bit extraction (an address of the
                // registers would put them in scratch)
                auto lo = [](uint32_t d) { return f_of_raw<T>(d & 0xFFFFu); };
                auto hi = [](uint32_t d) { return f_of_raw<T>(d >> 16); };
                // window shift (conv1d.metal:127-130): taps 1..3 move down, x lands in 3;
                // the multiply-adds spelled out so that every kernel using this
                // epilogue rounds alike
                a = fmaf(to_f(v), hi(p.w.y),
                         fmaf(hi(p.s.y), lo(p.w.y), fmaf(lo(p.s.y), hi(p.w.x), fmaf(hi(p.s.x), lo(p.w.x), f_of_raw<T>(p.b)))));
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
        return from_f<T>(silu_fast(rnd<T>(a)));
    }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const T v = value(m, n, acc, p);
        if (n < d_inner) z[(size_t)m * d_inner + n] = v;
        else if (n < d_inner + xbc) xbc_act[(size_t)m * xbc + (n - d_inner)] = v;
        else dt[(size_t)m * H + (n - d_inner - xbc)] = v;
    }
    // four rows m[0..3] of one channel n: the conv weights and bias once
    struct Pre4 {
        uint2 s[4], w;
        uint32_t b;
    };
    __device__ __forceinline__ Pre4 prefetch4(const uint32_t (&m)[4], uint32_t n) const {
        Pre4 p;
        const Pre p0 = prefetch((int)m[0], n);
        p.s[0] = p0.s;
        p.w = p0.w;
        p.b = p0.b;
        if constexpr (kVec) {
            uint32_t c = n < d_inner ? 0u : n - d_inner;
            c = c < xbc ? c : xbc - 1;
            c = dconv == 4 ? c : 0u;
#pragma unroll
            for (int r = 1; r < 4; ++r) p.s[r] = *reinterpret_cast<const uint2*>(conv_state + (m[r] * xbc + c) * dconv);
        }
        return p;
    }
    __device__ __forceinline__ void store4(const uint32_t (&m)[4], uint32_t n, const float (&acc)[4], const Pre4& p,
                                           uint32_t live) const {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (live & (1u << r)) (*this)((int)m[r], n, acc[r], Pre{p.s[r], p.w, p.b});
    }
};

// ---------------------------------------------------------------------------
// gemv1: M <= 4 rows of x staged once per block as packed pairs
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ uint32_t bits16(T v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, v);
}
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return bits16(from_f<T>(a)) | (bits16(from_f<T>(b)) << 16);
}
// bf16: one v_cvt_pk_bf16_f32 for the pair (round to nearest even, as the
// conversion of each value alone)
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2p __attribute__((ext_vector_type(2)));
template <> __device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{a, b}, bf16x2p));
}
// fp32 value of the low / high 16-bit half of a packed pair
template <typename T> __device__ __forceinline__ float lo_f(uint32_t u) { return f_of_bits<T>((uint16_t)(u & 0xFFFFu)); }
template <typename T> __device__ __forceinline__ float hi_f(uint32_t u) { return f_of_bits<T>((uint16_t)(u >> 16)); }
template <> __device__ __forceinline__ float lo_f<bf16>(uint32_t u) { return __uint_as_float(u << 16); }
template <> __device__ __forceinline__ float hi_f<bf16>(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
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

template <int FMT> constexpr bool is_q4() { return FMT == LSSM_W_Q4_B32 || FMT == LSSM_W_Q4_G64; }
// int4 x bf16: byte-select unpack, q + 136 per weight, 136 * sum(x) subtracted per chunk
template <int FMT, typename T> constexpr bool q4_bf16() { return is_q4<FMT>() && __is_same(T, bf16); }

// LDS dwords per staged x chunk: the packed pairs, the chunk's sum(x) when the
// unpack is biased, padding so that the 16-byte reads of consecutive lanes
// (consecutive chunks) fall in distinct banks.
template <int NP> constexpr int xs_of() { return NP == 4 ? 4 : NP == 8 ? 12 : 20; }

// Position (within the chunk) of the two x values paired with packed pair p.
//  int4 x bf16: dword i gives lo = nibbles (0, 2, 4, 6), hi = (1, 3, 5, 7) of
//    its 8 weights 8i..8i+7 as bytes; pairs (lo.b0, lo.b1), (lo.b2, lo.b3),
//    (hi.b0, hi.b1), (hi.b2, hi.b3) = weights (0,2), (4,6), (1,3), (5,7).
//  int4 x f16: dword i, pair j (shift 4j) holds weights 8i+j and 8i+j+4.
//  int8: dword i holds weights 4i..4i+3; pair 0 = (4i, 4i+2), pair 1 = (4i+1, 4i+3).
//  dense: natural pairs (2p, 2p+1).
template <int FMT, typename T> __device__ __forceinline__ void pair_pos(int p, int& a, int& b) {
    if constexpr (q4_bf16<FMT, T>()) {
        const int i = p / 4, j = p % 4;
        a = 8 * i + ((j & 2) ? 1 : 0) + ((j & 1) ? 4 : 0);
        b = a + 2;
    } else if constexpr (is_q4<FMT>()) {
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

// One 16-byte weight chunk unpacked into packed fp16 / bf16 pairs.
template <int FMT, typename T> struct Unpacked {
    static constexpr int NP = Fmt<FMT, T>::WPC / 2;
    uint32_t p[NP];
};
template <int FMT, typename T>
__device__ __forceinline__ Unpacked<FMT, T> unpack(const uint4 wv) {
    const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
    Unpacked<FMT, T> u;
    if constexpr (q4_bf16<FMT, T>()) {
        // q + 8 per nibble, as bytes; v_perm puts each byte under a 0x43 byte:
        // bf16 0x43XX = 128 + XX
        constexpr uint32_t MAGIC = 0x43434343u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (d[i] ^ 0x08080808u) & 0x0F0F0F0Fu;
            const uint32_t hi = ((d[i] >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu;
            u.p[4 * i + 0] = __builtin_amdgcn_perm(MAGIC, lo, 0x04010400u);
            u.p[4 * i + 1] = __builtin_amdgcn_perm(MAGIC, lo, 0x04030402u);
            u.p[4 * i + 2] = __builtin_amdgcn_perm(MAGIC, hi, 0x04010400u);
            u.p[4 * i + 3] = __builtin_amdgcn_perm(MAGIC, hi, 0x04030402u);
        }
    } else if constexpr (is_q4<FMT>()) {
        // fp16 0x64XX = 1024 + XX; - 1032 is exact
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = d[i] ^ 0x88888888u;
#pragma unroll
            for (int j = 0; j < 4; ++j) u.p[4 * i + j] = pk_add_f16(((v >> (4 * j)) & 0x000F000Fu) | 0x64006400u, -1032.0f);
        }
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = d[i] ^ 0x80808080u;            // byte -> q + 128
            u.p[2 * i] = pk_add_f16((v & 0x00FF00FFu) | 0x64006400u, -1152.0f);
            u.p[2 * i + 1] = pk_add_f16(((v >> 8) & 0x00FF00FFu) | 0x64006400u, -1152.0f);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) u.p[i] = d[i];
    }
    return u;
}

}  // namespace

}  // namespace lssm

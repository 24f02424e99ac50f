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
#include "common.hpp"
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

    // Each column tile starts its K walk at its own step: W rows of a
    // power-of-two pitch (8 KB for K = 4096 bf16) otherwise put every block's
    // row segments on the same few memory channels at once.  (The order
    // depends on the column only, not on the row tile.)
    const uint32_t KT = a.K / BK;
    const uint32_t rot = KT ? blockIdx.x % KT : 0u;
    auto kof = [&](uint32_t kt) { const uint32_t q = kt + rot; return (q >= KT ? q - KT : q) * BK; };
    load_a(kof(0));
    load_b<FMT, T>(breg, a, n0, kof(0));
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
            load_a(kof(kt + 1));
            load_b<FMT, T>(breg, a, n0, kof(kt + 1));
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
                    if (a.row_scale) v *= a.row_scale[m];
                    if (n < a.silu_cols) v = silu_fast(v);
                    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
                    if (EPI == LSSM_EPI_ADD) v = to_f(R[yi]) + rnd<T>(v);
                    Y[yi] = from_f<T>(v);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-tile GEMM.  512 threads own a 256 x 128 tile of Y.  Waves 0..3
// compute: each owns 128 x 64 = 4 x 2 v_mfma_f32_32x32x16, reads its LDS
// fragments one k16 sub-step ahead, and between the MFMAs issues the
// global -> LDS DMA (global_load_lds_dwordx4: lane i of a wave writes bytes
// 16 i .. 16 i + 15 of a 1 KiB run, i.e. 8 tile rows) of X two K steps ahead
// into a 3-stage ring.  Waves 4..7 handle W: quantized W is loaded into
// registers and dequantized (to r(q s) in the activation type, as the
// reference GEMM does) into a 2-stage ring one step ahead; dense W goes by
// DMA into a 3-stage ring.  So loads and dequantization run beside the
// MFMAs instead of between them.  One barrier per K step.  LDS rows are 64
// elements (128 B) whose 16-byte slots are XOR-swizzled by swz(row), so the
// fragment reads of 16 consecutive rows hit distinct banks without padding.
// ---------------------------------------------------------------------------
constexpr int G2M = 256, G2K = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16 consecutive quantized weights of one row: raw bits + fp16 scale bits.
template <int FMT> struct WRaw { u32x2 q; uint32_t s; };
template <> struct WRaw<LSSM_W_Q8_G32> { u32x4 q; uint32_t s; };

template <typename T> __device__ __forceinline__ uint32_t pk2(float lo, float hi) {
    if constexpr (__is_same(T, bf16)) {
        typedef __bf16 v2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, v2{(__bf16)lo, (__bf16)hi});
    } else {
        typedef _Float16 v2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, v2{from_f<f16>(lo), from_f<f16>(hi)});
    }
}

// r(q s) for 8 consecutive weights -> 4 packed pairs (k order).  The
// unsigned value u (int4: q + 8, int8: q + 128) of two weights is placed by
// one v_perm into the mantissas of two fp16 values 1024 + u (bits
// 0x6400 | u), and fma(1024 + u, s, c) with c = -(1024 + 8) s (int8:
// -(1024 + 128) s) is q s exactly: both products have at most 11 + 11
// significant bits and q s at most 15, all exact in fp32; the fp16 operands
// convert inside v_fma_mix_f32.  One rounding, at the pack.  int4: q0 holds
// the 8 nibbles (k = nibble index); int8: q0, q1 the 8 bytes.
template <int FMT, typename T>
__device__ __forceinline__ u32x4 dequant8(uint32_t q0, uint32_t q1, float s, float c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    // bytes (b0 of v, 0x64, b1 of v, 0x64) and (b2, 0x64, b3, 0x64)
    auto pair01 = [](uint32_t v) { return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)); };
    auto pair23 = [](uint32_t v) { return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)); };
    auto f = [&](_Float16 e) { return __builtin_fmaf((float)e, s, c); };
    if constexpr (FMT == LSSM_W_Q8_G32) {
        const uint32_t d0 = q0 ^ 0x80808080u, d1 = q1 ^ 0x80808080u;
        const h2 a = pair01(d0), b = pair23(d0), e = pair01(d1), g = pair23(d1);
        return u32x4{pk2<T>(f(a.x), f(a.y)), pk2<T>(f(b.x), f(b.y)), pk2<T>(f(e.x), f(e.y)), pk2<T>(f(g.x), f(g.y))};
    } else {
        // u of k 0, 2, 4, 6 (low nibbles) and k 1, 3, 5, 7
        const uint32_t lo = (q0 & 0x0F0F0F0Fu) ^ 0x08080808u;
        const uint32_t hi = ((q0 >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
        const h2 e02 = pair01(lo), e46 = pair23(lo), e13 = pair01(hi), e57 = pair23(hi);
        return u32x4{pk2<T>(f(e02.x), f(e13.x)), pk2<T>(f(e02.y), f(e13.y)),
                     pk2<T>(f(e46.x), f(e57.x)), pk2<T>(f(e46.y), f(e57.y))};
    }
}
template <int FMT> __device__ __forceinline__ float dequant_bias(float s) {
    return (FMT == LSSM_W_Q8_G32 ? -1152.0f : -1032.0f) * s;
}

// 16 weights -> 8 packed pairs
template <int FMT, typename T>
__device__ __forceinline__ void dequant16(const WRaw<FMT>& r, uint32_t out[8]) {
    const float s = fp16_bits_to_f((uint16_t)r.s), c = dequant_bias<FMT>(s);
    u32x4 a, b;
    if constexpr (FMT == LSSM_W_Q8_G32) {
        a = dequant8<FMT, T>(r.q[0], r.q[1], s, c);
        b = dequant8<FMT, T>(r.q[2], r.q[3], s, c);
    } else {
        a = dequant8<FMT, T>(r.q[0], 0u, s, c);
        b = dequant8<FMT, T>(r.q[1], 0u, s, c);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[i] = a[i];
        out[4 + i] = b[i];
    }
}

__device__ __forceinline__ void lds_dma16(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}
// The same DMA as inline asm, for waves that also read LDS: the compiler does
// not see it, so it does not wait for it before every LDS read (it cannot
// tell which LDS bytes a DMA writes); the issuing wave waits with an explicit
// vmcnt.  m0 (the LDS base of the 1 KiB run) is saved and restored.
__device__ __forceinline__ void lds_dma16_asm(const void* g, uint32_t lds_byte) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(lds_byte)
        : "memory");
}
template <typename T> __device__ __forceinline__ uint32_t lds_addr(const T* p) {
    return (uint32_t)(size_t)((const __attribute__((address_space(3))) T*)p);
}

// LDS tile rows are 128 B (64 16-bit elements, 8 slots of 16 B) and the
// banks repeat every 256 B, so rows r and r + 2 share banks.  Physical slot =
// logical slot ^ ((r / 2) % 8): 16 consecutive rows read or written at one
// logical slot then cover all 16 16-byte positions of the 256 B window (row
// parity picks the half, the XOR the position), with no bank conflict.
__device__ __forceinline__ constexpr uint32_t swz(uint32_t row) { return (row >> 1) & 7u; }

// Workgroups go to the 8 XCDs round-robin in launch order (linear id % 8),
// and each XCD has its own L2.  Give XCD x a contiguous run of the tiles in
// M-major order, so the blocks that share an X row block (all N tiles of one
// M tile) run on one XCD and read X through one L2.  A bijection for any grid.
__device__ __forceinline__ void xcd_tile(uint32_t& mt, uint32_t& nt) {
    const uint32_t nbx = gridDim.x, total = nbx * gridDim.y;
    const uint32_t lin = blockIdx.x + nbx * blockIdx.y;
    const uint32_t x = lin % 8, q = total / 8, r = total % 8;
    const uint32_t tile = x * q + min(x, r) + lin / 8;
    mt = tile / nbx;
    nt = tile % nbx;
}

// CW compute waves: 4 -> 256 x 128 tile, 8 -> 256 x 256 (quantized W only:
// the LDS is then exactly full, 3 x 32 KiB of X + 2 x 32 KiB of W).
template <int FMT, typename T, int EPI, int CW>
__global__ __launch_bounds__(64 * (CW + 4)) void gemm2_kernel(GemmArgs a) {
    constexpr bool DENSE = FMT == LSSM_W_DENSE;
    static_assert(CW == 4 || (CW == 8 && !DENSE), "tile");
    constexpr int BN = 32 * CW;                   // tile columns (rows of W)
    constexpr int SB = DENSE ? 3 : 2;             // W stages (dense W also goes by DMA)
    constexpr int XR = G2M / CW;                  // X rows each compute wave loads
    constexpr bool DB = CW == 4;                  // fragments double-buffered (registers allow)
    __shared__ __attribute__((aligned(16))) T As[3][G2M * G2K];
    __shared__ __attribute__((aligned(16))) T Bs[SB][BN * G2K];
    using Op = MfmaOp<T>;
    using frag = typename Op::frag;

    const int t = threadIdx.x;
    const int lane = t % WAVE;
    const int w = __builtin_amdgcn_readfirstlane(t / WAVE);
    uint32_t tm, tn;
    xcd_tile(tm, tn);
    const uint32_t m0 = tm * G2M, n0 = tn * BN;
    // split K (gridDim.z > 1, small grids): slice z takes steps z KT .. + KT
    // and writes its fp32 sums to a.ws; K stays the row length of X and W
    const uint32_t K = a.K, KT = K / G2K / gridDim.z, kz = blockIdx.z * KT * G2K;
    // a barrier without __syncthreads' release fence (which would wait for
    // every DMA in flight); the empty asm keeps memory operations in place
    auto barrier = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    if (w >= CW) {
        // ---------------- producers: the last 4 waves, W only ----------------
        const int q = w - CW;
        const uint32_t p = t - 64 * CW;
        if constexpr (DENSE) {
            // by DMA: producer wave q fills tile rows 32 q .. + 32, 8 rows per
            // instruction (lane i: row r = run + i / 8, physical slot i % 8 =
            // logical slot (i % 8) ^ swz(r)); rows past N re-read row N - 1.
            const char* wq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t sl = (lane % 8) ^ swz(8 * j + lane / 8);
                const uint32_t n = min(n0 + 32 * q + 8 * j + lane / 8, a.N - 1);
                wq[j] = (const char*)a.w + ((size_t)n * K + kz + 8 * sl) * sizeof(T);
            }
            auto dma_w = [&](uint32_t kt) {
                T* dst = Bs[kt % SB] + (32 * q) * G2K;
#pragma unroll
                for (int j = 0; j < 4; ++j) lds_dma16(wq[j] + (size_t)kt * G2K * sizeof(T), dst + 8 * j * G2K);
            };
            // 4 DMAs per step: vmcnt(4) = the previous step's are done
            dma_w(0);
            dma_w(min(1u, KT - 1));
            __builtin_amdgcn_s_waitcnt(0x0F74);
            barrier();
            for (uint32_t kt = 0; kt < KT; ++kt) {
                dma_w(min(kt + 2, KT - 1));
                __builtin_amdgcn_s_waitcnt(0x0F74);
                barrier();
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);
            return;
        } else {
            // thread p owns row p / TPR of the tile and CPT chunks of 16 k of
            // a step (BN = 128: half a row, BN = 256: a whole row); step k +
            // 2's are loaded into registers at the start of step k (two
            // register sets) and dequantized into LDS in step k + 1.
            constexpr int CPT = BN / 64, TPR = 4 / CPT;
            const uint32_t br = p / TPR, c0 = (p % TPR) * CPT;
            constexpr uint32_t GS = FMT == LSSM_W_Q4_G64 ? 64 : 32;
            const uint32_t nrow = min(n0 + br, a.N - 1);
            const char* wq = (const char*)a.w + (size_t)nrow * (FMT == LSSM_W_Q8_G32 ? K : K / 2) +
                             (FMT == LSSM_W_Q8_G32 ? kz : kz / 2);
            const uint16_t* sp = (const uint16_t*)a.s + (size_t)nrow * (K / GS) + kz / GS;
            using R = WRaw<FMT>;
            auto load_w = [&](uint32_t kt, R (&r)[CPT]) {
#pragma unroll
                for (int h = 0; h < CPT; ++h) {
                    const uint32_t k = kt * G2K + 16 * (c0 + h);
                    if constexpr (FMT == LSSM_W_Q8_G32) r[h].q = *reinterpret_cast<const u32x4*>(wq + k);
                    else r[h].q = *reinterpret_cast<const u32x2*>(wq + k / 2);
                    r[h].s = sp[k / GS];
                }
            };
            auto store_w = [&](uint32_t kt, const R (&r)[CPT]) {
                T* Brow = Bs[kt % SB] + br * G2K;
                const uint32_t sw = swz(br);
#pragma unroll
                for (int h = 0; h < CPT; ++h) {
                    uint32_t d[8];
                    dequant16<FMT, T>(r[h], d);
                    const uint32_t s0 = 2 * (c0 + h);
                    *reinterpret_cast<u32x4*>(Brow + 8 * (s0 ^ sw)) = u32x4{d[0], d[1], d[2], d[3]};
                    *reinterpret_cast<u32x4*>(Brow + 8 * ((s0 + 1) ^ sw)) = u32x4{d[4], d[5], d[6], d[7]};
                }
            };
            R r0[CPT], r1[CPT];
            load_w(0, r0);
            load_w(min(1u, KT - 1), r1);
            store_w(0, r0);
            __builtin_amdgcn_s_waitcnt(0xC07F);
            barrier();
            // step kt: load step kt + 2, then write step kt + 1 (its loads were
            // issued a step ago).  Branch-free: past the end it re-loads step
            // KT - 1 and writes the idle stage.
            auto step = [&](uint32_t kt, R (&ld)[CPT], const R (&wr)[CPT]) {
                load_w(min(kt + 2, KT - 1), ld);
                __builtin_amdgcn_sched_barrier(0);    // loads first
                store_w(kt + 1, wr);
                __builtin_amdgcn_s_waitcnt(0xC07F);
                barrier();
            };
            uint32_t kt = 0;
            for (; kt + 1 < KT; kt += 2) {
                step(kt, r0, r1);
                step(kt + 1, r1, r0);
            }
            if (kt < KT) step(kt, r0, r1);
            return;
        }
    }

    // ---------------- compute waves: 128 x 64 of Y each ----------------
    // They also DMA X: wave c fills tile rows XR c .. + XR of the stage two
    // steps ahead, 8 rows per instruction (lane i: row r = run + i / 8,
    // physical slot i % 8 = logical slot (i % 8) ^ swz(r); XR c is a multiple
    // of 16); rows past M re-read row M - 1.
    const int wm = w / (CW / 2), wn = w % (CW / 2);
    constexpr int XJ = XR / 8;                    // DMA instructions per step
    uint32_t xo[XJ];
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
        const uint32_t xl = (lane % 8) ^ swz(8 * j + lane / 8);
        const uint32_t m = min(m0 + XR * w + 8 * j + lane / 8, a.M - 1);
        xo[j] = (m * a.x_stride + 8 * xl) * (uint32_t)sizeof(T);
    }
    const uint32_t as0 = lds_addr(&As[0][0]) + (XR * w) * G2K * (uint32_t)sizeof(T);
    auto dma_x = [&](uint32_t kt, int j0, int j1) {
        const char* base = (const char*)a.x + ((size_t)kz + (size_t)kt * G2K) * sizeof(T);
        const uint32_t dst = as0 + (kt % 3) * (G2M * G2K * (uint32_t)sizeof(T));
        for (int j = j0; j < j1; ++j) lds_dma16_asm(base + xo[j], dst + 8 * j * G2K * (uint32_t)sizeof(T));
    };

    // row scales of the wave's 128 tile rows, requested now and spread over
    // the lanes (lane l: rows l and 64 + l of the half): the epilogue takes
    // each row's from its lane by readlane instead of waiting, per 32-row
    // block, on 16 scattered loads
    float rs_lo = 1.0f, rs_hi = 1.0f;
    if (a.row_scale && gridDim.z == 1) {
        const uint32_t mb = m0 + wm * 128;
        rs_lo = a.row_scale[min(mb + lane, a.M - 1)];
        rs_hi = a.row_scale[min(mb + 64 + lane, a.M - 1)];
    }

    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // fragment offsets (elements): fragment rows are 32 i + lane % 32 (tile
    // bases are multiples of 16), so swz(row) == swz(lane % 32)
    uint32_t fo[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) fo[ks] = (lane % 32) * G2K + 8 * ((2 * ks + lane / 32) ^ swz(lane % 32));

    // XJ DMAs per step: vmcnt(XJ) = the previous step's are done
    auto wait_prev = [] {
        if constexpr (XJ == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    };
    dma_x(0, 0, XJ);
    dma_x(min(1u, KT - 1), 0, XJ);
    wait_prev();
    barrier();                                    // step 0 in LDS
    for (uint32_t kt = 0; kt < KT; ++kt) {
        const T* Ab = As[kt % 3] + (wm * 128) * G2K;
        const T* Bb = Bs[kt % SB] + (wn * 64) * G2K;
        const uint32_t k2 = min(kt + 2, KT - 1);
        frag af[DB ? 2 : 1][4], bfr[DB ? 2 : 1][2];
        auto rd = [&](int ks, frag (&fa)[4], frag (&fb)[2]) {
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const frag*>(Ab + 32 * i * G2K + fo[ks]);
#pragma unroll
            for (int j = 0; j < 2; ++j) fb[j] = *reinterpret_cast<const frag*>(Bb + 32 * j * G2K + fo[ks]);
        };
        if constexpr (DB) rd(0, af[0], bfr[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int cb = DB ? ks % 2 : 0;
            if constexpr (DB) {
                if (ks + 1 < 4) rd(ks + 1, af[(ks + 1) % 2], bfr[(ks + 1) % 2]);
            } else {
                // two compute waves per SIMD hide the LDS latency instead
                rd(ks, af[0], bfr[0]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = Op::mma(af[cb][i], bfr[cb][j], acc[i][j]);
            if constexpr (DB) {
                // next sub-step's fragment reads ahead of this sub-step's
                // MFMAs (the asm DMA below ends the scheduling region)
                if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
                else if (ks < 3) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            }
            // step kt + 2's X, spread over the sub-steps
            dma_x(k2, ks * XJ / 4, (ks + 1) * XJ / 4);
        }
        // step kt + 1's X in LDS, this step's fragment reads done
        if constexpr (XJ == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
        barrier();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // D layout of v_mfma_f32_32x32x*: element r of lane l is
    // row (r/4)*8 + (l/32)*4 + r%4, column l%32.
    if (gridDim.z > 1) {
        float* ws = a.ws + (size_t)blockIdx.z * a.M * a.N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t n = n0 + wn * 64 + j * 32 + lane % 32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t m = m0 + wm * 128 + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + r % 4;
                    if (m < a.M && n < a.N) ws[(size_t)m * a.N + n] = acc[i][j][r];
                }
            }
        }
        return;
    }
    T* Y = (T*)a.y;
    const T* Rz = (const T*)a.res;
    const bool vec = a.y_stride % 8 == 0 && (uintptr_t)a.y % 16 == 0 &&
                     (EPI != LSSM_EPI_ADD || (uintptr_t)a.res % 16 == 0);
    if (vec) {
        // The tile goes through LDS (rows 0..127 over the X stages, 128..255
        // over the W stages) as the rounded outputs, then out in 16-byte runs
        // of 8 columns: scattered 2-byte stores (and residual loads) cost the
        // tile's last round ~13 % of the out_proj launch.  Same arithmetic:
        // r(acc) / r(silu(acc)) staged, the residual added to the staged value.
        constexpr uint32_t RB = BN * 2;                        // staged row bytes
        char* half = wm == 0 ? reinterpret_cast<char*>(&As[0][0]) : reinterpret_cast<char*>(&Bs[0][0]);
        // 16-byte slot s of row r sits at slot s ^ 4 ((r / 4) % 2): rows r and
        // r + 4 (one store instruction) fall in different banks
        auto slot_of = [](uint32_t r, uint32_t sl) { return sl ^ (4u * ((r >> 2) & 1u)); };
        barrier();                                             // every wave's DMAs and reads done
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // the row scales of this thread's 16 rows of the 32-row block i:
            // row rr of the half is lane rr % 64 of rs_lo (rr < 64) or rs_hi;
            // lanes 0..31 take row r0, lanes 32..63 row r0 + 4
            float rsv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t r0 = i * 32 + (r / 4) * 8 + r % 4, r1 = r0 + 4;
                const float s0 = readlane_f(r0 < 64 ? rs_lo : rs_hi, (int)(r0 % 64));
                const float s1 = readlane_f(r1 < 64 ? rs_lo : rs_hi, (int)(r1 % 64));
                rsv[r] = lane < 32 ? s0 : s1;
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t c = wn * 64 + j * 32 + lane % 32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t rr = i * 32 + (r / 4) * 8 + (lane / 32) * 4 + r % 4;
                    float v = acc[i][j][r];
                    if (a.row_scale) v *= rsv[r];
                    if (n0 + c < a.silu_cols) v = silu_fast(v);
                    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
                    *reinterpret_cast<T*>(half + rr * RB + 16 * slot_of(rr, c / 8) + 2 * (c % 8)) = from_f<T>(v);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);                    // lgkmcnt(0)
        barrier();
        constexpr uint32_t SPR = BN / 8;                       // slots per row
        constexpr uint32_t NT = 64 * CW;
        // a thread's slot (NT % SPR == 0): the next norm's weights of its 8
        // columns, one load for all its rows
        u32x4 y2w{0u, 0u, 0u, 0u};
        if (EPI == LSSM_EPI_ADD && a.y2) {
            const uint32_t nw = n0 + 8 * (threadIdx.x % SPR);
            if (nw + 8 <= a.N) y2w = *reinterpret_cast<const u32x4*>((const T*)a.y2_w + nw);
        }
#pragma unroll 4
        for (uint32_t q = threadIdx.x; q < G2M * SPR; q += NT) {
            const uint32_t R = q / SPR, sl = q % SPR, rr = R % 128;
            const char* hp = R < 128 ? reinterpret_cast<const char*>(&As[0][0]) : reinterpret_cast<const char*>(&Bs[0][0]);
            const u32x4 st = *reinterpret_cast<const u32x4*>(hp + rr * RB + 16 * slot_of(rr, sl));
            const uint32_t m = m0 + R, n = n0 + 8 * sl;
            if (m >= a.M) continue;
            const size_t yi = (size_t)m * a.y_stride + n;
            if (n + 8 <= a.N) {
                if constexpr (EPI == LSSM_EPI_ADD) {
                    const u32x4 rv = *reinterpret_cast<const u32x4*>(Rz + yi);
                    u32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = f_of_bits<T>((uint16_t)rv[e]) + f_of_bits<T>((uint16_t)st[e]);
                        const float hi = f_of_bits<T>((uint16_t)(rv[e] >> 16)) + f_of_bits<T>((uint16_t)(st[e] >> 16));
                        o[e] = (uint32_t)__builtin_bit_cast(uint16_t, from_f<T>(lo)) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, from_f<T>(hi)) << 16);
                    }
                    *reinterpret_cast<u32x4*>(Y + yi) = o;
                    if (a.y2) {
                        // the next RMSNorm's input r(y w) and the sums of y^2
                        // over the 128 columns of this thread's 16-lane row
                        // (the rows of a DPP row share m; N % 128 == 0)
                        const u32x4 wv = y2w;
                        u32x4 o2;
                        float sq = 0.0f;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float lo = f_of_bits<T>((uint16_t)o[e]);
                            const float hi = f_of_bits<T>((uint16_t)(o[e] >> 16));
                            sq = fmaf(lo, lo, sq);
                            sq = fmaf(hi, hi, sq);
                            const float wl = f_of_bits<T>((uint16_t)wv[e]);
                            const float wh = f_of_bits<T>((uint16_t)(wv[e] >> 16));
                            o2[e] = (uint32_t)__builtin_bit_cast(uint16_t, from_f<T>(lo * wl)) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, from_f<T>(hi * wh)) << 16);
                        }
                        *reinterpret_cast<u32x4*>((T*)a.y2 + yi) = o2;
                        sq = group_sum<16>(sq);
                        if (threadIdx.x % 16 == 0) a.y2_part[(size_t)(n / 128) * a.M + m] = sq;
                    }
                } else {
                    *reinterpret_cast<u32x4*>(Y + yi) = st;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (n + e >= a.N) break;
                    const uint16_t sb = (uint16_t)(st[e / 2] >> (16 * (e % 2)));
                    float v = f_of_bits<T>(sb);
                    if (EPI == LSSM_EPI_ADD) v = to_f(Rz[yi + e]) + v;
                    Y[yi + e] = from_f<T>(v);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + lane % 32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + wm * 128 + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + r % 4;
                if (m < a.M && n < a.N) {
                    const size_t yi = (size_t)m * a.y_stride + n;
                    float v = acc[i][j][r];
                    if (a.row_scale) v *= a.row_scale[m];
                    if (n < a.silu_cols) v = silu_fast(v);
                    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
                    if (EPI == LSSM_EPI_ADD) v = to_f(Rz[yi]) + rnd<T>(v);
                    Y[yi] = from_f<T>(v);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for decode batches (5 <= M <= 64): the weights are streamed once.
// A block covers 16 rows of W; its KS waves split K into slices of UPW units,
// and the slices are summed in LDS.  A lane loads 16 bytes of one W row per
// unit (int4: 32 k, int8: 16, dense: 8) and dequantizes them (to r(q s), GEMM
// semantics) straight into v_mfma_f32_16x16x32 A operands: MFMA k-step s of a
// unit takes, in lane group q = lane / 16, the k = unit + KPL q + 8 s .. + 8
// (the k order inside an MFMA is free as long as both operands follow it), so
// x is read as matching 16-byte runs of its rows (L2-resident, shared by all
// blocks).  All loads of a wave are issued before its first MFMA.
// ---------------------------------------------------------------------------
template <int FMT> struct SkUnit {
    static constexpr int KPL = FMT == LSSM_W_DENSE ? 8 : (FMT == LSSM_W_Q8_G32 ? 16 : 32);
    static constexpr int U = 4 * KPL;            // k per unit
    static constexpr int STEPS = KPL / 8;        // MFMA k-steps per unit
};
constexpr int SK_MAXW = 16;                      // K slices (waves) per block

template <typename T> __device__ __forceinline__ floatx4 mma16x32(u32x4 a, u32x4 b, floatx4 c) {
    if constexpr (__is_same(T, bf16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

template <int FMT, typename T, int EPI, int MT, int UPW>
__global__ __launch_bounds__(64 * SK_MAXW) void gemm_skinny_kernel(GemmArgs a) {
    using SU = SkUnit<FMT>;
    constexpr int KPL = SU::KPL, U = SU::U, STEPS = SU::STEPS;
    constexpr uint32_t GS = FMT == LSSM_W_Q4_G64 ? 64 : 32;
    __shared__ floatx4 red[SK_MAXW - 1][MT][64];

    const int lane = threadIdx.x % WAVE;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int KS = blockDim.x / WAVE;
    const int li = lane % 16, lq = lane / 16;
    const uint32_t n0 = blockIdx.x * 16;
    const uint32_t K = a.K, kb = w * (UPW * U);
    const uint32_t n = min(n0 + li, a.N - 1);

    const char* wrow;
    const uint16_t* srow = nullptr;
    if constexpr (FMT == LSSM_W_DENSE) wrow = (const char*)a.w + (size_t)n * K * sizeof(T);
    else {
        wrow = (const char*)a.w + (size_t)n * (FMT == LSSM_W_Q8_G32 ? K : K / 2);
        srow = (const uint16_t*)a.s + (size_t)n * (K / GS);
    }
    const T* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xrow[mt] = (const T*)a.x + (size_t)min(16u * mt + li, a.M - 1) * a.x_stride;

    struct Unit { u32x4 w; uint32_t s; u32x4 x[MT][STEPS]; };
    Unit r[UPW];
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
        const uint32_t k = kb + uu * U + KPL * lq;
        if constexpr (FMT == LSSM_W_DENSE) r[uu].w = *reinterpret_cast<const u32x4*>(wrow + (size_t)k * sizeof(T));
        else if constexpr (FMT == LSSM_W_Q8_G32) r[uu].w = *reinterpret_cast<const u32x4*>(wrow + k);
        else r[uu].w = *reinterpret_cast<const u32x4*>(wrow + k / 2);
        if constexpr (FMT != LSSM_W_DENSE) r[uu].s = srow[k / GS];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int st = 0; st < STEPS; ++st) r[uu].x[mt][st] = *reinterpret_cast<const u32x4*>(xrow[mt] + k + 8 * st);
    }
    // all loads in flight before the first MFMA (when they fit the registers:
    // 16-wave blocks leave 128 VGPRs)
    if constexpr (UPW * MT <= 4) __builtin_amdgcn_sched_barrier(0);
    floatx4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int uu = 0; uu < UPW; ++uu) {
        u32x4 af[STEPS];
        if constexpr (FMT == LSSM_W_DENSE) {
            af[0] = r[uu].w;
        } else if constexpr (FMT == LSSM_W_Q8_G32) {
            WRaw<FMT> q{r[uu].w, r[uu].s};
            uint32_t d[8];
            dequant16<FMT, T>(q, d);
            af[0] = u32x4{d[0], d[1], d[2], d[3]};
            af[1] = u32x4{d[4], d[5], d[6], d[7]};
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                WRaw<FMT> q{u32x2{r[uu].w[2 * h], r[uu].w[2 * h + 1]}, r[uu].s};
                uint32_t d[8];
                dequant16<FMT, T>(q, d);
                af[2 * h] = u32x4{d[0], d[1], d[2], d[3]};
                af[2 * h + 1] = u32x4{d[4], d[5], d[6], d[7]};
            }
        }
#pragma unroll
        for (int st = 0; st < STEPS; ++st)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = mma16x32<T>(af[st], r[uu].x[mt][st], acc[mt]);
    }

    // sum the K slices; wave 0 stores.  D element r of lane l: row
    // 4 (l / 16) + r (W row n0 + .), column l % 16 (x row 16 mt + .).
    if (w > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[w - 1][mt][lane] = acc[mt];
    }
    __syncthreads();
    if (w != 0) return;
    T* Y = (T*)a.y;
    const T* R = (const T*)a.res;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        floatx4 v = acc[mt];
        for (int q = 0; q < KS - 1; ++q) v += red[q][mt][lane];
        const uint32_t m = 16 * mt + li;
        if (m >= a.M) continue;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const uint32_t nn = n0 + 4 * lq + rr;
            if (nn >= a.N) continue;
            const size_t yi = (size_t)m * a.y_stride + nn;
            float o = v[rr];
            if (a.row_scale) o *= a.row_scale[m];
            if (nn < a.silu_cols) o = silu_fast(o);
            if (EPI == LSSM_EPI_SILU) o = silu_f(o);
            if (EPI == LSSM_EPI_ADD) o = to_f(R[yi]) + rnd<T>(o);
            Y[yi] = from_f<T>(o);
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
    if (a.row_scale) v *= a.row_scale[m];
    if (n < a.silu_cols) v = silu_fast(v);
    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
    if (EPI == LSSM_EPI_ADD) v = to_f(((const T*)a.res)[yi]) + rnd<T>(v);
    ((T*)a.y)[yi] = from_f<T>(v);
}

template <int FMT, typename T, int MT, int UPW>
hipError_t go_skinny(hipStream_t s, const GemmArgs& a) {
    const dim3 grid((a.N + 15) / 16);
    const dim3 block(64 * (a.K / (UPW * SkUnit<FMT>::U)));
    switch (a.epi) {
        case LSSM_EPI_SILU: gemm_skinny_kernel<FMT, T, LSSM_EPI_SILU, MT, UPW><<<grid, block, 0, s>>>(a); break;
        case LSSM_EPI_ADD: gemm_skinny_kernel<FMT, T, LSSM_EPI_ADD, MT, UPW><<<grid, block, 0, s>>>(a); break;
        default: gemm_skinny_kernel<FMT, T, LSSM_EPI_NONE, MT, UPW><<<grid, block, 0, s>>>(a); break;
    }
    return hipGetLastError();
}

// Units per wave for the skinny GEMM: preferably 4 / MT (all of a wave's loads
// then fit in registers at once), else the nearest that splits K into at most
// SK_MAXW whole slices; 0 = not supported.
template <int FMT> int skinny_upw(uint32_t K, int mt) {
    constexpr uint32_t U = SkUnit<FMT>::U;
    const int pref = 4 / mt;
    const int order[3][3] = {{1, 2, 4}, {2, 1, 4}, {4, 2, 1}};
    for (int upw : order[pref == 1 ? 0 : (pref == 2 ? 1 : 2)])
        if (K % (upw * U) == 0 && K / (upw * U) <= (uint32_t)SK_MAXW) return upw;
    return 0;
}

template <int FMT, typename T, int MT>
hipError_t go_skinny_mt(hipStream_t s, const GemmArgs& a, int upw) {
    if (upw == 4) return go_skinny<FMT, T, MT, 4>(s, a);
    if (upw == 2) return go_skinny<FMT, T, MT, 2>(s, a);
    return go_skinny<FMT, T, MT, 1>(s, a);
}

// The split slices' fp32 sums added in slice order, then gemm2_kernel's
// epilogue: r(v), r(silu(v)) or r(res + r(v)).
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_split_sum_kernel(GemmArgs a, uint32_t S) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, MN = (size_t)a.M * a.N;
    if (i >= MN) return;
    float v = 0.0f;
    for (uint32_t z = 0; z < S; ++z) v += a.ws[z * MN + i];
    const uint32_t m = (uint32_t)(i / a.N), n = (uint32_t)(i % a.N);
    const size_t yi = (size_t)m * a.y_stride + n;
    if (a.row_scale) v *= a.row_scale[m];
    if (n < a.silu_cols) v = silu_fast(v);
    if (EPI == LSSM_EPI_SILU) v = silu_f(v);
    if (EPI == LSSM_EPI_ADD) v = to_f(((const T*)a.res)[yi]) + rnd<T>(v);
    ((T*)a.y)[yi] = from_f<T>(v);
}

// The same, four consecutive outputs a thread (N and the row strides
// multiples of 4): 16-byte loads of the slices' sums.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_split_sum4_kernel(GemmArgs a, uint32_t S) {
    const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x, MN = (size_t)a.M * a.N;
    if (4 * q >= MN) return;
    floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t z = 0; z < S; ++z) {
        const floatx4 p = reinterpret_cast<const floatx4*>(a.ws + z * MN)[q];
        v[0] += p[0];
        v[1] += p[1];
        v[2] += p[2];
        v[3] += p[3];
    }
    const uint32_t m = (uint32_t)(4 * q / a.N), n = (uint32_t)(4 * q % a.N);
    const size_t yi = (size_t)m * a.y_stride + n;
    T o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float x = v[e];
        if (a.row_scale) x *= a.row_scale[m];
        if (n + e < a.silu_cols) x = silu_fast(x);
        if (EPI == LSSM_EPI_SILU) x = silu_f(x);
        if (EPI == LSSM_EPI_ADD) x = to_f(((const T*)a.res)[yi + e]) + rnd<T>(x);
        o[e] = from_f<T>(x);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ((T*)a.y)[yi + e] = o[e];
}

// K slices for a prefill GEMM whose 256 x 128 tiles would leave most CUs idle
// (the 130M out_proj at 2048 rows: 48 tiles): as many as fill about half the
// CUs, K / 64 divisible, the workspace large enough; 1 = no split.
inline uint32_t gemm_split(const GemmArgs& a, uint32_t gs) {
    static const bool off = [] {
        const char* v = getenv("LSSM_GEMM_SPLIT");
        return v && v[0] == '0';
    }();
    if (!a.ws || off) return 1;
    const size_t narrow = (size_t)((a.M + G2M - 1) / G2M) * ((a.N + 127) / 128), cus = num_cus();
    if (2 * narrow > cus) return 1;
    uint32_t S = 1;
    for (uint32_t c : {2u, 4u, 8u})
        if (narrow * c <= cus && (a.K / G2K) % c == 0 && (a.K / c) % gs == 0 &&
            (size_t)c * a.M * a.N <= a.ws_floats)
            S = c;
    return S;
}

template <int FMT, typename T>
hipError_t go_epi(hipStream_t s, const GemmArgs& a) {
    // decode batches: weights streamed once
    if (a.M <= 64) {
        const int mt = a.M <= 16 ? 1 : (a.M <= 32 ? 2 : 4);
        if (const int upw = skinny_upw<FMT>(a.K, mt)) {
            if (mt == 1) return go_skinny_mt<FMT, T, 1>(s, a, upw);
            if (mt == 2) return go_skinny_mt<FMT, T, 2>(s, a, upw);
            return go_skinny_mt<FMT, T, 4>(s, a, upw);
        }
    }
    // the large tile for prefill-sized M; X byte offsets within a 256-row
    // tile fit 32 bits
    if (a.M > 128 && (uint64_t)a.M * a.x_stride * sizeof(T) < (1ull << 31)) {
        // 256-wide tiles halve the X re-reads: a wide tile takes about 1.5x
        // the time of a 128-wide one (measured at the 2.7B out_proj shape),
        // so take them when their rounds of blocks (one block per CU) cost
        // less: 1.5 ceil(wide tiles / CUs) <= ceil(narrow tiles / CUs)
        const uint32_t mt = (a.M + G2M - 1) / G2M;
        const size_t cus = num_cus();
        const size_t rw = (mt * (size_t)((a.N + 255) / 256) + cus - 1) / cus;
        const size_t rn = (mt * (size_t)((a.N + 127) / 128) + cus - 1) / cus;
        const bool wide = FMT != LSSM_W_DENSE && 3 * rw <= 2 * rn;
        auto run_wide = [&](const GemmArgs& g) {
            dim3 grid((g.N + 255) / 256, mt);
            if constexpr (FMT != LSSM_W_DENSE) {
                switch (g.epi) {
                    case LSSM_EPI_SILU: gemm2_kernel<FMT, T, LSSM_EPI_SILU, 8><<<grid, 768, 0, s>>>(g); break;
                    case LSSM_EPI_ADD: gemm2_kernel<FMT, T, LSSM_EPI_ADD, 8><<<grid, 768, 0, s>>>(g); break;
                    default: gemm2_kernel<FMT, T, LSSM_EPI_NONE, 8><<<grid, 768, 0, s>>>(g); break;
                }
            }
        };
        const uint32_t S = FMT == LSSM_W_DENSE ? 1u : gemm_split(a, FMT == LSSM_W_Q4_G64 ? 64u : 32u);
        if (S > 1) {
            // small grid: K in S slices, then the slices' sums (one launch)
            dim3 grid((a.N + 127) / 128, mt, S);
            gemm2_kernel<FMT, T, LSSM_EPI_NONE, 4><<<grid, 512, 0, s>>>(a);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            if (a.N % 4 == 0 && (uintptr_t)a.ws % 16 == 0) {
                const unsigned nb = (unsigned)(((size_t)a.M * a.N / 4 + 255) / 256);
                switch (a.epi) {
                    case LSSM_EPI_SILU: gemm_split_sum4_kernel<T, LSSM_EPI_SILU><<<nb, 256, 0, s>>>(a, S); break;
                    case LSSM_EPI_ADD: gemm_split_sum4_kernel<T, LSSM_EPI_ADD><<<nb, 256, 0, s>>>(a, S); break;
                    default: gemm_split_sum4_kernel<T, LSSM_EPI_NONE><<<nb, 256, 0, s>>>(a, S); break;
                }
                return hipGetLastError();
            }
            const unsigned nb = (unsigned)(((size_t)a.M * a.N + 255) / 256);
            switch (a.epi) {
                case LSSM_EPI_SILU: gemm_split_sum_kernel<T, LSSM_EPI_SILU><<<nb, 256, 0, s>>>(a, S); break;
                case LSSM_EPI_ADD: gemm_split_sum_kernel<T, LSSM_EPI_ADD><<<nb, 256, 0, s>>>(a, S); break;
                default: gemm_split_sum_kernel<T, LSSM_EPI_NONE><<<nb, 256, 0, s>>>(a, S); break;
            }
            return hipGetLastError();
        }
        auto run_narrow = [&](const GemmArgs& g) {
            dim3 grid((g.N + 127) / 128, mt);
            switch (g.epi) {
                case LSSM_EPI_SILU: gemm2_kernel<FMT, T, LSSM_EPI_SILU, 4><<<grid, 512, 0, s>>>(g); break;
                case LSSM_EPI_ADD: gemm2_kernel<FMT, T, LSSM_EPI_ADD, 4><<<grid, 512, 0, s>>>(g); break;
                default: gemm2_kernel<FMT, T, LSSM_EPI_NONE, 4><<<grid, 512, 0, s>>>(g); break;
            }
        };
        if (wide) {
            // A last round of wide tiles at most half full (2.7B out_proj: 640
            // tiles = 2.5 rounds) runs instead as one round of narrow tiles,
            // which take about two thirds of a wide tile's time: the columns of
            // the full rounds go to the wide launch, the rest to a narrow one
            // (pointers offset by whole output columns, so each output is
            // computed exactly as in the single launch).
            const size_t wt = mt * (size_t)((a.N + 255) / 256);
            const size_t full = wt / cus, rem = wt % cus;
            const uint32_t n1 = full ? (uint32_t)((full * cus) / mt) * 256u : 0u;
            const bool split = full >= 1 && rem > 0 && 2 * rem <= cus && n1 > 0 && n1 < a.N &&
                               mt * (size_t)((a.N - n1 + 127) / 128) <= cus;
            if (!split) {
                run_wide(a);
                return hipGetLastError();
            }
            GemmArgs a1 = a, a2 = a;
            a1.N = n1;
            a2.N = a.N - n1;
            const size_t wrow = FMT == LSSM_W_Q8_G32 ? a.K : a.K / 2;     // packed bytes per W row
            const uint32_t gs = FMT == LSSM_W_Q4_G64 ? 64u : 32u;
            a2.w = (const uint8_t*)a.w + (size_t)n1 * wrow;
            a2.s = (const uint16_t*)a.s + (size_t)n1 * (a.K / gs);
            a2.y = (T*)a.y + n1;
            if (a.res) a2.res = (const T*)a.res + n1;
            a2.silu_cols = a.silu_cols > n1 ? a.silu_cols - n1 : 0u;   // columns count from n1
            if (a.y2) {
                a2.y2 = (T*)a.y2 + n1;
                a2.y2_w = (const T*)a.y2_w + n1;
                a2.y2_part = a.y2_part + (size_t)(n1 / 128) * a.M;
            }
            run_wide(a1);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            run_narrow(a2);
            return hipGetLastError();
        }
        run_narrow(a);
        return hipGetLastError();
    }
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

bool gemm_norm_fold_takes(const GemmArgs& a) {
    const size_t es = 2;
    if (a.act != LSSM_F16 && a.act != LSSM_BF16) return false;
    if (a.epi != LSSM_EPI_ADD || !a.res || !a.y2 || !a.y2_w || !a.y2_part) return false;
    if (a.M <= 128 || (uint64_t)a.M * a.x_stride * es >= (1ull << 31)) return false;
    if (a.N % 128 != 0 || a.y_stride % 8 != 0) return false;
    for (const void* p : {(const void*)a.y, a.res, (const void*)a.y2, a.y2_w})
        if ((uintptr_t)p % 16 != 0) return false;
    if (a.wfmt != LSSM_W_DENSE && gemm_split(a, a.wfmt == LSSM_W_Q4_G64 ? 64u : 32u) > 1) return false;
    return true;
}

hipError_t launch_gemm(hipStream_t s, const GemmArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.y2 && !gemm_norm_fold_takes(a)) return hipErrorInvalidValue;
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

// gemv_mma.hip — decode batches of 2..64 rows on MFMA with the GEMV rule
// (exact dequantization, linear.metal:440-474), RMSNorm prologue and the
// per-row epilogues of gemv.hip fused.
#include <algorithm>
#include <cstdlib>

#include "gemv_core.hpp"

namespace lssm {

namespace {

// ---------------------------------------------------------------------------
// gemv_mma: decode batches (2..64 rows of x) on v_mfma_f32_16x16x32, GEMV rule
// ---------------------------------------------------------------------------
// y[m, n] = epi(sum_g s[n, g] * sum_{k in g} q[n, k] x[m, k]): the unpacked
// integers (136 + q for int4 x bf16, whose 136 * sum(x) per group is taken off
// again; exact q otherwise) are the MFMA operands and each group's fp32 sum is
// scaled once, so no weight is rounded (linear.metal:440-474), as in gemv1.
//
// A block owns CT tiles of 16 W rows; its KS waves split K into whole quads
// (QK = 4 chunks of one row: one 16-byte load by each of the row's 4 lanes),
// QPW quads per wave.  MFMA operands: A = x (16 batch rows), B = W (16 W rows
// as columns); lane l = 16 q + i supplies row i and k-slice q (8 values) of an
// MFMA's 32, and holds D rows 4 q .. 4 q + 3 (batch) of column i (W row) after
// it.  An MFMA must stay inside one scale group, so after the load the 4 lanes
// of a row trade dwords (v_permlane32_swap for 64-wide groups, and then
// v_permlane16_swap for 32-wide ones) until each k-slice a lane supplies lies
// in one group; x is read from LDS in the matching order.
//
// x rows [base, base + mpb) are staged per pass, RMSNorm'ed when fused
// (norm.metal:52-79: r((x w) rrms), rrms = 1 / sqrt(mean(x^2) + eps)), in LDS
// as the packed pairs of the weight unpack (pair_pos order, row pitch K/2 + 4
// dwords: the 16-byte reads of 8 consecutive rows fall in distinct banks),
// plus each group's sum(x) for the int4 x bf16 bias.  More rows than fit take
// further passes over the same weights, which stay in registers.  The weights
// are requested after the staging barrier: x is not queued behind them.  The
// KS partial sums meet in LDS, summed in wave order (deterministic); wave t
// finishes tile t through the epilogue.
// Waves per block a (tiles, quads per wave) shape is built for: more weight
// registers per lane, fewer waves (VGPRs per lane: 128 / 168 / 256).
constexpr int mma_waves(int ct, int qpw) { return ct * qpw <= 2 ? 16 : (ct * qpw <= 8 ? 12 : 8); }
// The instantiated shapes: several tiles per block for int4 only (the large
// models' formats).
constexpr bool mma_shape_ok(int ct, int qpw, bool q4) {
    return (ct == 1 && (qpw == 1 || qpw == 2 || qpw == 4 || qpw == 8)) ||
           (q4 && ((qpw == 2 && ct >= 2 && ct <= 4) || (ct == 4 && qpw == 4)));
}
constexpr int MM_MAXJ = 8;                       // staged octets per thread and pass
constexpr size_t MM_LDS_MAX = 150 * 1024;        // dynamic LDS (static: < 5 KiB)

template <int V> struct FmtTag {
    static constexpr int value = V;
};

template <int FMT, typename T> struct Mma {
    using F = Fmt<FMT, T>;
    static constexpr int WPC = F::WPC;
    static constexpr int NP = WPC / 2;                                  // pairs per chunk
    static constexpr int QK = 4 * WPC;                                  // k per quad
    static constexpr int G = F::G;                                      // 0: dense
    static constexpr int SPQ = FMT == LSSM_W_DENSE ? 1 : (FMT == LSSM_W_Q8_G32 ? 2 : 4);  // MFMAs per quad
    static constexpr int GPQ = G ? QK / G : 1;                          // scale groups per quad
    static constexpr int SPG = SPQ / GPQ;                               // MFMAs per group
    static constexpr bool BIAS = q4_bf16<FMT, T>();
};

// Chunk (within the quad) and pair offset of MFMA k-slice s of lane group q,
// after mma_swap: the x pairs that slice s meets in lane group q.
template <int FMT> __device__ __forceinline__ void mma_slice_pos(int s, int q, int& ch, int& po) {
    if constexpr (FMT == LSSM_W_Q4_G64) {
        ch = (q & 1) + 2 * (s >> 1);
        po = 4 * ((s & 1) + 2 * (q >> 1));
    } else if constexpr (FMT == LSSM_W_Q4_B32) {
        ch = s;
        po = 4 * q;
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
        ch = (q & 1) + 2 * s;
        po = 4 * (q >> 1);
    } else {
        ch = q;
        po = 0;
    }
}

// Lane group q loaded chunk q of the quad (dwords C_q[0..3]).  After the
// 32-lane swap, lane group q holds C_{q&1}[2(q>>1)], C_{q&1}[2(q>>1)+1],
// C_{(q&1)+2}[2(q>>1)], C_{(q&1)+2}[2(q>>1)+1]: dwords 0-1 come from chunks
// 0-1 and dwords 2-3 from chunks 2-3 (one 64-wide group each).  After the
// 16-lane swap as well it holds C_0[q], C_1[q], C_2[q], C_3[q] (dword j from
// chunk j: one 32-wide group each).
template <int FMT> __device__ __forceinline__ u32x4 mma_swap(u32x4 v) {
    if constexpr (FMT == LSSM_W_DENSE) {
        return v;
    } else {
        const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
        u32x4 r = u32x4{a[0], b[0], a[1], b[1]};
        if constexpr (FMT == LSSM_W_Q4_B32) {
            const auto c = __builtin_amdgcn_permlane16_swap(r[0], r[1], false, false);
            const auto d = __builtin_amdgcn_permlane16_swap(r[2], r[3], false, false);
            r = u32x4{c[0], c[1], d[0], d[1]};
        }
        return r;
    }
}

// Pair q of an octet (8 consecutive k, 8-aligned) in pair_pos order: the
// positions (within the octet) of its two values.  Octets never straddle the
// pair structure of a chunk, so these are constants.
template <int FMT, typename T> __device__ __forceinline__ void octet_pos(int q, int& a, int& b) {
    if constexpr (q4_bf16<FMT, T>()) {
        a = ((q & 2) ? 1 : 0) + ((q & 1) ? 4 : 0);
        b = a + 2;
    } else if constexpr (is_q4<FMT>()) {
        a = q;
        b = q + 4;
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
        a = 4 * (q / 2) + q % 2;
        b = a + 2;
    } else {
        a = 2 * q;
        b = a + 1;
    }
}

// The 8 weights of MFMA k-slice s of a swapped quad as packed pairs: dword s
// (int4), dwords 2s, 2s+1 (int8), the whole quad chunk (dense).
template <int FMT, typename T> __device__ __forceinline__ u32x4 unpack_slice(u32x4 v, int s) {
    if constexpr (FMT == LSSM_W_DENSE) {
        return v;
    } else if constexpr (FMT == LSSM_W_Q8_G32) {
        const Unpacked<FMT, T> u = unpack<FMT, T>(make_uint4(v[2 * s], v[2 * s + 1], 0u, 0u));
        return u32x4{u.p[0], u.p[1], u.p[2], u.p[3]};
    } else {
        const Unpacked<FMT, T> u = unpack<FMT, T>(make_uint4(v[s], 0u, 0u, 0u));
        return u32x4{u.p[0], u.p[1], u.p[2], u.p[3]};
    }
}

template <typename T> __device__ __forceinline__ floatx4 mfma16(u32x4 a, u32x4 b, floatx4 c) {
    if constexpr (__is_same(T, bf16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// ra: dwords of the LDS region that holds, in turn, the lanes' sums of
// squares, the staged x rows and each pass's partial sums.
template <int FMT, typename T, int CT, int QPW, bool NORM, bool PACKED, class Epi>
__global__ __launch_bounds__(64 * mma_waves(CT, QPW)) void gemv_mma_kernel(GemvCore c, Epi epi, uint32_t M, uint32_t mpb,
                                                                 uint32_t ra) {
    using P = Mma<FMT, T>;
    using F = Fmt<FMT, T>;
    constexpr int NP = P::NP, GPQ = P::GPQ, SPG = P::SPG;
    constexpr bool BIAS = P::BIAS;
    extern __shared__ __attribute__((aligned(16))) uint32_t mm_lds[];
    __shared__ float rinv_s[16];

    const uint32_t K = c.K, N = c.N;
    const int lane = threadIdx.x % WAVE, li = lane % 16, lq = lane / 16;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int KS = blockDim.x / WAVE;
    const uint32_t RS = K / 2 + 4;                             // x row pitch (dwords)
    const uint32_t KO = K / 8;                                 // octets per row
    const uint32_t SEG = (KO + 63) / 64;                       // 64-octet segments per row
    // segment u -> (row u / SEG, place u % SEG) by one multiply-high: exact
    // for u, SEG < 2^16 with ceil(2^32 / SEG) (a division per segment costs
    // ~15 scalar instructions, and the staging is issue-bound)
    const uint32_t seg_magic = SEG == 1 ? 0u : 0xFFFFFFFFu / SEG + 1u;
    auto seg_row = [&](uint32_t u) -> uint32_t { return SEG == 1 ? u : __umulhi(u, seg_magic); };
    auto seg_at = [&](uint32_t u) -> uint32_t { return u - seg_row(u) * SEG; };
    uint32_t* xl = mm_lds;
    const uint32_t tiles = (N + 15) / 16;
    const uint32_t tile0 = blockIdx.x * CT;
    // A block barrier that waits for this wave's LDS accesses only: the weight
    // loads in flight are not waited for (__syncthreads' release would).
    auto lds_barrier = [] {
        __builtin_amdgcn_s_waitcnt(0xC07F);                    // lgkmcnt(0)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // ---- x rows of one pass -> LDS ----
    // A pass stages mpb rows in segments of 64 octets (8 k each); wave w takes
    // segments w, w + KS, ... (at most MM_MAXJ), so a segment's row and place
    // are wave-uniform and a lane's octet is segment * 64 + lane.
    // KEEP: the x octets stay in registers between the sum of squares and
    // the normalisation (the first pass, before any weight is in registers);
    // later passes load them again (cache hits) to keep the registers free.
    u32x4 xk[MM_MAXJ], nk[MM_MAXJ];                            // the first pass's x octets
    auto stage = [&](uint32_t base, auto keep) {
        constexpr bool KEEP = decltype(keep)::value;
        const uint32_t nseg = mpb * SEG;
        // the lane index through an empty asm: the addresses below are
        // recomputed per pass instead of being kept live across the compute
        uint32_t lane = threadIdx.x % WAVE;
        asm volatile("" : "+v"(lane));
        auto load = [&](int j, u32x4& xv, u32x4& nv) {
            const uint32_t u = w + KS * j;
            const uint32_t m = min(base + seg_row(u), M - 1), cc = min(seg_at(u) * 64 + lane, KO - 1);
            xv = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(c.x) + (size_t)m * c.x_stride + 8 * cc);
            if constexpr (NORM) nv = reinterpret_cast<const u32x4*>(c.norm_w)[cc];
        };
        if constexpr (NORM) {
            // sum(x^2) per segment: each lane's share in LDS (region A, before
            // x lands there), then one wave per row sums it in a fixed order
            float* part = reinterpret_cast<float*>(mm_lds);    // [segment][lane]
            auto squares = [&](int j, const u32x4& d) {
                const uint32_t u = w + KS * j;
                float q = dot2(d[0], d[0], 0.0f, T{});
                q = dot2(d[1], d[1], q, T{});
                q = dot2(d[2], d[2], q, T{});
                q = dot2(d[3], d[3], q, T{});
                part[u * WAVE + lane] = seg_at(u) * 64 + lane < KO ? q : 0.0f;
            };
            if constexpr (KEEP) {
#pragma unroll
                for (int j = 0; j < MM_MAXJ; ++j)
                    if (w + KS * j < nseg) squares(j, xk[j]);
            } else {
                // rounds of MM_MAXJ / 2 segments (any number of them per wave)
                for (int j0 = 0; w + KS * j0 < nseg; j0 += MM_MAXJ / 2) {
                    u32x4 xv[MM_MAXJ / 2], dummy;
#pragma unroll
                    for (int jj = 0; jj < MM_MAXJ / 2; ++jj)
                        if (w + KS * (j0 + jj) < nseg) load(j0 + jj, xv[jj], dummy);
#pragma unroll
                    for (int jj = 0; jj < MM_MAXJ / 2; ++jj)
                        if (w + KS * (j0 + jj) < nseg) squares(j0 + jj, xv[jj]);
                }
            }
            lds_barrier();
            for (uint32_t r = w; r < mpb; r += KS) {
                float t = 0.0f;
                for (uint32_t g = 0; g < SEG; ++g) t += part[(r * SEG + g) * WAVE + lane];
                t = wave_sum(t);
                if (lane == 0) rinv_s[r] = 1.0f / sqrtf(t / (float)K + c.eps);
            }
            lds_barrier();
        }
        auto put = [&](int j, const u32x4& xv, const u32x4& nv, float rr) {
            const uint32_t u = w + KS * j;
            const uint32_t r = seg_row(u), cc = seg_at(u) * 64 + lane;
            const bool live = cc < KO;
            float v[8];
            if constexpr (NORM) {
                // x w is exact in fp32 (products of 8- or 11-bit significands), then * rr
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] = lo_f<T>(xv[e]) * lo_f<T>(nv[e]) * rr;
                    v[2 * e + 1] = hi_f<T>(xv[e]) * hi_f<T>(nv[e]) * rr;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] = f_of_bits<T>((uint16_t)(xv[e] & 0xFFFFu));
                    v[2 * e + 1] = f_of_bits<T>((uint16_t)(xv[e] >> 16));
                }
            }
            u32x4 pk;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                int pa, pb;
                octet_pos<FMT, T>(q, pa, pb);
                pk[q] = pack2<T>(v[pa], v[pb]);                         // the rounding r()
            }
            // the pairs of k .. k + 7 sit at dwords k / 2 .. k / 2 + 3 of the row
            if (live) *reinterpret_cast<u32x4*>(xl + r * RS + 4 * cc) = pk;
        };
        if constexpr (KEEP) {
            // the rows' 1 / rms first, all at once (one LDS wait, not one per segment)
            float rr[MM_MAXJ];
#pragma unroll
            for (int j = 0; j < MM_MAXJ; ++j) {
                rr[j] = 1.0f;
                if constexpr (NORM) {
                    if (w + KS * j < nseg) rr[j] = rinv_s[seg_row(w + KS * j)];
                }
            }
#pragma unroll
            for (int j = 0; j < MM_MAXJ; ++j)
                if (w + KS * j < nseg) put(j, xk[j], nk[j], rr[j]);
        } else {
            // rounds of MM_MAXJ / 2 segments (any number of them per wave)
            for (int j0 = 0; w + KS * j0 < nseg; j0 += MM_MAXJ / 2) {
                u32x4 xv[MM_MAXJ / 2], nv[MM_MAXJ / 2];
                float rr[MM_MAXJ / 2];
#pragma unroll
                for (int jj = 0; jj < MM_MAXJ / 2; ++jj) {
                    rr[jj] = 1.0f;
                    if (w + KS * (j0 + jj) < nseg) {
                        load(j0 + jj, xv[jj], nv[jj]);
                        if constexpr (NORM) rr[jj] = rinv_s[seg_row(w + KS * (j0 + jj))];
                    }
                }
#pragma unroll
                for (int jj = 0; jj < MM_MAXJ / 2; ++jj)
                    if (w + KS * (j0 + jj) < nseg) put(j0 + jj, xv[jj], nv[jj], rr[jj]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        lds_barrier();
    };

    // ---- x pre-packed by launch_mma_pack: rows [base, base + mpb) copied ----
    // (16-byte pieces p = row * KO + octet, eight in flight per thread)
    auto copy_in = [&](uint32_t base) {
        const uint32_t NT = blockDim.x, KH = K / 2;
        const uint32_t n = min(mpb, M - base) * KO;
        const uint32_t ko_magic = 0xFFFFFFFFu / KO + 1u;           // KO >= 16: exact for p < 2^16
        for (uint32_t p0 = threadIdx.x; p0 < n; p0 += 8 * NT) {
            u32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t p = p0 + i * NT;
                if (p < n) {
                    const uint32_t r = __umulhi(p, ko_magic), cc = p - r * KO;
                    v[i] = *reinterpret_cast<const u32x4*>(c.xp + (size_t)(base + r) * KH + 4 * cc);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t p = p0 + i * NT;
                if (p < n) {
                    const uint32_t r = __umulhi(p, ko_magic), cc = p - r * KO;
                    *reinterpret_cast<u32x4*>(xl + r * RS + 4 * cc) = v[i];
                }
            }
        }
        lds_barrier();
    };

    // ---- weights (and raw scale bits) of the wave's quads, all in flight ----
    // With few weight registers (CT * QPW <= 8) they are held over all
    // passes; otherwise a later pass reads them again (L2 hits) rather than
    // holding them across its staging.
    constexpr bool HOLD = CT * QPW <= 8;
    const size_t rb = F::row_bytes(K);
    u32x4 wr[CT][QPW];
    constexpr int SW = (QPW * GPQ + 1) / 2;                    // scale dwords per tile and wave
    uint32_t sr[CT][SW];
    auto load_w = [&] {
    #pragma unroll
        for (int t = 0; t < CT; ++t) {
            const uint32_t n = min(16 * (tile0 + t) + li, N - 1);
    #pragma unroll
            for (int qd = 0; qd < QPW; ++qd) {
                const uint32_t qa = w * QPW + qd;
                wr[t][qd] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(c.w + n * rb + 16 * (4 * qa + lq)));
            }
            if constexpr (P::G > 0) {
                // the wave's QPW * GPQ scales of the row, contiguous (the plan
                // keeps their offset a multiple of their size)
                const uint16_t* sp = c.s + n * (K / P::G) + w * QPW * GPQ;
                if constexpr (SW == 1) {
                    sr[t][0] = *reinterpret_cast<const uint32_t*>(sp);
                } else if constexpr (SW == 2) {
                    const uint2 v = *reinterpret_cast<const uint2*>(sp);
                    sr[t][0] = v.x;
                    sr[t][1] = v.y;
                } else {
#pragma unroll
                    for (int i = 0; i < SW / 4; ++i) {
                        const u32x4 v = *reinterpret_cast<const u32x4*>(sp + 8 * i);
#pragma unroll
                        for (int e = 0; e < 4; ++e) sr[t][4 * i + e] = v[e];
                    }
                }
            }
        }
    };
    epi.pin();
    // x of the first pass, staged before any weight is requested: requested
    // behind the weights, x would queue behind the whole chip's weight
    // traffic (measured: staging done ~7 us after the start instead of ~2)
    constexpr bool packed = PACKED;                            // x from launch_mma_pack (c.xp)
    const bool keep0 = !packed && mpb * SEG <= (uint32_t)(MM_MAXJ * KS);   // the first pass's x fits the registers
    if (keep0) {
        const uint32_t nseg = mpb * SEG;
        const uint32_t lane0 = threadIdx.x % WAVE;
        // KS a multiple of SEG: every segment of a wave sits at the same place
        // in its row, so the norm weight is loaded once
        const bool one_place = KS % SEG == 0;
#pragma unroll
        for (int j = 0; j < MM_MAXJ; ++j) {
            const uint32_t u = w + KS * j;
            if (u < nseg) {
                const uint32_t m = min(seg_row(u), M - 1), cc = min(seg_at(u) * 64 + lane0, KO - 1);
                xk[j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(c.x) + (size_t)m * c.x_stride + 8 * cc);
                if constexpr (NORM) {
                    if (j == 0 || !one_place) nk[j] = reinterpret_cast<const u32x4*>(c.norm_w)[cc];
                    else nk[j] = nk[0];
                }
            }
        }
    }
    if (packed) copy_in(0u);
    else if (keep0) stage(0u, FmtTag<1>{});
    else stage(0u, FmtTag<0>{});
    load_w();

    for (uint32_t base = 0; base < M; base += mpb) {
        if (base > 0) {
            if (packed) copy_in(base);
            else stage(base, FmtTag<0>{});
            if constexpr (!HOLD) load_w();
        }
        const uint32_t rows = min(mpb, M - base);
        // Epilogue: output element o of the block (tile o / 256, D element o %
        // 256 as lane * 4 + element) is finished by thread o % NT; its inputs
        // are requested now.  Element e of lane 16 q + i is batch row 4 q + e,
        // W row i of the tile.
        const uint32_t NT = blockDim.x;
        constexpr int EPT = (CT + 1) / 2;                       // elements per thread (the plan: 64 KS EPT >= 256 CT)
        typename Epi::Pre pre[EPT];
        auto out_mn = [&](uint32_t o, uint32_t& m, uint32_t& n) {
            const uint32_t t = o / 256, l = (o % 256) / 4, e = o % 4;
            m = base + 4 * (l / 16) + e;
            n = 16 * (tile0 + t) + l % 16;
        };
        // unconditional (clamped) and pinned ahead of the compute: a branch
        // around them, or their sinking to the epilogue, would expose their latency
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            uint32_t m, n;
            out_mn(min(threadIdx.x + NT * k, CT * 256u - 1), m, n);
            pre[k] = epi.prefetch((int)min(m, M - 1), min(n, N - 1));
        }
        __builtin_amdgcn_sched_barrier(0);
        floatx4 acc[CT];
#pragma unroll
        for (int t = 0; t < CT; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t xrow = min((uint32_t)li, mpb - 1) * RS;   // A rows past the pass: duplicates
#pragma unroll
        for (int qd = 0; qd < QPW; ++qd) {
            const uint32_t qa = w * QPW + qd;
            // the 4 lanes of each row trade dwords (one scale group per k-slice);
            // waits only for this quad's loads
            u32x4 wq[CT];
#pragma unroll
            for (int t = 0; t < CT; ++t) wq[t] = mma_swap<FMT>(wr[t][qd]);
#pragma unroll
            for (int g = 0; g < GPQ; ++g) {
                // x fragments of the group's MFMA k-slices (shared by the CT tiles)
                u32x4 xf[SPG];
#pragma unroll
                for (int e = 0; e < SPG; ++e) {
                    int ch, po;
                    mma_slice_pos<FMT>(g * SPG + e, lq, ch, po);
                    xf[e] = *reinterpret_cast<const u32x4*>(xl + xrow + (4 * qa + ch) * NP + po);
                }
                // int4 x bf16: sum(x) of the group's k per batch row, an MFMA
                // against ones (exact products), shared by the CT tiles
                floatx4 sxv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (BIAS) {
                    constexpr uint32_t ONE2 = 0x3F803F80u;             // bf16 (1, 1)
#pragma unroll
                    for (int e = 0; e < SPG; ++e) sxv = mfma16<T>(xf[e], u32x4{ONE2, ONE2, ONE2, ONE2}, sxv);
                }
#pragma unroll
                for (int t = 0; t < CT; ++t) {
                    // tile by tile: interleaving the tiles' unpacks runs out of registers
                    if (t > 0) __builtin_amdgcn_sched_barrier(0);
                    floatx4 d = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int e = 0; e < SPG; ++e) {
                        const int sl = g * SPG + e;
                        d = mfma16<T>(xf[e], unpack_slice<FMT, T>(wq[t], sl), P::G == 0 ? acc[t] : d);
                    }
                    if constexpr (P::G == 0) {
                        acc[t] = d;
                    } else {
                        const int h = qd * GPQ + g;                         // the scale's half-word
                        const uint32_t sw = sr[t][h / 2];
                        const float sc = fp16_bits_to_f((uint16_t)((h & 1) ? sw >> 16 : sw & 0xFFFFu));
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float dr = BIAS ? __builtin_fmaf(-136.0f, sxv[r], d[r]) : d[r];
                            acc[t][r] = __builtin_fmaf(sc, dr, acc[t][r]);
                        }
                    }
                }
            }
        }
        // ---- the KS partial sums of each tile, in wave order ----
        lds_barrier();                                         // x no longer read
        floatx4* red = reinterpret_cast<floatx4*>(mm_lds);      // [wave][tile][lane]
        const float* redf = reinterpret_cast<const float*>(mm_lds);
#pragma unroll
        for (int t = 0; t < CT; ++t) red[(w * CT + t) * WAVE + lane] = acc[t];
        lds_barrier();
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t o = threadIdx.x + NT * k;
            if (o < CT * 256u) {
                // the KS partial sums in wave order (deterministic)
                float v = 0.0f;
                for (int ww = 0; ww < KS; ++ww) v += redf[ww * CT * 256 + o];
                uint32_t m, n;
                out_mn(o, m, n);
                if (m - base < rows && n < N && o / 256 + tile0 < tiles) epi((int)m, n, v, pre[k]);
            }
        }
        lds_barrier();                                         // red read before the next staging
    }
}

// ---------------------------------------------------------------------------
// gemv_mmx: the gemv_mma product for x packed by launch_mma_pack, 2..32 rows
// in one pass (RT = 1 or 2 tiles of 16 batch rows), int4 group 64 x bf16
// (the 2.7B / 8B decode linears).  Nothing is staged: the A fragments are
// read straight from x packed in fragment order (launch_mma_pack, frag: at
// most 32 rows, which stay in L2; each load instruction reads 1 KiB of
// consecutive bytes, where the row-major rows would cost the vector L1 one
// access per lane), and every unpacked weight slice meets all RT row tiles.  A
// wave requests the x of its first XD quads (2 to 8, as registers allow),
// then all its weights and scales (one round trip to HBM per block), then,
// while it works through the quads, the x of the quad XD ahead.  (A wave's loads complete in the order
// they were issued: x requested behind the weights could not be used before
// every weight had arrived.)  The LDS holds only the KS partial sums, and a
// block owns up to three tiles of 16 W rows so that the grid is about one
// block per CU; where three would leave more blocks than CUs (the 8B
// in_proj: 1160 tiles), 8-wave blocks take five, keep one scale
// register per tile and, by default, run their quads through a ring of two
// (x and weights of two quads in flight).  Weights are read with ordinary
// loads: a load instruction reads 64 bytes of each of 16 rows, the other half
// of each 128-byte line is the next quad's, and nontemporal loads lost the
// line in between (8B in_proj at batch 32: 51.5 MB fetched from HBM against
// 44.5 MB, 19.4 against 16.1 us).  Per wave, the k-slices and the group scaling are
// gemv_mma_kernel's and the partials are summed in wave order; the K split
// (at most 8 waves here) can differ from that kernel's, so the two may round
// the fp32 sum of an output differently.
// With NX, x holds r(x w) without the rows' 1 / rms (written so by the kernel
// before, with partial sums of squares of x: the out_proj epilogue EpiResFrag,
// the SSD step, or launch_mma_pack with part); the block adds each row's
// partials in a fixed order and scales its fp32 sums by 1 / rms in the
// epilogue, where the reference scales x before rounding it (the same one
// rounding of each input, at another point).
// ---------------------------------------------------------------------------
constexpr int MMX_MAXW = 8;                      // waves per block: the K split

// NX: the rows' partial sums of squares are read by 16 lanes a row, 16 x 4
// floats a step (at most this many partials a row)
constexpr uint32_t MMX_MAXPARTS = GEMV_MAX_XPARTS;
static_assert(MMX_MAXPARTS % 64 == 0, "16 lanes x float4 per step");

// Epilogue h = r(res + r(acc)) (res may be y) that also writes r(h nw) in
// fragment order for the next single-pass GEMV (nw: the norm weight of the
// RMSNorm in front of it) and returns h^2: the kernel adds each row's 16
// values of a tile and hands the sum to put_part.
template <typename T> struct EpiResFrag {
    static constexpr bool kParts = true;
    T* y;
    uint32_t y_stride;
    const T* res;
    T* frag;
    float* part;
    const T* nw;
    uint32_t quads, nparts;                    // of the next GEMV's x (K = N here)
    struct Pre {
        uint32_t r, w;
    };
    __device__ __forceinline__ void pin() const {
        pin_arg(y);
        pin_arg(y_stride);
        pin_arg(res);
        pin_arg(frag);
        pin_arg(part);
        pin_arg(nw);
        pin_arg(quads);
        pin_arg(nparts);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const {
        return Pre{raw_at(res + ((uint32_t)m * y_stride + n)), raw_at(nw + n)};
    }
    __device__ __forceinline__ float store(uint32_t m, uint32_t n, float acc, const Pre& p) const {
        const T h = from_f<T>(f_of_raw<T>(p.r) + rnd<T>(acc));
        const float v = to_f(h);
        y[(size_t)m * y_stride + n] = h;
        frag[frag_half(m, n, quads)] = from_f<T>(v * f_of_raw<T>(p.w));
        return v * v;
    }
    __device__ __forceinline__ void put_part(uint32_t m, uint32_t tile, float q) const {
        part[(size_t)m * nparts + tile] = q;
    }
};
// Engine decode at batch 2..16 (x packed with partial sums, the single-pass
// kernel): the in_proj rows of EpiInproj published as tagged words,
// xfer[m proj + n] = value bits | step tag << 32 (the batch-1 launch's
// scheme, gemv.hip), then the SSD step + SiLU(z) gate of the items (row m,
// 32 consecutive rows j = h P + p of the flattened (H, P)) blockIdx.x,
// blockIdx.x + grid, ... in the same launch, with ssd_step_kernel<FRAG>'s
// arithmetic and outputs (ssd_step.metal:33-77): y, r(y w) in out_proj's
// fragment order and the 32 values' sum of squares of y.  An item waits for
// its 2N + 65 words (B and C of the group, x and z of its rows, dt of the
// head), which other blocks of the launch store; the launcher takes grids of
// at most one block per CU, so every block is resident and every awaited word
// gets written.  The wait is bounded all the same: an item whose words do not
// all arrive leaves its state as it was, writes NaN and sets
// STATUS_WAIT_TIMEOUT in the context's status word.
template <typename T> struct EpiInprojSsdB {
    static constexpr bool kTail = true;
    static constexpr uint32_t IP = 32;                    // state rows per item
    static constexpr uint32_t NV = 8;                     // lanes per state row
    static constexpr uint32_t NN = 128;                   // d_state
    static constexpr int F = (int)(NN / (4 * NV));        // 16-byte state pieces per lane
    static constexpr uint32_t NWD = 2 * NN + 2 * IP + 1;  // words an item reads
    static constexpr uint32_t SPIN = 1u << 16;            // polls before giving up
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    EpiInproj<T> in;                                      // routing / conv (its z, xbc_act, dt unused)
    uint64_t* xfer;                                       // [M][proj] tagged words of this layer
    uint32_t proj;
    const uint32_t* seq;                                  // the step tag (device)
    float* state;                                         // [M][H][P][NN] of this layer
    const T* A_log;
    const T* dt_bias;
    const T* D;                                           // nullptr: no D term
    T* y;                                                 // [M][d_inner]
    T* yfrag;                                             // r(y w), out_proj's fragment order
    float* ypart;                                         // [M][H P / IP] sums of y^2
    const T* ynorm_w;                                     // out_proj's norm weight
    uint32_t P, G, M;
    float dt_min, dt_max;
    uint32_t* status;
    uint32_t wait_skew;                                   // 0; 1 = wait for a tag nobody publishes
    using Pre = typename EpiInproj<T>::Pre;
    __device__ __forceinline__ void pin() const {
        in.pin();
        pin_arg(xfer);
        pin_arg(proj);
        pin_arg(seq);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const { return in.prefetch(m, n); }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const T v = in.value(m, n, acc, p);
        const uint64_t word = (uint64_t)bits16(v) | ((uint64_t)*seq << 32);
        __hip_atomic_store(xfer + (size_t)m * proj + n, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    static constexpr int GI = 4;                          // items a block takes at once
    // The state slice of item `it` (every thread loads: threads past the
    // item's 256 take row 0's, unused)
    __device__ __forceinline__ void load_state(uint32_t it, f32x4 (&s)[F]) const {
        const uint32_t H = in.H, ipr = H * P / IP, b = it / ipr, j0 = (it % ipr) * IP;
        const uint32_t t = threadIdx.x, pl = t < IP * NV ? t / NV : 0, j = j0 + pl;
        const f32x4* S = reinterpret_cast<const f32x4*>(state + (((size_t)b * H + j / P) * P + j % P) * NN);
#pragma unroll
        for (int f = 0; f < F; ++f) s[f] = __builtin_nontemporal_load(&S[t % NV + NV * f]);   // streamed once
    }
    // Word u of item `it`'s NWD words: its index in the row's projection.
    __device__ __forceinline__ uint32_t word_idx(uint32_t it, uint32_t u) const {
        const uint32_t d_inner = in.d_inner, H = in.H, GN = G * NN;
        const uint32_t ipr = H * P / IP, j0 = (it % ipr) * IP, h = j0 / P, g = h / (H / G);
        if (u < NN) return 2 * d_inner + g * NN + u;                                  // B
        if (u < 2 * NN) return 2 * d_inner + GN + g * NN + (u - NN);                  // C
        if (u < 2 * NN + IP) return d_inner + j0 + (u - 2 * NN);                      // x
        if (u < 2 * NN + 2 * IP) return j0 + (u - 2 * NN - IP);                       // z
        return d_inner + in.xbc + h;                                                  // dt
    }
    // The step of item `it` (slot d of the group) from its state slice and
    // its words in wv[d]; q: this thread's share of the 32 rows' sum of y^2.
    __device__ __forceinline__ float step(uint32_t it, const f32x4 (&s)[F], const uint32_t* wv,
                                          bool timed_out) const {
        const uint32_t d_inner = in.d_inner, H = in.H;
        const uint32_t ipr = H * P / IP, b = it / ipr, j0 = (it % ipr) * IP, h = j0 / P;
        const uint32_t t = threadIdx.x, lr = t % NV, pl = t / NV, j = j0 + pl, p = j % P;
        f32x4* S = reinterpret_cast<f32x4*>(state + (((size_t)b * H + h) * P + p) * NN);
        const float xv = f_of_raw<T>(wv[2 * NN + pl]);
        const float A_h = -expf(f_of_raw<T>(raw_at(A_log + h)));
        float dt = softplus_f(f_of_raw<T>(wv[2 * NN + 2 * IP]) + f_of_raw<T>(raw_at(dt_bias + h)));
        dt = fminf(fmaxf(dt, dt_min), dt_max);
        const float decay = expf(A_h * dt);
        float ys = 0.0f;
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const uint32_t n0 = 4 * (lr + NV * f);
            const float b0 = f_of_raw<T>(wv[n0]), b1 = f_of_raw<T>(wv[n0 + 1]);
            const float b2 = f_of_raw<T>(wv[n0 + 2]), b3 = f_of_raw<T>(wv[n0 + 3]);
            const float c0 = f_of_raw<T>(wv[NN + n0]), c1 = f_of_raw<T>(wv[NN + n0 + 1]);
            const float c2 = f_of_raw<T>(wv[NN + n0 + 2]), c3 = f_of_raw<T>(wv[NN + n0 + 3]);
            // the same fused multiply-adds as ssd_step_kernel
            f32x4 tt = s[f];
            tt.x = fmaf(decay, tt.x, dt * b0 * xv);
            tt.y = fmaf(decay, tt.y, dt * b1 * xv);
            tt.z = fmaf(decay, tt.z, dt * b2 * xv);
            tt.w = fmaf(decay, tt.w, dt * b3 * xv);
            if (!timed_out) __builtin_nontemporal_store(tt, &S[lr + NV * f]);
            ys += fmaf(c3, tt.w, fmaf(c2, tt.z, fmaf(c0, tt.x, c1 * tt.y)));
        }
        ys = group_sum<NV>(ys);
        float q = 0.0f;
        if (lr == 0) {
            const float dv = D ? f_of_raw<T>(raw_at(D + h)) : 0.0f;
            float yv = rnd<T>(fmaf(dv, xv, ys));
            yv = silu_fast(f_of_raw<T>(wv[2 * NN + IP + pl])) * yv;
            const T yr = from_f<T>(yv);
            y[(size_t)b * d_inner + j] = yr;
            const float yf = to_f(yr);
            yfrag[frag_half(b, j, H * P / 128)] = from_f<T>(yf * f_of_raw<T>(raw_at(ynorm_w + j)));
            q = yf * yf;
        }
        // the wave's 8 rows (lanes 8 i)
        q += __shfl_xor(q, 8);
        q += __shfl_xor(q, 16);
        q += __shfl_xor(q, 32);
        return q;
    }
    __device__ __forceinline__ uint32_t mine() const {
        const uint32_t items = M * (in.H * P / IP), gs = gridDim.x;
        return blockIdx.x < items ? (items - blockIdx.x + gs - 1) / gs : 0u;
    }
    // Items k0 .. k0 + GI - 1 of the block (b + k grid), state in st: all
    // their words awaited together (one round trip to the other workgroups'
    // stores per group, not per item), then the steps.  Threads 256..
    // (blocks of more than four waves) take part in the waits and barriers only.
    __device__ __forceinline__ void group(uint32_t k0, uint32_t n, const f32x4 (&st)[GI][F], uint32_t tag) const {
        __shared__ uint32_t wv[GI][NWD];                  // B, C, x, z, dt value bits
        __shared__ float red[GI][4];
        constexpr uint32_t QNAN = __is_same(T, f16) ? 0x7E00u : 0x7FC0u;
        const uint32_t ipr = in.H * P / IP, gs = gridDim.x, t = threadIdx.x;
        __syncthreads();                                  // the previous group's words and sums read
        int late = 0;                                     // a word of this thread never arrived
        for (uint32_t v = t; v < n * NWD; v += blockDim.x) {
            const uint32_t d = v / NWD, u = v % NWD, it = blockIdx.x + (k0 + d) * gs;
            const uint64_t* wp = xfer + (size_t)(it / ipr) * proj + word_idx(it, u);
            uint64_t w = __hip_atomic_load(wp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (uint32_t c = 0; (uint32_t)(w >> 32) != tag && c < SPIN; ++c)
                w = __hip_atomic_load(wp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            late |= (uint32_t)(w >> 32) != tag;
            wv[d][u] = (uint32_t)(w >> 32) == tag ? (uint32_t)w : QNAN;
        }
        // the state slices are stored only when every word of the group arrived
        const bool timed_out = __syncthreads_or(late) != 0;
        if (timed_out && t == 0) atomicOr(status, STATUS_WAIT_TIMEOUT);
#pragma unroll
        for (int d = 0; d < GI; ++d) {
            if ((uint32_t)d < n && t < IP * NV) {
                const float q = step(blockIdx.x + (k0 + d) * gs, st[d], wv[d], timed_out);
                if (t % WAVE == 0) red[d][t / WAVE] = q;
            }
        }
        __syncthreads();
        // the 4 waves' sums of each item in order (ssd_step_kernel's)
        if (t < n) {
            const uint32_t it = blockIdx.x + (k0 + t) * gs;
            ypart[(size_t)(it / ipr) * ipr + it % ipr] = red[t][0] + red[t][1] + red[t][2] + red[t][3];
        }
    }
    // The block's items b, b + grid, ... in groups of GI, each group's state
    // slices requested before its words are awaited.
    __device__ __forceinline__ void tail() const {
        const uint32_t tag = *seq + wait_skew, n = mine(), gs = gridDim.x;
        for (uint32_t k0 = 0; k0 < n; k0 += GI) {
            const uint32_t c = min((uint32_t)GI, n - k0);
            f32x4 st[GI][F];
#pragma unroll
            for (int d = 0; d < GI; ++d)
                if ((uint32_t)d < c) load_state(blockIdx.x + (k0 + d) * gs, st[d]);
            group(k0, c, st, tag);
        }
    }
};
template <class E, class = void> struct epi_tail {
    static constexpr bool value = false;
};
template <class E> struct epi_tail<E, decltype((void)E::kTail)> {
    static constexpr bool value = E::kTail;
};

template <class E, class = void> struct epi_parts {
    static constexpr bool value = false;
};
template <class E> struct epi_parts<E, decltype((void)E::kParts)> {
    static constexpr bool value = E::kParts;
};

template <int FMT, typename T, int CT, int RT, int QPW, int DR, bool NX, class Epi>
__global__ __launch_bounds__(64 * MMX_MAXW) void gemv_mmx_kernel(GemvCore c, Epi epi, uint32_t M) {
    using P = Mma<FMT, T>;
    using F = Fmt<FMT, T>;
    constexpr int GPQ = P::GPQ, SPG = P::SPG, SPQ = P::SPQ;
    constexpr bool BIAS = P::BIAS;
    static_assert(P::G > 0 && GPQ == 2, "int4 group 64");
    extern __shared__ __attribute__((aligned(16))) uint32_t mm_lds[];

    const uint32_t K = c.K, N = c.N;
    const int lane = threadIdx.x % WAVE, li = lane % 16, lq = lane / 16;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const uint32_t KS = blockDim.x / WAVE;
    const uint32_t qa0 = w * QPW;
    const uint32_t tiles = (N + 15) / 16, tile0 = blockIdx.x * CT;
    const size_t rb = F::row_bytes(K);
    epi.pin();

    // x in fragment order (launch_mma_pack, frag): the 16 bytes lane l supplies
    // to k-slice s of quad qa for row tile rt at u32x4 ((rt quads + qa) SPQ + s) 64 + l,
    // so each of these loads reads 1 KiB of consecutive bytes
    const u32x4* xf = reinterpret_cast<const u32x4*>(c.xp);
    const uint32_t quads = K / P::QK;

    // NX (x = r(x_raw w), not scaled by the rows' 1 / rms): the block's
    // rows' partial sums of squares of x_raw (16 lanes a row, NT / 16 rows a
    // pass, two passes at most) are requested before anything else, reduced
    // once the x and weight requests are out (loads return in issue order),
    // and the rows' 1 / rms left in LDS behind the epilogue's partial-sum
    // area, where the epilogue (after its barrier) scales the sums by them
    constexpr uint32_t NPV = MMX_MAXPARTS / 64;                // float4 per lane and row
    [[maybe_unused]] floatx4 pv[2][NPV];
    const uint32_t NT0 = blockDim.x;
    [[maybe_unused]] float* rrl = reinterpret_cast<float*>(mm_lds + KS * RT * CT * WAVE * 4);
    if constexpr (NX) {
        const uint32_t np = c.nparts, rpp = NT0 / 16;          // rows per pass
        const uint32_t r0 = threadIdx.x / 16, l16 = threadIdx.x % 16;
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            const uint32_t r = min(r0 + ps * rpp, (uint32_t)(16 * RT) - 1);
            const floatx4* pr = reinterpret_cast<const floatx4*>(c.part + (size_t)r * np);
#pragma unroll
            for (uint32_t j = 0; j < NPV; ++j) {
                const uint32_t f = l16 + 16 * j;               // float4 index in the row
                pv[ps][j] = 4 * f < np ? pr[f] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
    // x of XD quads in flight (a ring): as many as the registers left by the
    // weights and sums allow, at least two
    constexpr int XD = CT == 1 ? (QPW < (RT == 2 ? 4 : 8) ? QPW : (RT == 2 ? 4 : 8))
                               : (CT == 2 ? (QPW < 3 ? QPW : 3) : (QPW < 2 ? QPW : 2));
    u32x4 xr[XD][RT][SPQ];
    auto load_x = [&](int qd, u32x4 (&xb)[RT][SPQ]) {
        const uint32_t qa = qa0 + qd;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int sl = 0; sl < SPQ; ++sl) xb[rt][sl] = xf[(((size_t)rt * quads + qa) * SPQ + sl) * WAVE + lane];
    };
    // DR > 0: x and weights of DR quads in flight (a ring of quads), so that
    // the products of a quad overlap the loads of the ones after it
    constexpr bool RING = DR > 0;
    if constexpr (!RING) {
#pragma unroll
        for (int qd = 0; qd < XD; ++qd) load_x(qd, xr[qd]);
    }
    // all weights and scales of the wave's quads.  Blocks of more than three
    // tiles (four quads a wave) keep one scale register per tile: lane group
    // q holds its row's scales of quad q, handed to the other lanes as needed.
    constexpr bool SQ = CT > 3;
    static_assert(!SQ || QPW == 4, "one quad per lane group");
    constexpr int SR = SQ ? 1 : QPW;
    // Requested quad by quad (all tiles of a quad together), so that the
    // first quads' products start while the later weights are on their way.
    u32x4 wr[QPW][CT];
    uint32_t sr[SR][CT];                                       // the quad's two group scales
    const uint8_t* wp[CT];
    const uint32_t* sp[CT];
#pragma unroll
    for (int t = 0; t < CT; ++t) {
        const uint32_t n = min(16 * (tile0 + t) + li, N - 1);
        wp[t] = c.w + n * rb + 16 * lq + 64 * qa0;
        sp[t] = reinterpret_cast<const uint32_t*>(c.s + (size_t)n * (K / P::G)) + qa0;
        if constexpr (SQ) sr[0][t] = sp[t][lq];
    }
    static_assert(!RING || SQ, "the ring keeps the scales of all quads");
    constexpr int NR = RING ? DR : 1;
    u32x4 xg[NR][RT][SPQ], wg[NR][CT];
    auto load_q = [&](int qd, int slot) {
        load_x(qd, xg[slot]);
#pragma unroll
        for (int t = 0; t < CT; ++t)
            wg[slot][t] = *reinterpret_cast<const u32x4*>(wp[t] + 64 * qd);
    };
    if constexpr (RING) {
#pragma unroll
        for (int qd = 0; qd < DR; ++qd) load_q(qd, qd);
    } else {
#pragma unroll
        for (int qd = 0; qd < QPW; ++qd)
#pragma unroll
            for (int t = 0; t < CT; ++t) {
                wr[qd][t] = *reinterpret_cast<const u32x4*>(wp[t] + 64 * qd);
                if constexpr (!SQ) sr[qd][t] = sp[t][qd];
            }
    }

    if constexpr (NX) {
        const uint32_t rpp = NT0 / 16, r0 = threadIdx.x / 16;
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            // the row's partials in order within each lane, then over the 16
            // lanes by a fixed butterfly
            float t = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < NPV; ++j) t = t + pv[ps][j][0] + pv[ps][j][1] + pv[ps][j][2] + pv[ps][j][3];
            t += __shfl_xor(t, 8);
            t += __shfl_xor(t, 4);
            t += __shfl_xor(t, 2);
            t += __shfl_xor(t, 1);
            const uint32_t r = r0 + ps * rpp;
            if (threadIdx.x % 16 == 0 && r < 16u * RT) rrl[r] = 1.0f / sqrtf(t / (float)K + c.eps);
        }
    }

    floatx4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < CT; ++t) acc[rt][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_q = [&](const u32x4 (&wb)[CT], const uint32_t (&sb)[CT], const u32x4 (&xb)[RT][SPQ]) {
        // the 4 lanes of each row trade dwords (one scale group per k-slice)
        u32x4 wq[CT];
#pragma unroll
        for (int t = 0; t < CT; ++t) wq[t] = mma_swap<FMT>(wb[t]);
#pragma unroll
        for (int g = 0; g < GPQ; ++g) {
            // int4 x bf16: sum(x) of the group's k per batch row (exact)
            floatx4 sxv[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                sxv[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (BIAS) {
                    constexpr uint32_t ONE2 = 0x3F803F80u;             // bf16 (1, 1)
#pragma unroll
                    for (int e = 0; e < SPG; ++e)
                        sxv[rt] = mfma16<T>(xb[rt][g * SPG + e], u32x4{ONE2, ONE2, ONE2, ONE2}, sxv[rt]);
                }
            }
#pragma unroll
            for (int t = 0; t < CT; ++t) {
                if (t > 0) __builtin_amdgcn_sched_barrier(0);
                u32x4 u[SPG];
#pragma unroll
                for (int e = 0; e < SPG; ++e) u[e] = unpack_slice<FMT, T>(wq[t], g * SPG + e);
                const float sc = fp16_bits_to_f((uint16_t)(g ? sb[t] >> 16 : sb[t] & 0xFFFFu));
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    floatx4 d = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int e = 0; e < SPG; ++e) d = mfma16<T>(xb[rt][g * SPG + e], u[e], d);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float dr = BIAS ? __builtin_fmaf(-136.0f, sxv[rt][r], d[r]) : d[r];
                        acc[rt][t][r] = __builtin_fmaf(sc, dr, acc[rt][t][r]);
                    }
                }
            }
        }
    };

    // the epilogue's inputs, behind the weights (used after the sums)
    const uint32_t NT = blockDim.x;
    constexpr uint32_t NO = RT * CT * 256;                     // output elements of the block
    constexpr uint32_t NTMIN = CT > 3 ? 64 * 8 : 64 * 4;       // blocks of > 3 tiles have 8 waves
    constexpr int EPT = (NO + NTMIN - 1) / NTMIN;              // per thread
    typename Epi::Pre pre[EPT];
    auto out_mn = [&](uint32_t o, uint32_t& m, uint32_t& n) {
        const uint32_t rt = o / (CT * 256), t = (o / 256) % CT, l = (o % 256) / 4, e = o % 4;
        m = 16 * rt + 4 * (l / 16) + e;
        n = 16 * (tile0 + t) + l % 16;
    };
    auto prefetch = [&] {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            uint32_t m, n;
            out_mn(min(threadIdx.x + NT * k, NO - 1), m, n);
            pre[k] = epi.prefetch((int)min(m, M - 1), min(n, N - 1));
        }
    };
    // (blocks of more than three tiles have no registers to spare for them
    // during the sums: their epilogue inputs are requested behind the last quad)
    if constexpr (!SQ) prefetch();
#pragma unroll
    for (int qd = 0; qd < QPW; ++qd) {
        if constexpr (SQ) {
            uint32_t sb[CT];
#pragma unroll
            for (int t = 0; t < CT; ++t) sb[t] = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (16 * qd + li), (int)sr[0][t]);
            if constexpr (RING) {
                compute_q(wg[qd % DR], sb, xg[qd % DR]);
                if (qd + DR < QPW) load_q(qd + DR, qd % DR);
                continue;
            }
            compute_q(wr[qd], sb, xr[qd % XD]);
        } else {
            compute_q(wr[qd], sr[qd], xr[qd % XD]);
        }
        if (qd + XD < QPW) load_x(qd + XD, xr[qd % XD]);
    }

    if constexpr (SQ) prefetch();

    // ---- the KS partial sums of each output element, in wave order ----
    floatx4* red = reinterpret_cast<floatx4*>(mm_lds);          // [wave][row tile][tile][lane]
    const float* redf = reinterpret_cast<const float*>(mm_lds);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < CT; ++t) red[((w * RT + rt) * CT + t) * WAVE + lane] = acc[rt][t];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const uint32_t o = threadIdx.x + NT * k;
        if (o < NO) {                                          // whole waves (NT, NO multiples of 64)
            float v = 0.0f;
            for (uint32_t ww = 0; ww < KS; ++ww) v += redf[ww * NO + o];
            uint32_t m, n;
            out_mn(o, m, n);
            if constexpr (NX) v *= rrl[m];
            const uint32_t tl = o / 256 % CT + tile0;
            if constexpr (epi_parts<Epi>::value) {
                float q = 0.0f;
                if (m < M && n < N && tl < tiles) q = epi.store(m, n, v, pre[k]);
                // a wave holds 4 rows (lane % 4) x the tile's 16 columns
                // (lane / 4 % 16): the row sums by a fixed butterfly
                q += __shfl_xor(q, 4);
                q += __shfl_xor(q, 8);
                q += __shfl_xor(q, 16);
                q += __shfl_xor(q, 32);
                if (lane < 4 && tl < tiles) epi.put_part(m, tl, q);
            } else {
                if (m < M && n < N && tl < tiles) epi((int)m, n, v, pre[k]);
            }
        }
    }
    if constexpr (epi_tail<Epi>::value) epi.tail();
}

// LSSM_MMA_STAGED=1 (read once) keeps packed x on the staging kernel, for A/B
// measurements.
inline bool mmx_disabled() {
    static const bool off = [] {
        const char* v = getenv("LSSM_MMA_STAGED");
        return v && v[0] == '1';
    }();
    return off;
}

inline bool mmx_wide() {
    static const bool on = [] {
        const char* v = getenv("LSSM_MMX_WIDE");
        return !v || v[0] != '0';
    }();
    return on;
}

// ---- gemv_mmx launch plan: int4 group 64 x bf16; K split into KS (4..8)
// waves of QPW (4, 5 or 8) quads; tiles per block from {1, 2, 3} so the
// blocks cover the CUs about once ----
struct MmxPlan {
    uint32_t ct = 0, rt = 0, ks = 0, qpw = 0;
    size_t lds = 0;
};

template <int FMT, typename T> bool mmx_plan(uint32_t M, uint32_t N, uint32_t K, MmxPlan& p) {
    using P = Mma<FMT, T>;
    if constexpr (FMT != LSSM_W_Q4_G64 || !__is_same(T, bf16)) {
        return false;
    } else {
        if (M < 2 || M > 32 || N == 0 || K % P::QK != 0) return false;
        const uint32_t quads = K / P::QK;
        uint32_t ks = 0, qpw = 0;
        for (uint32_t q : {4u, 5u, 8u})
            if (ks == 0 && quads % q == 0 && quads / q >= 4 && quads / q <= (uint32_t)MMX_MAXW) {
                qpw = q;
                ks = quads / q;
            }
        if (ks == 0) return false;
        const uint32_t tiles = (N + 15) / 16, cus = num_cus();
        const uint32_t want = (tiles + cus - 1) / cus;
        p.ct = want <= 1 ? 1 : (want == 2 ? 2 : 3);
        // 5 tiles (the 8B in_proj): built for 8 waves of 4 quads
        if (want > 3 && qpw == 4 && ks == (uint32_t)MMX_MAXW && mmx_wide()) p.ct = 5;
        p.rt = M > 16 ? 2 : 1;
        p.ks = ks;
        p.qpw = qpw;
        p.lds = (size_t)ks * p.rt * p.ct * WAVE * 16;
        return p.lds <= MM_LDS_MAX;
    }
}

template <int FMT, typename T, int CT, int RT, int QPW, class Epi, int DR = 0>
hipError_t mmx_run(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmxPlan& p) {
    auto go = [&](auto k, size_t lds) -> hipError_t {
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)MM_LDS_MAX);
        if (attr != hipSuccess) return attr;
        if (lds > MM_LDS_MAX) return hipErrorInvalidValue;
        const uint32_t tiles = (c.N + 15) / 16;
        k<<<(tiles + CT - 1) / CT, WAVE * p.ks, lds, s>>>(c, e, M);
        return hipGetLastError();
    };
    if (c.part) {
        // x = r(x_raw w): 32 rows' 1 / rms behind the epilogue area
        if (c.nparts % 4 || c.nparts > MMX_MAXPARTS || (uintptr_t)c.part % 16) return hipErrorInvalidValue;
        return go(gemv_mmx_kernel<FMT, T, CT, RT, QPW, DR, true, Epi>, p.lds + 32 * sizeof(float));
    }
    return go(gemv_mmx_kernel<FMT, T, CT, RT, QPW, DR, false, Epi>, p.lds);
}

template <int FMT, typename T, int CT, int RT, class Epi>
hipError_t mmx_q(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmxPlan& p) {
    switch (p.qpw) {
        case 4: return mmx_run<FMT, T, CT, RT, 4, Epi>(s, c, e, M, p);
        case 5: return mmx_run<FMT, T, CT, RT, 5, Epi>(s, c, e, M, p);
        default: return mmx_run<FMT, T, CT, RT, 8, Epi>(s, c, e, M, p);
    }
}

// blocks of 5 tiles: quads in a ring of mmx_ring() (0: all weights up front)
inline int mmx_ring() {
    static const int r = [] {
        const char* v = getenv("LSSM_MMX_RING");
        return v ? (int)strtol(v, nullptr, 10) : 2;
    }();
    return r;
}

template <int FMT, typename T, int CT, int RT, class Epi>
hipError_t mmx_wide(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmxPlan& p) {
    switch (mmx_ring()) {
        case 0: return mmx_run<FMT, T, CT, RT, 4, Epi, 0>(s, c, e, M, p);
        default: return mmx_run<FMT, T, CT, RT, 4, Epi, 2>(s, c, e, M, p);
    }
}

template <int FMT, typename T, class Epi>
hipError_t mmx_go(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmxPlan& p) {
    if constexpr (FMT == LSSM_W_Q4_G64 && __is_same(T, bf16)) {
        if (p.rt == 1) {
            switch (p.ct) {
                case 1: return mmx_q<FMT, T, 1, 1, Epi>(s, c, e, M, p);
                case 2: return mmx_q<FMT, T, 2, 1, Epi>(s, c, e, M, p);
                case 3: return mmx_q<FMT, T, 3, 1, Epi>(s, c, e, M, p);
                default: return mmx_wide<FMT, T, 5, 1, Epi>(s, c, e, M, p);
            }
        }
        switch (p.ct) {
            case 1: return mmx_q<FMT, T, 1, 2, Epi>(s, c, e, M, p);
            case 2: return mmx_q<FMT, T, 2, 2, Epi>(s, c, e, M, p);
            case 3: return mmx_q<FMT, T, 3, 2, Epi>(s, c, e, M, p);
            default: return mmx_wide<FMT, T, 5, 2, Epi>(s, c, e, M, p);
        }
    } else {
        return hipErrorInvalidValue;
    }
}

// ---- gemv_mma launch plan ----
struct MmaPlan {
    uint32_t ct = 0, qpw = 0, ks = 0, mpb = 0, ra = 0;
    size_t lds = 0;
};

// Quads per wave from {1, 2, 4} (the smallest that splits K into <= 16 waves),
// tiles per block so that the blocks cover the CUs about once, rows per pass
// from the LDS budget and the staging registers (<= 8 octets per thread).
template <int FMT, typename T> bool mma_plan(uint32_t M, uint32_t N, uint32_t K, MmaPlan& p) {
    using P = Mma<FMT, T>;
    if (M < 2 || M > 64 || N == 0 || K % P::QK != 0) return false;
    const uint32_t quads = K / P::QK;
    constexpr bool q4 = FMT == LSSM_W_Q4_G64 || FMT == LSSM_W_Q4_B32;
    const uint32_t tiles = (N + 15) / 16, cus = num_cus();
    uint32_t want = (tiles + cus - 1) / cus;             // tiles per block: blocks ~ CUs
    want = want < 1 ? 1 : (want > 4 ? 4 : want);
    // the most tiles (up to want), then the fewest quads per wave, such that
    // the shape is built and its waves split K into whole quads
    for (uint32_t ct = want; ct >= 1 && p.qpw == 0; --ct) {
        for (uint32_t q : {1u, 2u, 4u, 8u}) {
            // every output element has a thread: 64 KS ((ct + 1) / 2) >= 256 ct
            if (mma_shape_ok((int)ct, (int)q, q4) && quads % q == 0 && (quads / q) * ((ct + 1) / 2) >= 4 * ct &&
                quads / q <= (uint32_t)mma_waves((int)ct, (int)q)) {
                p.qpw = q;
                p.ct = ct;
                break;
            }
        }
    }
    if (p.qpw == 0) return false;
    p.ks = quads / p.qpw;
    // a wave's scales are loaded as one vector: their offset in a row must be
    // a multiple of their count (P::GPQ * qpw half-words, at least 2)
    const uint32_t nsc = std::max<uint32_t>(P::GPQ * p.qpw, 2u);
    if (P::G > 0 && (K / P::G) % nsc != 0) return false;
    const size_t RS = K / 2 + 4;
    size_t fit = MM_LDS_MAX / (RS * 4);
    fit = fit < 16 ? fit : 16;
    if (fit < 1) return false;
    const uint32_t passes = (uint32_t)((M + fit - 1) / fit);
    p.mpb = (M + passes - 1) / passes;
    const size_t ra = std::max((size_t)p.mpb * RS, (size_t)p.ks * p.ct * WAVE * 4);
    p.ra = (uint32_t)ra;
    p.lds = ra * 4;
    return p.lds <= MM_LDS_MAX;
}

template <typename T> bool mma_aligned(const GemvCore& c, bool norm) {
    return (uintptr_t)c.x % 16 == 0 && ((size_t)c.x_stride * sizeof(T)) % 16 == 0 &&
           (!norm || (uintptr_t)c.norm_w % 16 == 0) && (uintptr_t)c.w % 16 == 0 && (uintptr_t)c.s % 16 == 0;
}

template <int FMT, typename T, int CT, int QPW, bool NORM, bool PACKED, class Epi>
hipError_t mma_run(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmaPlan& p) {
    auto k = gemv_mma_kernel<FMT, T, CT, QPW, NORM, PACKED, Epi>;
    // opt in to the dynamic LDS once per instantiation (a host attribute)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)MM_LDS_MAX);
    if (attr != hipSuccess) return attr;
    const uint32_t tiles = (c.N + 15) / 16;
    k<<<(tiles + CT - 1) / CT, WAVE * p.ks, p.lds, s>>>(c, e, M, p.mpb, p.ra);
    return hipGetLastError();
}

template <int FMT, typename T, bool NORM, bool PACKED, class Epi>
hipError_t mma_shape(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, const MmaPlan& p) {
    if (p.ct == 1) {
        switch (p.qpw) {
            case 1: return mma_run<FMT, T, 1, 1, NORM, PACKED, Epi>(s, c, e, M, p);
            case 2: return mma_run<FMT, T, 1, 2, NORM, PACKED, Epi>(s, c, e, M, p);
            case 4: return mma_run<FMT, T, 1, 4, NORM, PACKED, Epi>(s, c, e, M, p);
            default: return mma_run<FMT, T, 1, 8, NORM, PACKED, Epi>(s, c, e, M, p);
        }
    }
    if constexpr (FMT == LSSM_W_Q4_G64 || FMT == LSSM_W_Q4_B32) {
        if (p.qpw == 4) return mma_run<FMT, T, 4, 4, NORM, PACKED, Epi>(s, c, e, M, p);
        switch (p.ct) {
            case 2: return mma_run<FMT, T, 2, 2, NORM, PACKED, Epi>(s, c, e, M, p);
            case 3: return mma_run<FMT, T, 3, 2, NORM, PACKED, Epi>(s, c, e, M, p);
            default: return mma_run<FMT, T, 4, 2, NORM, PACKED, Epi>(s, c, e, M, p);
        }
    }
    return hipErrorInvalidValue;                       // not a planned shape
}

// Formats the MFMA decode kernel takes: int4 (both layouts) with fp16 / bf16,
// int8 and dense weights with fp16.
template <typename T, class F> bool mma_fmt(int wfmt, F&& f) {
    if constexpr (__is_same(T, float)) {
        return false;
    } else {
        switch (wfmt) {
            case LSSM_W_Q4_G64: return f(FmtTag<LSSM_W_Q4_G64>{});
            case LSSM_W_Q4_B32: return f(FmtTag<LSSM_W_Q4_B32>{});
            case LSSM_W_Q8_G32:
                if constexpr (__is_same(T, f16)) return f(FmtTag<LSSM_W_Q8_G32>{});
                else return false;
            case LSSM_W_DENSE:
                if constexpr (__is_same(T, f16)) return f(FmtTag<LSSM_W_DENSE>{});
                else return false;
            default: return false;
        }
    }
}

// Runs the MFMA decode kernel when it takes this call (returns false, and
// launches nothing, otherwise).
// Only RMSNorm-fused calls (the engine's decode linears and inproj_decode).
// Batches below this many rows go to the VALU GEMV (gemv1 takes up to 4):
// at 2 rows it is the faster of the two (2.7B decode at batch 2: 1470 against
// 1406 tok/s), at 3 and 4 the MFMA kernel (1953 / 2453 against 1170 / 1492).
// LSSM_MMA_MIN_ROWS=n overrides it, for A/B measurements.
inline uint32_t mma_min_rows() {
    static const uint32_t r = [] {
        const char* v = getenv("LSSM_MMA_MIN_ROWS");
        return v ? (uint32_t)strtoul(v, nullptr, 10) : 3u;
    }();
    return r;
}

template <typename T, class Epi>
bool try_mma(hipStream_t s, const GemvCore& c, const Epi& e, uint32_t M, int wfmt, bool norm, hipError_t& err) {
    if (!norm || M < mma_min_rows() || !mma_aligned<T>(c, norm)) return false;
    return mma_fmt<T>(wfmt, [&](auto tag) -> bool {
        constexpr int FMT = decltype(tag)::value;
        MmaPlan p;
        if (!mma_plan<FMT, T>(M, c.N, c.K, p)) return false;
        // packed x of up to 32 rows: one pass without staging
        MmxPlan q;
        if (c.xp && !mmx_disabled() && mmx_plan<FMT, T>(M, c.N, c.K, q)) {
            err = mmx_go<FMT, T, Epi>(s, c, e, M, q);
            return true;
        }
        if (c.part) {                                          // raw x: only the single-pass kernel
            err = hipErrorInvalidValue;
            return true;
        }
        err = c.xp ? mma_shape<FMT, T, true, true, Epi>(s, c, e, M, p)
                   : mma_shape<FMT, T, true, false, Epi>(s, c, e, M, p);
        return true;
    });
}

template <typename T> bool mma_takes(uint32_t M, uint32_t N, uint32_t K, int wfmt) {
    if (M < mma_min_rows()) return false;
    return mma_fmt<T>(wfmt, [&](auto tag) -> bool {
        MmaPlan p;
        return mma_plan<decltype(tag)::value, T>(M, N, K, p);
    });
}

// ---- x normalised and packed once for a whole gemv_mma launch ----
// Row m: rr = 1 / sqrt(mean(x^2) + eps), then each octet's r(x w rr) in the
// staging's pair order (norm.metal:52-79), stored as the staging would put it
// in LDS (pairs of k .. k + 7 at dwords k / 2 .. k / 2 + 3 of the row) or, with
// FRAG (int4 group 64 only), in gemv_mmx_kernel's fragment order: the 16 bytes
// lane l = 16 q + (m % 16) supplies to k-slice s of quad qa for row tile m / 16
// at u32x4 ((m / 16 quads + qa) 4 + s) 64 + l.  With FRAG the grid covers the
// rows up to the next multiple of 16, and rows past M are zeros.
template <int FMT, typename T, bool FRAG>
__global__ __launch_bounds__(1024) void mma_pack_kernel(const T* x, uint32_t x_stride, const T* nw, float eps,
                                                        uint32_t K, uint32_t M, uint32_t* out, float* part) {
    // one octet per thread (blockDim.x >= K / 8), x and w read once
    __shared__ float red[1024 / WAVE];
    const uint32_t m = blockIdx.x, KO = K / 8, cc = threadIdx.x;
    const bool live = cc < KO;
    const bool row = !FRAG || m < M;
    u32x4 xv = u32x4{0u, 0u, 0u, 0u}, nv = xv;
    if (live && row) {
        xv = reinterpret_cast<const u32x4*>(x + (size_t)m * x_stride)[cc];
        nv = reinterpret_cast<const u32x4*>(nw)[cc];
    }
    float q = dot2(xv[0], xv[0], 0.0f, T{});
    q = dot2(xv[1], xv[1], q, T{});
    q = dot2(xv[2], xv[2], q, T{});
    q = dot2(xv[3], xv[3], q, T{});
    // block sum in a fixed order: waves, then the wave sums in wave order
    q = wave_sum(q);
    const uint32_t nwv = blockDim.x / WAVE;
    if (threadIdx.x % WAVE == 0) red[threadIdx.x / WAVE] = q;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t i = 0; i < nwv; ++i) t += red[i];
    const float rr = 1.0f / sqrtf(t / (float)K + eps);
    // part: x w without 1 / rms, the sum of squares to part[4 m]
    const bool raw = FRAG && part != nullptr;
    if (raw && threadIdx.x < 4) part[4 * m + threadIdx.x] = threadIdx.x == 0 ? t : 0.0f;
    if (!live) return;
    const float sc = raw ? 1.0f : rr;
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = lo_f<T>(xv[e]) * lo_f<T>(nv[e]) * sc;
        v[2 * e + 1] = hi_f<T>(xv[e]) * hi_f<T>(nv[e]) * sc;
    }
    u32x4 pk;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        int pa, pb;
        octet_pos<FMT, T>(qq, pa, pb);
        pk[qq] = pack2<T>(v[pa], v[pb]);
    }
    if constexpr (FRAG) {
        // octet cc = 16 qa + 4 ch + p (chunk ch, pair offset 4 p of the quad):
        // k-slice s and lane group q with mma_slice_pos(s, q) = (ch, 4 p)
        const uint32_t qa = cc / 16, ch = (cc % 16) / 4, p4 = cc % 4;
        const uint32_t sl = 2 * (ch >> 1) + (p4 & 1), lg = (ch & 1) + 2 * (p4 >> 1);
        const uint32_t quads = K / 128;
        reinterpret_cast<u32x4*>(out)[(((size_t)(m / 16) * quads + qa) * 4 + sl) * WAVE + 16 * lg + m % 16] = pk;
    } else {
        reinterpret_cast<u32x4*>(out + (size_t)m * (K / 2))[cc] = pk;
    }
}

}  // namespace

hipError_t launch_mma_pack(hipStream_t s, const void* x, uint32_t x_stride, const void* norm_w, float eps,
                           uint32_t M, uint32_t K, int wfmt, int act, void* out, bool frag, float* part) {
    if (M == 0 || K % 128 != 0 || K > 8192 || (uintptr_t)x % 16 || (x_stride * 2u) % 16 ||
        (uintptr_t)norm_w % 16 || (uintptr_t)out % 16)
        return hipErrorInvalidValue;
    if (frag && (wfmt != LSSM_W_Q4_G64 || act != LSSM_BF16)) return hipErrorInvalidValue;
    if (part && !frag) return hipErrorInvalidValue;
    const uint32_t nt = (K / 8 + WAVE - 1) / WAVE * WAVE;      // one octet per thread
    if (frag) {
        mma_pack_kernel<LSSM_W_Q4_G64, bf16, true><<<(M + 15) / 16 * 16, nt, 0, s>>>(
            static_cast<const bf16*>(x), x_stride, static_cast<const bf16*>(norm_w), eps, K, M,
            static_cast<uint32_t*>(out), part);
        return hipGetLastError();
    }
    hipError_t err = hipErrorInvalidValue;
    auto go = [&](auto tag) -> bool {
        using T = decltype(tag);
        return mma_fmt<T>(wfmt, [&](auto ft) -> bool {
            constexpr int FMT = decltype(ft)::value;
            mma_pack_kernel<FMT, T, false><<<M, nt, 0, s>>>(static_cast<const T*>(x), x_stride,
                                                             static_cast<const T*>(norm_w), eps, K, M,
                                                             static_cast<uint32_t*>(out), nullptr);
            err = hipGetLastError();
            return true;
        });
    };
    if (act == LSSM_F16) go(f16{});
    else if (act == LSSM_BF16) go(bf16{});
    return err;
}

bool gemv_mmx_takes(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act) {
    if (act != LSSM_BF16 || wfmt != LSSM_W_Q4_G64 || mmx_disabled()) return false;
    MmxPlan p;
    return mmx_plan<LSSM_W_Q4_G64, bf16>(M, N, K, p);
}

uint32_t gemv_mmx_parts(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act) {
    if (act != LSSM_BF16 || wfmt != LSSM_W_Q4_G64 || mmx_disabled()) return 0;
    MmxPlan p;
    if (!mmx_plan<LSSM_W_Q4_G64, bf16>(M, N, K, p) || p.ct != 1) return 0;
    const uint32_t np = (N + 15) / 16;
    return N % 128 == 0 && np % 4 == 0 && np <= MMX_MAXPARTS ? np : 0;
}

bool gemv_mma_takes(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act) {
    if (act == LSSM_F16) return mma_takes<f16>(M, N, K, wfmt);
    if (act == LSSM_BF16) return mma_takes<bf16>(M, N, K, wfmt);
    return false;
}

bool launch_gemv_mma(hipStream_t s, const GemvArgs& a, hipError_t& err) {
    if (a.M < 2 && !a.yfrag) return false;
    GemvCore c{a.x, a.x_stride, (const uint8_t*)a.w, (const uint16_t*)a.s, a.norm_w, a.eps, a.N, a.K, 1.0f / (float)a.K};
    c.xp = static_cast<const uint32_t*>(a.xpack);
    c.part = a.xpart;
    c.nparts = a.nparts;
    if (a.yfrag) {
        // the rows also in fragment order with their partial sums of squares:
        // residual add, one tile a block (gemv_mmx_parts)
        const uint32_t np = gemv_mmx_parts(a.M, a.N, a.K, a.wfmt, a.act);
        MmxPlan p;
        err = hipErrorInvalidValue;
        if (np == 0 || a.epi != LSSM_EPI_ADD || !a.res || !a.ypart || !a.ynorm_w || !a.norm_w || !a.xpack ||
            (uintptr_t)a.yfrag % 16 || (uintptr_t)a.ypart % 16 ||
            !mmx_plan<LSSM_W_Q4_G64, bf16>(a.M, a.N, a.K, p) || !mma_aligned<bf16>(c, true))
            return true;
        EpiResFrag<bf16> e{(bf16*)a.y, a.y_stride, (const bf16*)a.res, (bf16*)a.yfrag, a.ypart,
                             (const bf16*)a.ynorm_w, a.N / 128, np};
        err = p.rt == 1 ? mmx_q<LSSM_W_Q4_G64, bf16, 1, 1, EpiResFrag<bf16>>(s, c, e, a.M, p)
                        : mmx_q<LSSM_W_Q4_G64, bf16, 1, 2, EpiResFrag<bf16>>(s, c, e, a.M, p);
        return true;
    }
    auto go = [&](auto tag) -> bool {
        using T = decltype(tag);
        EpiPlain<T> e{(T*)a.y, a.y_stride, (const T*)a.res, a.epi};
        return try_mma<T>(s, c, e, a.M, a.wfmt, a.norm_w != nullptr, err);
    };
    if (a.act == LSSM_F16) return go(f16{});
    if (a.act == LSSM_BF16) return go(bf16{});
    return false;
}

bool launch_inproj_ssd_decode_mma(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseBArgs& f,
                                  hipError_t& err) {
    const GemvArgs& g = a.g;
    if (g.act != LSSM_BF16 || g.wfmt != LSSM_W_Q4_G64 || !g.xpack || !g.xpart || !g.norm_w) return false;
    if (g.M < 2 || g.M > 16 || g.M < mma_min_rows() || mmx_disabled()) return false;
    if (f.N != 128 || f.P == 0 || f.P % 32 != 0 || f.G == 0 || a.H % f.G != 0 || (a.H * f.P) % 128 != 0 ||
        a.d_inner != a.H * f.P || a.xbc != a.d_inner + 2 * f.G * f.N || g.N != a.d_inner + a.xbc + a.H)
        return false;
    if (!f.xfer || !f.seq || !f.state || !f.y || !f.yfrag || !f.ypart || !f.ynorm_w || !f.status) return false;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K, 1.0f / (float)g.K};
    c.xp = static_cast<const uint32_t*>(g.xpack);
    c.part = g.xpart;
    c.nparts = g.nparts;
    if (!mma_aligned<bf16>(c, true)) return false;
    MmxPlan q;
    if (!mmx_plan<LSSM_W_Q4_G64, bf16>(g.M, g.N, g.K, q)) return false;
    // every block resident at once (one per CU at most), four waves an item
    const uint32_t blocks = ((g.N + 15) / 16 + q.ct - 1) / q.ct;
    if (blocks > num_cus() || q.ks * WAVE < 256) return false;
    using T = bf16;
    EpiInprojSsdB<T> e{EpiInproj<T>{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state, (const T*)a.conv_w,
                                    (const T*)a.conv_b, nullptr, nullptr, nullptr},
                       f.xfer, g.N, f.seq, f.state, (const T*)f.A_log, (const T*)f.dt_bias, (const T*)f.D,
                       (T*)f.y, (T*)f.yfrag, f.ypart, (const T*)f.ynorm_w, f.P, f.G, g.M, f.dt_min, f.dt_max,
                       f.status, f.wait_skew};
    err = mmx_go<LSSM_W_Q4_G64, T>(s, c, e, g.M, q);
    return true;
}

bool launch_inproj_decode_mma(hipStream_t s, const InprojDecodeArgs& a, hipError_t& err) {
    const GemvArgs& g = a.g;
    if (g.M < 2) return false;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K, 1.0f / (float)g.K};
    c.xp = static_cast<const uint32_t*>(g.xpack);
    c.part = g.xpart;
    c.nparts = g.nparts;
    auto go = [&](auto tag) -> bool {
        using T = decltype(tag);
        EpiInproj<T> e{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state, (const T*)a.conv_w,
                       (const T*)a.conv_b, (T*)a.z, (T*)a.xbc_act, (T*)a.dt};
        return try_mma<T>(s, c, e, g.M, g.wfmt, g.norm_w != nullptr, err);
    };
    if (g.act == LSSM_F16) return go(f16{});
    if (g.act == LSSM_BF16) return go(bf16{});
    return false;
}

}  // namespace lssm

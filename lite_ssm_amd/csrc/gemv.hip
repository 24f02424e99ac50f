// gemv.hip — dequantize-in-register GEMV for decode (M <= 4 rows of x; decode
// batches of 2..64 rows take the MFMA kernel of gemv_mma.hip when it fits).
//
// Y[m, n] = epi( sum_k deq(W)[n, k] * x[m, k] ), W row-major [N, K] in one of
// the formats of lssm_wfmt.  Restates linear.metal:440-474 (int4 GEMV: exact
// dequantization float(q) * float(scale), fp32 accumulation, one rounding at
// the store) and linear.metal:82-109 (dense fp16 GEMV).
//
// Two kernels, both reading every weight byte from HBM exactly once with
// 16-byte loads (a "chunk": 32 int4 / 16 int8 / 8 dense weights of one row):
//
//  * gemv1 (fp16 / bf16, M <= 4): LPR lanes own one row; lane l owns chunks
//    l, l + LPR, ... (CPL of them), so the LPR lanes of a row cover all of K.
//    Every load of the kernel is issued first and unconditionally (indices
//    clamped, scale and epilogue bits kept raw): the x rows and the norm
//    weight, then the row's weight chunks, scales and epilogue inputs.  The
//    256-thread block RMSNorms x (when fused) and stages it in LDS as packed
//    pairs in the order the unpacked weights come out (plus each chunk's
//    sum(x) where the unpack is biased) while the weights are in flight; each
//    chunk is then unpacked once and multiplied with every x row (v_dot2:
//    exact products, fp32 sums).  Unpacking:
//      int4 x bf16: nibble ^ 8 as a byte, one v_perm per pair puts it under a
//            0x43 byte: bf16 0x43XX = 136 + q; 136 * sum(x) is subtracted per chunk;
//      int4 x fp16: ((q ^ 8) | 0x6400) = 1032 + q, then v_pk_add_f16 -1032 (exact);
//      int8 x fp16: ((q ^ 128) | 0x6400) = 1152 + q, then -1152 (exact).
//    Large N walks row groups with the next group's loads in flight
//    (ping-pong register sets: no copies, so no early waits).
//
//  * gemv_lds (any dtype, any alignment): x rows staged once per block in LDS
//    as fp32, padded by 4 floats per chunk so that the 16-byte reads of the 16
//    lanes of a row fall in distinct banks; 16 lanes per row.
#include <cfloat>
#include <type_traits>

#include "gemv_core.hpp"

namespace lssm {

namespace {


// ---------------------------------------------------------------------------
// Engine decode at batch 1: in_proj + conv + SSD step in one launch
// ---------------------------------------------------------------------------
// The in_proj epilogue (EpiInproj::value) publishes every output row as one
// 64-bit word, (value bits) | (step tag << 32), written by a single-copy-atomic
// device-coherent store; a reader on any CU takes a word once its tag is this
// step's, so neither a fence nor a counter is needed (the tag is a step
// counter the embedding kernel advances; each layer has its own words).
// After its rows, block b runs the SSD step + SiLU(z) gate of the (head,
// 32-column) items b, b + grid, ... with ssd_step_kernel's arithmetic
// (ssd_step.metal:33-77): it waits for the 2N + 65 words an item reads (B and
// C of the head's group, x and z of its columns, dt of the head), which other
// blocks of the same launch store.  The launcher fuses only when every block
// of the launch is resident at once (at most one block per CU), so every
// awaited word gets written; the wait is bounded all the same: an item whose
// words do not all arrive leaves its state slice as it was, writes NaN
// outputs and sets STATUS_WAIT_TIMEOUT in the context's status word, which
// the host reports as an error at its next synchronisation point.
template <typename T> struct EpiInprojSsd {
    static constexpr bool kNormOptional = false;
    static constexpr bool kTail = true;
    static constexpr uint32_t IP = 32;                    // state columns per item
    static constexpr uint32_t NV = 8;                     // lanes per column
    static constexpr uint32_t NN = 128;                   // d_state
    static constexpr int F = (int)(NN / (4 * NV));        // 16-byte state pieces per lane
    static constexpr uint32_t NWD = 2 * NN + 2 * IP + 1;  // words an item reads
    static constexpr uint32_t SPIN = 1u << 16;            // polls before giving up
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    EpiInproj<T> in;                                      // routing / conv (its z, xbc_act, dt unused)
    uint64_t* xfer;                                       // [proj] tagged words of this layer
    const uint32_t* seq;                                  // the step tag (device), or null:
    uint32_t tag0;                                        //   this one
    float* state;                                         // [H, P, NN] of this layer
    const T* A_log;
    const T* dt_bias;
    const T* D;                                           // nullptr: no D term
    T* y;                                                 // [d_inner] gated SSD output, or
    uint32_t* yx;                                         //   tagged 32-bit words when set:
                                                          //   value | (tag mod 2^16) << 16
    uint32_t P, G, items;                                 // items = H * P / IP
    float dt_min, dt_max;
    uint32_t* status;                                     // STATUS_WAIT_TIMEOUT on a failed wait
    uint32_t wait_skew;                                   // 0; 1 = wait for a tag nobody publishes
                                                          // (the failure-handling test's switch)
    using Pre = typename EpiInproj<T>::Pre;
    struct Early {
        f32x4 s[F];
        uint32_t alr, dbr, dr;
    };
    bool fits(uint32_t) const { return true; }           // host: workgroup size check
    __device__ __forceinline__ void pin() const {
        in.pin();
        pin_arg(xfer);
        pin_arg(seq);
        pin_arg(tag0);
        pin_arg(state);
        pin_arg(A_log);
        pin_arg(dt_bias);
        pin_arg(D);
        pin_arg(P);
        pin_arg(items);
        pin_arg(status);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const { return in.prefetch(m, n); }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        const T v = in.value(m, n, acc, p);
        const uint64_t word = (uint64_t)bits16(v) | ((uint64_t)(seq ? *seq : tag0) << 32);
        __hip_atomic_store(xfer + n, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The state columns and head scalars of the block's first item, requested
    // right behind the weights (every thread loads: clamped, values unused
    // where there is no item).
    __device__ __forceinline__ void early(Early& e) const {
        const uint32_t it = blockIdx.x < items ? blockIdx.x : items - 1;
        const uint32_t t = threadIdx.x % (IP * NV);
        const uint32_t ipp = P / IP, h = it / ipp, p = (it % ipp) * IP + t / NV;
        const f32x4* S = reinterpret_cast<const f32x4*>(state + ((size_t)h * P + p) * NN);
#pragma unroll
        for (int f = 0; f < F; ++f) e.s[f] = S[t % NV + NV * f];
        e.alr = raw_at(A_log + h);
        e.dbr = raw_at(dt_bias + h);
        e.dr = raw_at(D ? D + h : A_log + h);             // value unused without D
    }
    // One (head, 32-column) item: wait for its words, then the SSD step + gate.
    __device__ __forceinline__ void item(uint32_t it, const f32x4 (&s)[F], uint32_t alr, uint32_t dbr, uint32_t dr,
                                         uint32_t tag) const {
        __shared__ uint32_t wv[NWD];                      // B, C, x, z, dt value bits
        constexpr uint32_t QNAN = __is_same(T, f16) ? 0x7E00u : 0x7FC0u;
        const uint32_t d_inner = in.d_inner, H = in.H, GN = G * NN, ipp = P / IP;
        const uint32_t h = it / ipp, p0 = (it % ipp) * IP, g = h / (H / G);
        __syncthreads();                                  // a previous item's words read
        int late = 0;                                     // a word of this thread never arrived
        for (uint32_t t = threadIdx.x; t < NWD; t += blockDim.x) {
            uint32_t idx;
            if (t < NN) idx = 2 * d_inner + g * NN + t;                              // B
            else if (t < 2 * NN) idx = 2 * d_inner + GN + g * NN + (t - NN);         // C
            else if (t < 2 * NN + IP) idx = d_inner + h * P + p0 + (t - 2 * NN);     // x
            else if (t < 2 * NN + 2 * IP) idx = h * P + p0 + (t - 2 * NN - IP);      // z
            else idx = d_inner + in.xbc + h;                                         // dt
            uint64_t v = __hip_atomic_load(xfer + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (uint32_t n = 0; (uint32_t)(v >> 32) != tag && n < SPIN; ++n)
                v = __hip_atomic_load(xfer + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            late |= (uint32_t)(v >> 32) != tag;
            wv[t] = (uint32_t)(v >> 32) == tag ? (uint32_t)v : QNAN;
        }
        // the state slice is stored only when every word of the item arrived
        const bool timed_out = __syncthreads_or(late) != 0;
        if (timed_out && threadIdx.x == 0) atomicOr(status, STATUS_WAIT_TIMEOUT);
        if (threadIdx.x >= IP * NV) return;               // wave-uniform; no barrier follows
        const uint32_t lr = threadIdx.x % NV, pl = threadIdx.x / NV;
        f32x4* S = reinterpret_cast<f32x4*>(state + ((size_t)h * P + p0 + pl) * NN);
        const float xv = f_of_raw<T>(wv[2 * NN + pl]);
        const float A_h = -expf(f_of_raw<T>(alr));
        float dt = softplus_f(f_of_raw<T>(wv[2 * NN + 2 * IP]) + f_of_raw<T>(dbr));
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
            f32x4 t = s[f];
            t.x = fmaf(decay, t.x, dt * b0 * xv);
            t.y = fmaf(decay, t.y, dt * b1 * xv);
            t.z = fmaf(decay, t.z, dt * b2 * xv);
            t.w = fmaf(decay, t.w, dt * b3 * xv);
            if (!timed_out) S[lr + NV * f] = t;
            ys += fmaf(c3, t.w, fmaf(c2, t.z, fmaf(c0, t.x, c1 * t.y)));
        }
        ys = group_sum<NV>(ys);
        if (lr == 0) {
            float yv = rnd<T>(fmaf(D ? f_of_raw<T>(dr) : 0.0f, xv, ys));
            yv = silu_fast(f_of_raw<T>(wv[2 * NN + IP + pl])) * yv;
            const size_t yi = (size_t)h * P + p0 + pl;
            if (yx) __hip_atomic_store(yx + yi, bits16(from_f<T>(yv)) | (tag << 16), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            else y[yi] = from_f<T>(yv);
        }
    }
    __device__ __forceinline__ void tail(const Early& e) const {
        const uint32_t tag = (seq ? *seq : tag0) + wait_skew;
        if (blockIdx.x < items) item(blockIdx.x, e.s, e.alr, e.dbr, e.dr, tag);
        // items beyond one per workgroup (not with the engine's shapes): state loaded here
        const uint32_t ipp = P / IP;
        for (uint32_t it = blockIdx.x + gridDim.x; it < items; it += gridDim.x) {
            const uint32_t h = it / ipp, p = (it % ipp) * IP + threadIdx.x % (IP * NV) / NV;
            const f32x4* S = reinterpret_cast<const f32x4*>(state + ((size_t)h * P + p) * NN);
            f32x4 s[F];
#pragma unroll
            for (int f = 0; f < F; ++f) s[f] = S[threadIdx.x % NV + NV * f];
            item(it, s, raw_at(A_log + h), raw_at(dt_bias + h), raw_at(D ? D + h : A_log + h), tag);
        }
    }
};

// Engine decode at batch 1, a layer's whole mixer in one launch: EpiInprojSsd
// with the gated SSD outputs published as tagged words too, then out_proj with
// its gated-RMSNorm prologue and residual add, over weights requested behind
// the in_proj weights and held in registers.  Every workgroup waits for all
// d_inner words and stages them exactly as the separate out_proj launch
// (gemv1_kernel, NORM) would with its own workgroup size BDV: threads below
// BDV take the octets that launch's threads take, in the same order, so the
// sum of squares, the staged pairs and every row come out bit-identical.
// Row group r of out_proj goes to wave r % W of workgroup r / W (W waves per
// workgroup), so that only the first workgroups wait for the gated outputs.
// `hid` is read by every workgroup's in_proj staging and rewritten by the
// out_proj rows; a row is written only once all gated outputs exist, i.e.
// after every workgroup has staged and published its in_proj rows.
template <typename T, int FMT, int LPR2, int CPL2> struct EpiLayer {
    using S = EpiInprojSsd<T>;
    using F = Fmt<FMT, T>;
    static constexpr bool kNormOptional = false;
    static constexpr bool kTail = true;
    static constexpr int WPC = F::WPC, NP = WPC / 2, XS = xs_of<NP>();
    static constexpr int RPW2 = WAVE / LPR2;
    static constexpr uint32_t K2 = (uint32_t)LPR2 * CPL2 * WPC;   // the d_inner this is built for
    static constexpr uint32_t CPR2 = K2 / WPC, NOCT2 = K2 / 8;
    static constexpr int OCT2 = (int)((NOCT2 + G1_NT - 1) / G1_NT);
    static constexpr bool BIAS = q4_bf16<FMT, T>();
    static constexpr uint32_t GD = F::G ? F::G : 1;
    S ssd;                       // in_proj epilogue + SSD items, ssd.yx set
    const uint8_t* w2;           // out_proj [d_model, d_inner]
    const uint16_t* s2;
    const T* nw2;                // mixer (gated) norm weight [d_inner]
    float eps2;
    T* hid;                      // [d_model]: residual in, hidden out
    uint32_t N2;                 // d_model
    uint32_t bdv;                // the separate out_proj launch's workgroup size
    using Pre = typename S::Pre;
    // host: the staging above needs bdv's whole waves inside this launch's workgroups
    bool fits(uint32_t bd) const { return bdv % WAVE == 0 && bdv <= bd && bdv / WAVE <= 16; }
    struct Early {                                       // (vector types: a struct uint4
        typename S::Early e;                             //  would copy through scratch)
        u32x4 wq[CPL2];
        uint16_t sc[CPL2];
        uint32_t res;
        u32x4 nw[OCT2];
    };
    __device__ __forceinline__ void pin() const {
        ssd.pin();
        pin_arg(w2);
        pin_arg(s2);
        pin_arg(nw2);
        pin_arg(hid);
        pin_arg(N2);
        pin_arg(bdv);
    }
    __device__ __forceinline__ Pre prefetch(int m, uint32_t n) const { return ssd.prefetch(m, n); }
    __device__ __forceinline__ void operator()(int m, uint32_t n, float acc, const Pre& p) const {
        ssd(m, n, acc, p);
    }
    // this workgroup's out_proj rows: weights, scales, residual; the norm
    // weight octets its threads below bdv stage
    __device__ __forceinline__ void early(Early& e) const {
        ssd.early(e.e);
        const uint32_t ng = (N2 + RPW2 - 1) / RPW2;
        const uint32_t rg = blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
        uint32_t n = (rg < ng ? rg : ng - 1) * RPW2 + (threadIdx.x % WAVE) / LPR2;
        n = n < N2 ? n : N2 - 1;                        // clamped: every lane loads
        const uint32_t lr = threadIdx.x % LPR2;
        const uint8_t* wr = w2 + (size_t)n * F::row_bytes(K2);
#pragma unroll
        for (int j = 0; j < CPL2; ++j) {
            e.wq[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (size_t)(lr + LPR2 * j) * 16));
        }
        if constexpr (F::G > 0) {
#pragma unroll
            for (int j = 0; j < CPL2; ++j) e.sc[j] = s2[(size_t)n * (K2 / GD) + ((lr + LPR2 * j) * WPC) / GD];
        }
        e.res = raw_at(hid + n);
#pragma unroll
        for (int i = 0; i < OCT2; ++i) {
            uint32_t o = threadIdx.x + bdv * i;
            o = o < NOCT2 ? o : NOCT2 - 1;
            e.nw[i] = reinterpret_cast<const u32x4*>(nw2)[o];
        }
    }
    __device__ __forceinline__ void tail(const Early& e) const {
        __shared__ uint32_t xl2[CPR2 * XS];
        __shared__ float red2[16];
        ssd.tail(e.e);
        const uint32_t tag = ssd.seq ? *ssd.seq : ssd.tag0;
        constexpr uint32_t QNAN = __is_same(T, f16) ? 0x7E00u : 0x7FC0u;
        const int lane = threadIdx.x % WAVE;
        const uint32_t wbase = threadIdx.x & ~(uint32_t)(WAVE - 1);
        // ---- the gated outputs, as octets of packed pairs (threads < bdv) ----
        // Only the workgroups with out_proj rows wait for the gated outputs;
        // each reads the d_inner 32-bit words coalesced (a lane a word, all
        // of a lane's words requested at once, stale ones asked for again)
        // into LDS, from where the threads below bdv pick up their octets.
        const uint32_t nwb = blockDim.x / WAVE;
        const uint32_t ng = (N2 + RPW2 - 1) / RPW2;
        if (blockIdx.x * nwb >= ng) return;              // workgroup-uniform; no barrier follows
        __shared__ __attribute__((aligned(16))) uint16_t ybuf[K2];
        const uint32_t tag16 = tag & 0xFFFFu;
        for (uint32_t k0 = 0; k0 < K2; k0 += 8 * blockDim.x) {   // rounds of 8 words a lane
            uint32_t x[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                uint32_t k = k0 + threadIdx.x + blockDim.x * r;
                k = k < K2 ? k : K2 - 1;                 // clamped: every lane loads
                x[r] = __hip_atomic_load(ssd.yx + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            for (uint32_t it = 0; it < S::SPIN; ++it) {
                bool stale = false;
#pragma unroll
                for (int r = 0; r < 8; ++r) stale |= (x[r] >> 16) != tag16;
                if (!stale) break;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    uint32_t k = k0 + threadIdx.x + blockDim.x * r;
                    k = k < K2 ? k : K2 - 1;
                    if ((x[r] >> 16) != tag16)
                        x[r] = __hip_atomic_load(ssd.yx + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            bool late = false;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const uint32_t k = k0 + threadIdx.x + blockDim.x * r;
                if (k < K2) ybuf[k] = (uint16_t)((x[r] >> 16) == tag16 ? (x[r] & 0xFFFFu) : QNAN);
                late |= k < K2 && (x[r] >> 16) != tag16;
            }
            if (late) atomicOr(ssd.status, STATUS_WAIT_TIMEOUT);
        }
        __syncthreads();
        uint4 xo[OCT2];
        if (threadIdx.x < bdv) {                         // wave-uniform (bdv: whole waves)
#pragma unroll
            for (int i = 0; i < OCT2; ++i) {
                if (wbase + bdv * i >= NOCT2) break;
                uint32_t o = threadIdx.x + bdv * i;
                o = o < NOCT2 ? o : NOCT2 - 1;
                xo[i] = *reinterpret_cast<const uint4*>(ybuf + 8 * o);
            }
        }
        // ---- sum of squares and 1/rms, as gemv1_kernel with bdv threads ----
        float ss = 0.0f;
        if (threadIdx.x < bdv) {
#pragma unroll
            for (int i = 0; i < OCT2; ++i) {
                if (wbase + bdv * i >= NOCT2) break;
                const bool live = threadIdx.x + bdv * i < NOCT2;
                const uint4 d = xo[i];
                float q = dot2(d.x, d.x, 0.0f, T{});
                q = dot2(d.y, d.y, q, T{});
                q = dot2(d.z, d.z, q, T{});
                q = dot2(d.w, d.w, q, T{});
                ss += live ? q : 0.0f;
            }
        }
        ss = wave_sum(ss);
        if (lane == 0 && threadIdx.x < bdv) red2[threadIdx.x / WAVE] = ss;
        __syncthreads();
        float t = 0.0f;
        for (uint32_t w = 0; w < bdv / WAVE; ++w) t += red2[w];
        const float rr = rsqrtf(fmaf(t, 1.0f / (float)K2, eps2));   // as gemv1_kernel
        // ---- stage r(y * w * rr) as packed pairs (+ chunk sums), as gemv1 ----
        if (threadIdx.x < bdv) {
            constexpr uint32_t ONES = __is_same(T, f16) ? 0x3C003C00u : 0x3F803F80u;
#pragma unroll
            for (int i = 0; i < OCT2; ++i) {
                if (wbase + bdv * i >= NOCT2) break;
                const uint32_t o = threadIdx.x + bdv * i;
                const uint32_t k0 = o * 8, ch = k0 / WPC, off = k0 % WPC;
                const uint32_t xd[4] = {xo[i].x, xo[i].y, xo[i].z, xo[i].w};
                const uint32_t wd[4] = {e.nw[i][0], e.nw[i][1], e.nw[i][2], e.nw[i][3]};
                float v[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[2 * q] = lo_f<T>(xd[q]) * lo_f<T>(wd[q]) * rr;
                    v[2 * q + 1] = hi_f<T>(xd[q]) * hi_f<T>(wd[q]) * rr;
                }
                // the octet's offset in its chunk as a constant (a runtime
                // index into v would put it in scratch)
                uint32_t pq[4];
                auto pairs = [&](auto offc) {
                    constexpr int OFF = decltype(offc)::value;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        int a, b;
                        pair_pos<FMT, T>(OFF / 2 + q, a, b);
                        pq[q] = pack2<T>(v[a - OFF], v[b - OFF]);
                    }
                };
                if constexpr (WPC == 32) {
                    switch (off) {
                        case 0: pairs(std::integral_constant<int, 0>{}); break;
                        case 8: pairs(std::integral_constant<int, 8>{}); break;
                        case 16: pairs(std::integral_constant<int, 16>{}); break;
                        default: pairs(std::integral_constant<int, 24>{}); break;
                    }
                } else if constexpr (WPC == 16) {
                    if (off == 0) pairs(std::integral_constant<int, 0>{});
                    else pairs(std::integral_constant<int, 8>{});
                } else {
                    pairs(std::integral_constant<int, 0>{});   // dense: one octet per chunk
                }
                uint32_t* dst = xl2 + ch * XS;
                if (o < NOCT2) *reinterpret_cast<uint4*>(dst + off / 2) = make_uint4(pq[0], pq[1], pq[2], pq[3]);
                if constexpr (BIAS) {
                    float sx = dot2(pq[0], ONES, 0.0f, T{});
                    sx = dot2(pq[1], ONES, sx, T{});
                    sx = dot2(pq[2], ONES, sx, T{});
                    sx = dot2(pq[3], ONES, sx, T{});
                    sx = group_sum<WPC / 8>(sx);
                    if (o < NOCT2 && (o % (WPC / 8)) == 0) dst[NP] = __float_as_uint(sx);
                }
            }
        }
        __syncthreads();
        // ---- this wave's out_proj rows (gemv1_kernel's per-row arithmetic) ----
        const uint32_t rg = blockIdx.x * nwb + threadIdx.x / WAVE;
        if (rg >= ng) return;                            // wave-uniform; no barrier follows
        const uint32_t n = rg * RPW2 + lane / LPR2;
        const uint32_t lr = lane % LPR2;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL2; ++j) {
            const Unpacked<FMT, T> u = unpack<FMT, T>(make_uint4(e.wq[j][0], e.wq[j][1], e.wq[j][2], e.wq[j][3]));
            float sc = 1.0f;
            if constexpr (F::G > 0) sc = fp16_bits_to_f(e.sc[j]);
            const uint32_t* src = xl2 + (lr + LPR2 * j) * XS;
            uint32_t xp[NP];
#pragma unroll
            for (int q = 0; q < NP / 4; ++q) {
                const uint4 vv = *reinterpret_cast<const uint4*>(src + 4 * q);
                xp[4 * q] = vv.x;
                xp[4 * q + 1] = vv.y;
                xp[4 * q + 2] = vv.z;
                xp[4 * q + 3] = vv.w;
            }
            float d = 0.0f;
#pragma unroll
            for (int q = 0; q < NP; ++q) d = dot2(u.p[q], xp[q], d, T{});
            if constexpr (BIAS) d -= 136.0f * __uint_as_float(src[NP]);
            acc = fmaf(d, sc, acc);                     // as gemv1_kernel
        }
        const float a = group_sum<LPR2>(acc);
        if (lr == 0 && n < N2) hid[n] = from_f<T>(f_of_raw<T>(e.res) + rnd<T>(a));
    }
};

// What a kTail epilogue loads behind the weights (nothing for the others).
template <class Epi, bool = Epi::kTail> struct EarlyOf {
    struct type {};
};
template <class Epi> struct EarlyOf<Epi, true> {
    using type = typename Epi::Early;
};

// The lm_head of a batch-1 decode step with its greedy id (sampler.cpp:13-21):
// y[n] = r(acc) as EpiPlain stores it, and the lane that stores a row keeps
// the best (r(acc), n) of its rows by argmax_merge on the stored value; after
// the rows the block reduces them and writes its partial (pv, pi)[blockIdx.x],
// block 0 also the partial count (the grid size) to *count.  A reduction of
// the partials in any order gives the first index of the maximum, as
// argmax_partial_kernel over the stored logits does.  Nothing waits on other
// blocks.
template <typename T> struct EpiLogitsArgmax {
    static constexpr bool kNormOptional = true;
    static constexpr bool kTail = true;
    T* y;
    float* pv;
    int* pi;
    uint32_t* count;
    mutable float bv = -FLT_MAX;
    mutable int bi = 0x7fffffff;
    struct Pre {};
    struct Early {};
    bool fits(uint32_t bd) const { return bd % WAVE == 0 && bd / WAVE <= 16; }
    __device__ __forceinline__ void pin() const {
        pin_arg(y);
        pin_arg(pv);
        pin_arg(pi);
        pin_arg(count);
    }
    __device__ __forceinline__ Pre prefetch(int, uint32_t) const { return Pre{}; }
    __device__ __forceinline__ void operator()(int, uint32_t n, float acc, const Pre&) const {
        const T r = from_f<T>(acc);
        y[n] = r;
        argmax_merge(bv, bi, to_f(r), (int)n);
    }
    __device__ __forceinline__ void early(Early&) const {}
    __device__ __forceinline__ void tail(const Early&) const {
        __shared__ float sv[16];
        __shared__ int si[16];
        float v = bv;
        int i = bi;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(v, off, WAVE);
            const int oi = __shfl_xor(i, off, WAVE);
            argmax_merge(v, i, ov, oi);
        }
        const uint32_t wv = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
        if (threadIdx.x % WAVE == 0) {
            sv[wv] = v;
            si[wv] = i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (uint32_t k = 1; k < nw; ++k) argmax_merge(v, i, sv[k], si[k]);
            pv[blockIdx.x] = v;
            pi[blockIdx.x] = i;
            if (blockIdx.x == 0) *count = gridDim.x;
        }
    }
};

// Weights, raw scale bits and epilogue inputs of the rows one wave handles.
template <int CPL, int MR, class Epi> struct RowSet {
    uint4 wq[CPL];
    uint16_t sc[CPL];
    typename Epi::Pre pre[MR];
    uint32_t n;
};

template <int FMT, typename T, int LPR, int CPL, int OCT, int MR, bool NORM, bool LOOP, int NTMAX, class Epi>
__global__ __launch_bounds__(NTMAX) void gemv1_kernel(GemvCore c, Epi epi, uint32_t iters, int mr) {
    using F = Fmt<FMT, T>;
    constexpr int WPC = F::WPC;
    constexpr int NP = WPC / 2;                      // packed pairs per chunk
    constexpr int XS = xs_of<NP>();
    constexpr int RPW = WAVE / LPR;                  // rows per wave
    constexpr bool BIAS = q4_bf16<FMT, T>();
    constexpr uint32_t GD = F::G ? F::G : 1;
    extern __shared__ uint32_t xl[];                 // [MR][cpr][XS]
    __shared__ float red[MR][NTMAX / WAVE];
    const uint32_t BD = blockDim.x;                  // >= G1_NT, a multiple of the wave
    const uint32_t NWB = BD / WAVE;
    const int lane = threadIdx.x % WAVE;
    const int lr = lane % LPR;
    const uint32_t wbase = threadIdx.x & ~(uint32_t)(WAVE - 1);
    const uint32_t K = c.K;
    const uint32_t cpr = K / WPC;
    const uint32_t noct = K / 8;
    const size_t rb = F::row_bytes(K);
    const uint32_t gpr = K / GD;

    pin_arg(c.x);
    pin_arg(c.x_stride);
    pin_arg(c.w);
    pin_arg(c.s);
    pin_arg(c.norm_w);
    pin_arg(c.eps);
    pin_arg(c.N);
    pin_arg(c.K);
    pin_arg(c.inv_k);
    epi.pin();
    __builtin_amdgcn_sched_barrier(0);

    // ---- 1. x rows and the norm weight, requested before any weight ----
    // A CU's vector loads return in request order, so the block issues all its
    // x loads, meets at a barrier that waits for no memory, and only then asks
    // for its weights: x is not queued behind the weight traffic.
    uint4 xo[MR][OCT], wo[OCT];
#pragma unroll
    for (int i = 0; i < OCT; ++i) {
        if (wbase + BD * i < noct) {                 // wave-uniform
            uint32_t o = threadIdx.x + BD * i;
            o = o < noct ? o : noct - 1;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int mc = m < mr ? m : mr - 1;      // rows past mr: a duplicate, never stored
                xo[m][i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(c.x) + (size_t)mc * c.x_stride + 8 * o);
            }
            if constexpr (NORM) wo[i] = reinterpret_cast<const uint4*>(c.norm_w)[o];
        }
    }
    // ---- 2. scales and epilogue inputs of the first row set, then weights ----
    // The small loads (a 2-byte scale per chunk, the epilogue's inputs) go out
    // here, while the memory system is quiet: issued behind the weights they
    // would hold the wave as long as the weight traffic pushes back.  The
    // 16-byte weight chunks follow (below).  Scheduling barriers pin the issue
    // order; waits count loads in issue order.
    const uint32_t nwaves = gridDim.x * NWB;
    const uint32_t wv = blockIdx.x * NWB + threadIdx.x / WAVE;
    auto load_side = [&](RowSet<CPL, MR, Epi>& rs, uint32_t group) {
        rs.n = group * RPW + lane / LPR;
        const uint32_t nc = rs.n < c.N ? rs.n : c.N - 1;   // clamped: every lane loads
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (F::G > 0) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) rs.sc[j] = c.s[(size_t)nc * gpr + ((lr + LPR * j) * WPC) / GD];
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) rs.pre[m] = epi.prefetch(m < mr ? m : mr - 1, nc);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto load_w = [&](RowSet<CPL, MR, Epi>& rs) {
        const uint32_t nc = rs.n < c.N ? rs.n : c.N - 1;
        const uint8_t* wr = c.w + (size_t)nc * rb;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + (size_t)(lr + LPR * j) * 16));
            rs.wq[j] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    RowSet<CPL, MR, Epi> A;
    load_side(A, wv);
    // With the RMSNorm prologue (the decode linears) the weights are requested
    // right behind x: x still returns first (a wave's loads return in issue
    // order) and the weights stream in while x is normalised and staged
    // (2.7B batch-1 decode: in_proj + SSD 9.36 -> 8.76 us, out_proj 5.32 ->
    // 4.64 us, 1001 -> 1104 tok/s, against requesting them after the staging
    // barrier; a barrier between the x and the weight requests cost 1 %).
    constexpr bool EARLY_W = NORM && !LOOP;
    if constexpr (EARLY_W) load_w(A);

    // ---- 1b. sum(x^2) and 1/rms ----
    // sum(x^2) uses v_dot2 on packed pairs (exact products, fp32 sums).
    float rr[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) rr[m] = 1.0f;
    if constexpr (NORM) {
        float ss[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) ss[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < OCT; ++i) {
            if (wbase + BD * i >= noct) break;
            const bool live = threadIdx.x + BD * i < noct;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint4 d = xo[m][i];
                float q = dot2(d.x, d.x, 0.0f, T{});
                q = dot2(d.y, d.y, q, T{});
                q = dot2(d.z, d.z, q, T{});
                q = dot2(d.w, d.w, q, T{});
                ss[m] += live ? q : 0.0f;
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) ss[m] = wave_sum(ss[m]);
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) red[m][threadIdx.x / WAVE] = ss[m];
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float t = 0.0f;
            for (uint32_t w = 0; w < NWB; ++w) t += red[m][w];
            rr[m] = rsqrtf(fmaf(t, c.inv_k, c.eps));
        }
    } else {
        // no norm: the block meets once its x loads are issued (no wait)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }


    // ---- 3. stage x (RMSNorm'ed when fused, norm.metal:52-79) as packed pairs ----
    // Only the waves holding x octets stage (a wave-uniform branch).  The
    // normalised values are rounded straight into the pairs; the chunk sums
    // use v_dot2 with (1, 1).
    {
        constexpr uint32_t ONES = __is_same(T, f16) ? 0x3C003C00u : 0x3F803F80u;   // (1, 1)
#pragma unroll
        for (int i = 0; i < OCT; ++i) {
            if (wbase + BD * i >= noct) break;
            const uint32_t o = threadIdx.x + BD * i;
            const uint32_t k0 = o * 8, ch = k0 / WPC, off = k0 % WPC;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const T* t = reinterpret_cast<const T*>(&xo[m][i]);
                float v[8];
                if constexpr (NORM) {
                    // x * w exactly (a product of 8- or 11-bit significands in
                    // fp32), then * 1/rms: the fp32 products of the reference
                    const uint32_t* xd = reinterpret_cast<const uint32_t*>(&xo[m][i]);
                    const uint32_t* wd = reinterpret_cast<const uint32_t*>(&wo[i]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = lo_f<T>(xd[e]) * lo_f<T>(wd[e]) * rr[m];
                        v[2 * e + 1] = hi_f<T>(xd[e]) * hi_f<T>(wd[e]) * rr[m];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = to_f(t[e]);
                }
                uint4 pk;
                uint32_t* pq = reinterpret_cast<uint32_t*>(&pk);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int a, b;
                    pair_pos<FMT, T>((int)(off / 2) + q, a, b);
                    pq[q] = pack2<T>(v[a - (int)off], v[b - (int)off]);   // the rounding r()
                }
                uint32_t* dst = xl + ((size_t)m * cpr + ch) * XS;
                if (o < noct) *reinterpret_cast<uint4*>(dst + off / 2) = pk;
                if constexpr (BIAS) {
                    // sum(x) of a chunk: its WPC/8 octets sit in consecutive lanes
                    float s = dot2(pq[0], ONES, 0.0f, T{});
                    s = dot2(pq[1], ONES, s, T{});
                    s = dot2(pq[2], ONES, s, T{});
                    s = dot2(pq[3], ONES, s, T{});
                    s = group_sum<WPC / 8>(s);
                    if (o < noct && (o % (WPC / 8)) == 0) dst[NP] = __float_as_uint(s);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    }
    // Otherwise the weights are requested after the last barrier.
    if constexpr (!EARLY_W) load_w(A);
    [[maybe_unused]] typename EarlyOf<Epi>::type early;
    if constexpr (Epi::kTail) epi.early(early);


    // ---- 4. rows; the next row's loads are in flight while this one is reduced ----
    auto compute = [&](const RowSet<CPL, MR, Epi>& rs) {
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const Unpacked<FMT, T> u = unpack<FMT, T>(rs.wq[j]);
            float sc = 1.0f;
            if constexpr (F::G > 0) sc = fp16_bits_to_f(rs.sc[j]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const uint32_t* src = xl + ((size_t)m * cpr + lr + LPR * j) * XS;
                uint32_t xp[NP];
#pragma unroll
                for (int q = 0; q < NP / 4; ++q) {
                    const uint4 v = *reinterpret_cast<const uint4*>(src + 4 * q);
                    xp[4 * q] = v.x;
                    xp[4 * q + 1] = v.y;
                    xp[4 * q + 2] = v.z;
                    xp[4 * q + 3] = v.w;
                }
                float d = 0.0f;
#pragma unroll
                for (int q = 0; q < NP; ++q) d = dot2(u.p[q], xp[q], d, T{});
                if constexpr (BIAS) d -= 136.0f * __uint_as_float(src[NP]);
                acc[m] = fmaf(d, sc, acc[m]);           // spelled out: the one-launch mixer matches it
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = group_sum<LPR>(acc[m]);
            if (lr == 0 && rs.n < c.N && m < mr) epi(m, rs.n, a, rs.pre[m]);
        }
    };
    if constexpr (!LOOP) {
        compute(A);
    } else {
        // ping-pong between two row sets: no register copies, so no early waits
        RowSet<CPL, MR, Epi> B;
        for (uint32_t it = 0; it < iters; it += 2) {
            if (it + 1 < iters) {
                load_side(B, wv + (it + 1) * nwaves);
                load_w(B);
            }
            compute(A);
            if (it + 1 >= iters) break;
            if (it + 2 < iters) {
                load_side(A, wv + (it + 2) * nwaves);
                load_w(A);
            }
            compute(B);
        }
    }
    if constexpr (Epi::kTail) epi.tail(early);
}

template <int FMT, typename T, int LPR, int CPL, int MR, class Epi>
hipError_t go1(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int norm) {
    constexpr int RPW = WAVE / LPR;
    constexpr int NW = G1_NT / WAVE;
    using F = Fmt<FMT, T>;
    constexpr uint32_t KC = (uint32_t)LPR * CPL * F::WPC;     // the K this shape is built for
    constexpr int OCT = (int)((KC / 8 + G1_NT - 1) / G1_NT);
    static_assert(OCT >= 1 && OCT <= 4, "x staging: K <= 8192");
    // Dense single-row GEMVs (the lm_head, N up to 256k) walk row groups with
    // a bounded grid, so that x is staged by few blocks.  Otherwise every wave
    // takes one row group and single-row launches size their blocks to put
    // one block on each CU (x staged once per CU, requested ahead of the
    // CU's weight traffic); multi-row launches (high register use) keep
    // 256-thread blocks.
    constexpr bool LOOP = FMT == LSSM_W_DENSE && MR == 1;
    constexpr int NTMAX = MR == 1 ? 1024 : G1_NT;
    const uint32_t ngroups = (c.N + RPW - 1) / RPW;
    const uint32_t cap = 4096;                                 // 4 resident waves per SIMD
    const uint32_t iters = LOOP ? (ngroups + cap - 1) / cap : 1u;
    const uint32_t waves = (ngroups + iters - 1) / iters;
    uint32_t wpb = NW;                                         // waves per block
    if (MR == 1) {
        const uint32_t per_cu = (waves + num_cus() - 1) / num_cus();
        wpb = per_cu < (uint32_t)NW ? (uint32_t)NW : per_cu > 16u ? 16u : per_cu;
    }
    const uint32_t blocks = (waves + wpb - 1) / wpb;
    const size_t lds = (size_t)MR * (KC / F::WPC) * xs_of<F::WPC / 2>() * sizeof(uint32_t);
    if (c.K != KC || lds > GV_LDS_MAX) return hipErrorInvalidValue;
    // a tail that waits on other blocks' rows needs every block resident: one
    // block per CU (up to 16 waves at <= 128 VGPRs fits an idle CU)
    if constexpr (Epi::kTail) {
        if (blocks > num_cus() || MR != 1 || !e.fits(wpb * WAVE)) return hipErrorNotSupported;
    }
    auto run = [&](auto k) -> hipError_t {
        // opt in to the full dynamic LDS once per instantiation (a host attribute)
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, (int)GV_LDS_MAX);
        if (attr != hipSuccess) return attr;
        k<<<blocks, wpb * WAVE, lds, s>>>(c, e, iters, mr);
        return hipGetLastError();
    };
    if (norm) return run(gemv1_kernel<FMT, T, LPR, CPL, OCT, MR, true, LOOP, NTMAX, Epi>);
    if constexpr (Epi::kNormOptional) return run(gemv1_kernel<FMT, T, LPR, CPL, OCT, MR, false, LOOP, NTMAX, Epi>);
    return hipErrorInvalidValue;
}

// (lanes per row, chunks per lane) for the chunk counts of the model shapes
// (d_model / d_inner of 130M, 2.7B, 8B and 2048), per weight format.
template <int FMT, typename T, int MR, class Epi>
hipError_t launch_gemv1(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int norm, bool& done) {
    done = true;
    const uint32_t cpr = c.K / Fmt<FMT, T>::WPC;
    if constexpr (is_q4<FMT>()) {                             // K = 1536 .. 8192
        switch (cpr) {
            case 48: return go1<FMT, T, 16, 3, MR, Epi>(s, c, e, mr, norm);
            case 64: return go1<FMT, T, 16, 4, MR, Epi>(s, c, e, mr, norm);
            case 80: return go1<FMT, T, 16, 5, MR, Epi>(s, c, e, mr, norm);
            case 128: return go1<FMT, T, 32, 4, MR, Epi>(s, c, e, mr, norm);
            case 160: return go1<FMT, T, 32, 5, MR, Epi>(s, c, e, mr, norm);
            case 256: return go1<FMT, T, 64, 4, MR, Epi>(s, c, e, mr, norm);
        }
    } else if constexpr (FMT == LSSM_W_Q8_G32) {              // K = 768 .. 8192
        switch (cpr) {
            case 48: return go1<FMT, T, 16, 3, MR, Epi>(s, c, e, mr, norm);
            case 96: return go1<FMT, T, 32, 3, MR, Epi>(s, c, e, mr, norm);
            case 128: return go1<FMT, T, 32, 4, MR, Epi>(s, c, e, mr, norm);
            case 160: return go1<FMT, T, 32, 5, MR, Epi>(s, c, e, mr, norm);
            case 256: return go1<FMT, T, 64, 4, MR, Epi>(s, c, e, mr, norm);
            case 320: return go1<FMT, T, 64, 5, MR, Epi>(s, c, e, mr, norm);
            case 512: return go1<FMT, T, 64, 8, MR, Epi>(s, c, e, mr, norm);
        }
    } else {                                                  // dense, K = 768 .. 4096
        switch (cpr) {
            case 96: return go1<FMT, T, 32, 3, MR, Epi>(s, c, e, mr, norm);
            case 192: return go1<FMT, T, 64, 3, MR, Epi>(s, c, e, mr, norm);
            case 256: return go1<FMT, T, 64, 4, MR, Epi>(s, c, e, mr, norm);
            case 320: return go1<FMT, T, 64, 5, MR, Epi>(s, c, e, mr, norm);
            case 512: return go1<FMT, T, 64, 8, MR, Epi>(s, c, e, mr, norm);
        }
    }
    done = false;
    return hipSuccess;
}

template <int FMT> bool gemv1_shape(uint32_t cpr) {
    if constexpr (is_q4<FMT>()) return cpr == 48 || cpr == 64 || cpr == 80 || cpr == 128 || cpr == 160 || cpr == 256;
    else if constexpr (FMT == LSSM_W_Q8_G32)
        return cpr == 48 || cpr == 96 || cpr == 128 || cpr == 160 || cpr == 256 || cpr == 320 || cpr == 512;
    else return cpr == 96 || cpr == 192 || cpr == 256 || cpr == 320 || cpr == 512;
}

// Largest MR the gemv1 staging of this K / format fits (0 = not a gemv1 shape).
inline int gemv1_rows(uint32_t K, int wfmt, int act) {
    if (act == LSSM_F32 || (wfmt == LSSM_W_Q8_G32 && act != LSSM_F16)) return 0;
    const uint32_t wpc = wpc_of(wfmt, act);
    if (K % wpc != 0) return 0;
    const uint32_t cpr = K / wpc;
    bool ok;
    switch (wfmt) {
        case LSSM_W_Q4_B32:
        case LSSM_W_Q4_G64: ok = gemv1_shape<LSSM_W_Q4_G64>(cpr); break;
        case LSSM_W_Q8_G32: ok = gemv1_shape<LSSM_W_Q8_G32>(cpr); break;
        default: ok = gemv1_shape<LSSM_W_DENSE>(cpr); break;
    }
    if (!ok) return 0;
    const uint32_t np = wpc / 2;
    const size_t per_row = (size_t)cpr * (np == 4 ? 4 : np == 8 ? 12 : 20) * sizeof(uint32_t);
    const int mr = (int)(GV_LDS_MAX / per_row);
    return mr > 4 ? 4 : mr;
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

// Largest number of x rows per launch whose padded fp32 LDS staging fits.
inline int lds_rows(uint32_t K, int wfmt, int act) {
    const uint32_t wpc = wpc_of(wfmt, act);
    int mr = (int)(GV_LDS_MAX / ((size_t)padded_len(K, wpc) * sizeof(float)));
    return mr > 4 ? 4 : mr;
}

template <typename T> constexpr int act_of() {
    return __is_same(T, f16) ? LSSM_F16 : __is_same(T, bf16) ? LSSM_BF16 : LSSM_F32;
}

// Rows of x one launch of this call can take: gemv1 when its 16-byte loads
// are aligned and the shape is one of its table, else the fp32 LDS kernel.
template <typename T> int rows_for(const GemvCore& c, int wfmt, int norm) {
    const bool aligned = ((uintptr_t)c.x % 16 == 0) && ((c.x_stride * sizeof(T)) % 16 == 0) &&
                         (!norm || (uintptr_t)c.norm_w % 16 == 0) && ((uintptr_t)c.w % 16 == 0);
    const int g1 = aligned ? gemv1_rows(c.K, wfmt, act_of<T>()) : 0;
    return g1 > 0 ? g1 : lds_rows(c.K, wfmt, act_of<T>());
}

// MR in {1, 2, 4}; three rows run in the four-row kernel (a duplicate row, not stored).
template <int FMT, typename T, class Epi>
hipError_t launch_gemv1_mr(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int norm, bool& done) {
    switch (mr) {
        case 1: return launch_gemv1<FMT, T, 1, Epi>(s, c, e, mr, norm, done);
        case 2: return launch_gemv1<FMT, T, 2, Epi>(s, c, e, mr, norm, done);
        default: return launch_gemv1<FMT, T, 4, Epi>(s, c, e, mr, norm, done);
    }
}

// Format dispatch: fp16 / bf16 with aligned operands go to gemv1.
template <typename T, class Epi>
hipError_t launch_fmt(hipStream_t s, const GemvCore& c, const Epi& e, int mr, int wfmt, int norm) {
    if (mr < 1 || mr > rows_for<T>(c, wfmt, norm)) return hipErrorInvalidValue;
    if constexpr (!__is_same(T, float)) {
        const bool aligned = ((uintptr_t)c.x % 16 == 0) && ((c.x_stride * sizeof(T)) % 16 == 0) &&
                             (!norm || (uintptr_t)c.norm_w % 16 == 0) && ((uintptr_t)c.w % 16 == 0);
        if (aligned && gemv1_rows(c.K, wfmt, act_of<T>()) >= mr) {
            bool done = false;
            hipError_t err = hipSuccess;
            switch (wfmt) {
                case LSSM_W_Q4_B32: err = launch_gemv1_mr<LSSM_W_Q4_B32, T, Epi>(s, c, e, mr, norm, done); break;
                case LSSM_W_Q4_G64: err = launch_gemv1_mr<LSSM_W_Q4_G64, T, Epi>(s, c, e, mr, norm, done); break;
                case LSSM_W_Q8_G32:
                    if constexpr (__is_same(T, f16)) err = launch_gemv1_mr<LSSM_W_Q8_G32, T, Epi>(s, c, e, mr, norm, done);
                    break;
                default: err = launch_gemv1_mr<LSSM_W_DENSE, T, Epi>(s, c, e, mr, norm, done); break;
            }
            if (done) return err;
        }
    }
    if (mr > lds_rows(c.K, wfmt, act_of<T>())) return hipErrorInvalidValue;
    switch (wfmt) {
        case LSSM_W_Q4_B32: return launch_lds_mr<LSSM_W_Q4_B32, T, Epi>(s, c, e, mr, norm);
        case LSSM_W_Q4_G64: return launch_lds_mr<LSSM_W_Q4_G64, T, Epi>(s, c, e, mr, norm);
        case LSSM_W_Q8_G32: return launch_lds_mr<LSSM_W_Q8_G32, T, Epi>(s, c, e, mr, norm);
        default: return launch_lds_mr<LSSM_W_DENSE, T, Epi>(s, c, e, mr, norm);
    }
}

// Rows per launch when operands are aligned (what callers plan with).
inline int max_rows(uint32_t K, int wfmt, int act) {
    const int g1 = gemv1_rows(K, wfmt, act);
    const int l = lds_rows(K, wfmt, act);
    return g1 > l ? g1 : l;
}

template <typename T>
hipError_t gemv_plain(hipStream_t s, const GemvArgs& a) {
    const size_t es = sizeof(T);
    GemvCore c0{a.x, a.x_stride, (const uint8_t*)a.w, (const uint16_t*)a.s, a.norm_w, a.eps, a.N, a.K, 1.0f / (float)a.K};
    {
        // decode batches: all rows in one MFMA launch when the shape allows
        hipError_t err = hipSuccess;
        if (launch_gemv_mma(s, a, err)) return err;
    }
    const int mrmax = rows_for<T>(c0, a.wfmt, a.norm_w ? 1 : 0);
    if (mrmax < 1) return hipErrorInvalidValue;
    for (uint32_t m0 = 0; m0 < a.M; m0 += (uint32_t)mrmax) {
        const int mr = (int)((a.M - m0) < (uint32_t)mrmax ? (a.M - m0) : (uint32_t)mrmax);
        GemvCore c{(const char*)a.x + (size_t)m0 * a.x_stride * es, a.x_stride,
                   (const uint8_t*)a.w, (const uint16_t*)a.s, a.norm_w, a.eps, a.N, a.K, 1.0f / (float)a.K};
        EpiPlain<T> e{(T*)a.y + (size_t)m0 * a.y_stride, a.y_stride,
                      a.res ? (const T*)a.res + (size_t)m0 * a.y_stride : nullptr, a.epi};
        hipError_t err = launch_fmt<T>(s, c, e, mr, a.wfmt, a.norm_w ? 1 : 0);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

// The lm_head GEMV of one row with its argmax folded in (EpiLogitsArgmax),
// then the reduction of the blocks' partials.  Scratch: the count (16 bytes),
// then the partials' values and indices, room for at least one per CU (the
// tail epilogue runs only with at most one block per CU).
template <typename T>
hipError_t gemv_argmax(hipStream_t s, const GemvArgs& a, int32_t* ids, void* scratch, size_t bytes) {
    const size_t cap = bytes > 16 ? (bytes - 16) / 8 : 0;
    if (a.M != 1 || a.wfmt != LSSM_W_DENSE || a.epi != LSSM_EPI_NONE || a.res || cap < num_cus() ||
        (uintptr_t)scratch % 16 != 0)
        return hipErrorNotSupported;
    const bool norm = a.norm_w != nullptr;
    GemvCore c{a.x, a.x_stride, (const uint8_t*)a.w, nullptr, a.norm_w, a.eps, a.N, a.K, 1.0f / (float)a.K};
    const bool aligned = ((uintptr_t)c.x % 16 == 0) && ((c.x_stride * sizeof(T)) % 16 == 0) &&
                         (!norm || (uintptr_t)c.norm_w % 16 == 0) && ((uintptr_t)c.w % 16 == 0);
    if (!aligned || gemv1_rows(c.K, LSSM_W_DENSE, act_of<T>()) < 1) return hipErrorNotSupported;
    uint32_t* count = (uint32_t*)scratch;
    float* pv = (float*)((char*)scratch + 16);
    int* pi = (int*)(pv + cap);
    EpiLogitsArgmax<T> e{(T*)a.y, pv, pi, count};
    bool done = false;
    const hipError_t err = launch_gemv1<LSSM_W_DENSE, T, 1, EpiLogitsArgmax<T>>(s, c, e, 1, norm ? 1 : 0, done);
    if (!done) return hipErrorNotSupported;
    if (err != hipSuccess) return err;
    return launch_argmax_final(s, pv, pi, count, ids);
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

hipError_t launch_gemv_argmax(hipStream_t s, const GemvArgs& a, int32_t* ids, void* scratch,
                              size_t scratch_bytes) {
    if (a.act == LSSM_F16) return gemv_argmax<f16>(s, a, ids, scratch, scratch_bytes);
    if (a.act == LSSM_BF16) return gemv_argmax<bf16>(s, a, ids, scratch, scratch_bytes);
    return hipErrorNotSupported;
}
int gemv_lds_rows(uint32_t K, int wfmt, int act) { return lds_rows(K, wfmt, act); }

hipError_t launch_gemv(hipStream_t s, const GemvArgs& a) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.act == LSSM_F16) return gemv_plain<f16>(s, a);
    if (a.act == LSSM_BF16) return gemv_plain<bf16>(s, a);
    return gemv_plain<float>(s, a);
}

hipError_t launch_inproj_decode(hipStream_t s, const InprojDecodeArgs& a) {
    const GemvArgs& g = a.g;
    if (g.M == 0) return hipSuccess;
    {
        hipError_t err = hipSuccess;
        if (launch_inproj_decode_mma(s, a, err)) return err;
    }
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K, 1.0f / (float)g.K};
    auto go = [&](auto tag) -> hipError_t {
        using T = decltype(tag);
        // gemv1 / gemv_lds, in launches of as many rows as their staging takes
        const int mrmax = rows_for<T>(c, g.wfmt, g.norm_w ? 1 : 0);
        if (mrmax < 1) return hipErrorInvalidValue;
        for (uint32_t m0 = 0; m0 < g.M; m0 += (uint32_t)mrmax) {
            const int mr = (int)((g.M - m0) < (uint32_t)mrmax ? (g.M - m0) : (uint32_t)mrmax);
            GemvCore cm = c;
            cm.x = (const T*)g.x + (size_t)m0 * g.x_stride;
            EpiInproj<T> e{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state + (size_t)m0 * a.xbc * a.dconv,
                           (const T*)a.conv_w, (const T*)a.conv_b, (T*)a.z + (size_t)m0 * a.d_inner,
                           (T*)a.xbc_act + (size_t)m0 * a.xbc, (T*)a.dt + (size_t)m0 * a.H};
            hipError_t err = launch_fmt<T>(s, cm, e, mr, g.wfmt, g.norm_w ? 1 : 0);
            if (err != hipSuccess) return err;
        }
        return hipSuccess;
    };
    if (g.act == LSSM_F16) return go(f16{});
    if (g.act == LSSM_BF16) return go(bf16{});
    return go(float{});
}

namespace {
template <typename T> EpiInprojSsd<T> make_ssd_epi(const InprojDecodeArgs& a, const SsdFuseArgs& f) {
    EpiInprojSsd<T> e{};
    e.in = EpiInproj<T>{a.d_inner, a.xbc, a.H, a.dconv, (T*)a.conv_state, (const T*)a.conv_w,
                        (const T*)a.conv_b, nullptr, nullptr, nullptr};
    e.xfer = f.xfer;
    e.seq = f.seq;
    e.tag0 = f.tag;
    e.state = f.state;
    e.A_log = (const T*)f.A_log;
    e.dt_bias = (const T*)f.dt_bias;
    e.D = (const T*)f.D;
    e.y = (T*)f.y;
    e.yx = nullptr;
    e.P = f.P;
    e.G = f.G;
    e.items = a.H * (f.P / EpiInprojSsd<T>::IP);
    e.dt_min = f.dt_min;
    e.dt_max = f.dt_max;
    e.status = f.status;
    e.wait_skew = f.wait_skew;
    return e;
}
}  // namespace

bool launch_inproj_ssd_decode(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseArgs& f, hipError_t& err) {
    err = hipSuccess;
    const GemvArgs& g = a.g;
    if (g.M != 1 || !g.norm_w || (g.act != LSSM_F16 && g.act != LSSM_BF16)) return false;
    if (a.dconv != 4 || f.N != EpiInprojSsd<f16>::NN || f.P == 0 || f.P % EpiInprojSsd<f16>::IP != 0 ||
        f.G == 0 || a.H % f.G != 0 || a.d_inner != a.H * f.P || a.xbc != a.d_inner + 2 * f.G * f.N ||
        g.N != a.d_inner + a.xbc + a.H)
        return false;
    if (g.wfmt != LSSM_W_Q4_G64 && !(g.wfmt == LSSM_W_Q8_G32 && g.act == LSSM_F16)) return false;
    const bool aligned = ((uintptr_t)g.x % 16 == 0) && ((uintptr_t)g.norm_w % 16 == 0) &&
                         ((uintptr_t)g.w % 16 == 0) && ((uintptr_t)f.state % 16 == 0) &&
                         ((uintptr_t)a.conv_state % 8 == 0) && ((uintptr_t)a.conv_w % 8 == 0);
    if (!aligned || gemv1_rows(g.K, g.wfmt, g.act) < 1) return false;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K, 1.0f / (float)g.K};
    auto go = [&](auto tag) -> hipError_t {
        using T = decltype(tag);
        const EpiInprojSsd<T> e = make_ssd_epi<T>(a, f);
        bool done = false;
        hipError_t r = hipErrorNotSupported;
        if (g.wfmt == LSSM_W_Q4_G64) r = launch_gemv1<LSSM_W_Q4_G64, T, 1, EpiInprojSsd<T>>(s, c, e, 1, 1, done);
        else if constexpr (__is_same(T, f16)) r = launch_gemv1<LSSM_W_Q8_G32, T, 1, EpiInprojSsd<T>>(s, c, e, 1, 1, done);
        return done ? r : hipErrorNotSupported;
    };
    const hipError_t r = g.act == LSSM_F16 ? go(f16{}) : go(bf16{});
    if (r == hipErrorNotSupported) return false;   // nothing launched
    err = r;
    return true;
}

namespace {
// Workgroup size gemv1 picks for a single-row launch of N rows at lpr lanes
// per row (go1's rule).
uint32_t gemv1_bd(uint32_t N, uint32_t lpr) {
    const uint32_t ngroups = (N + (WAVE / lpr) - 1) / (WAVE / lpr);
    const uint32_t per_cu = (ngroups + num_cus() - 1) / num_cus();
    const uint32_t nw = G1_NT / WAVE;
    return WAVE * (per_cu < nw ? nw : per_cu > 16u ? 16u : per_cu);
}

template <typename T, int FMT, int LPR, int CPL, int LPR2, int CPL2>
hipError_t go_layer(hipStream_t s, const GemvCore& c, const EpiInprojSsd<T>& es, const OutprojFuseArgs& o) {
    using E = EpiLayer<T, FMT, LPR2, CPL2>;
    E e{};
    e.ssd = es;
    e.ssd.yx = o.yx;
    e.w2 = (const uint8_t*)o.w;
    e.s2 = (const uint16_t*)o.s;
    e.nw2 = (const T*)o.norm_w;
    e.eps2 = o.eps;
    e.hid = (T*)o.hidden;
    e.N2 = o.N;
    e.bdv = gemv1_bd(o.N, LPR2);
    return go1<FMT, T, LPR, CPL, 1, E>(s, c, e, 1, 1);
}
}  // namespace

bool launch_layer_decode(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseArgs& f, const OutprojFuseArgs& o,
                         hipError_t& err) {
    err = hipSuccess;
    const GemvArgs& g = a.g;
    if (!o.w || !o.norm_w || !o.hidden || !o.yx || o.hidden != g.x || o.N != g.K) return false;
    if (((uintptr_t)o.w % 16) != 0 || ((uintptr_t)o.norm_w % 16) != 0) return false;
    if (g.wfmt != LSSM_W_DENSE && !o.s) return false;
    // the in_proj + SSD part's own checks (launching nothing)
    if (g.M != 1 || !g.norm_w || (g.act != LSSM_F16 && g.act != LSSM_BF16)) return false;
    if (a.dconv != 4 || f.N != EpiInprojSsd<f16>::NN || f.P == 0 || f.P % EpiInprojSsd<f16>::IP != 0 ||
        f.G == 0 || a.H % f.G != 0 || a.d_inner != a.H * f.P || a.xbc != a.d_inner + 2 * f.G * f.N ||
        g.N != a.d_inner + a.xbc + a.H)
        return false;
    const bool aligned = ((uintptr_t)g.x % 16 == 0) && ((uintptr_t)g.norm_w % 16 == 0) &&
                         ((uintptr_t)g.w % 16 == 0) && ((uintptr_t)f.state % 16 == 0) &&
                         ((uintptr_t)a.conv_state % 8 == 0) && ((uintptr_t)a.conv_w % 8 == 0);
    if (!aligned) return false;
    GemvCore c{g.x, g.x_stride, (const uint8_t*)g.w, (const uint16_t*)g.s, g.norm_w, g.eps, g.N, g.K, 1.0f / (float)g.K};
    auto go = [&](auto tag) -> hipError_t {
        using T = decltype(tag);
        const EpiInprojSsd<T> es = make_ssd_epi<T>(a, f);
        const uint32_t ci = g.K / wpc_of(g.wfmt, g.act), co = a.d_inner / wpc_of(g.wfmt, g.act);
        if (g.wfmt == LSSM_W_Q4_G64) {
            if (ci == 80 && co == 160) return go_layer<T, LSSM_W_Q4_G64, 16, 5, 32, 5>(s, c, es, o);   // 2.7B
            if (ci == 64 && co == 64) return go_layer<T, LSSM_W_Q4_G64, 16, 4, 16, 4>(s, c, es, o);
        } else if constexpr (__is_same(T, f16)) {
            if (g.wfmt == LSSM_W_Q8_G32 && ci == 48 && co == 96)
                return go_layer<T, LSSM_W_Q8_G32, 16, 3, 32, 3>(s, c, es, o);                      // 130M
        }
        return hipErrorNotSupported;
    };
    const hipError_t r = g.act == LSSM_F16 ? go(f16{}) : go(bf16{});
    if (r == hipErrorNotSupported) return false;   // nothing launched
    err = r;
    return true;
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

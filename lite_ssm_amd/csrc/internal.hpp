// internal.hpp — host-side plumbing shared by the C-ABI translation units.
//
// The C entry points validate arguments on the host (so a bad shape becomes an
// LSSM_EINVAL, never an out-of-bounds kernel), launch on the context's stream,
// and then either return (inside a batch) or synchronise and check (outside),
// matching MetalOps' batched / one-shot split (ops.mm:82-149).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/lssm.h"

struct lssm_ctx {
    hipStream_t stream = nullptr;
    bool own_stream = false;
    bool batch = false;
    int device = 0;
    // Device status word (LSSM_STATUS_* bits, OR-ed by kernels that detect a
    // condition they cannot report otherwise) and its pinned host mirror; read
    // and cleared at every synchronisation point of the context.
    uint32_t* status = nullptr;
    uint32_t* status_host = nullptr;
    uint32_t debug = 0;      // LSSM_DEBUG_* switches (lssm_ctx_set_debug)
    // segment workspace of the chunked scan (lssm::ssd_seg_floats() floats),
    // allocated by the first lssm_ssd_chunked call that can use it
    float* ssd_seg = nullptr;
    // Gram tiles of lssm_ssd_chunked (lssm::ssd_gram_floats), grown on demand
    // to at least twice the last size.  A grown-out buffer is kept until
    // lssm_ctx_destroy: a graph captured on this stream may hold its address.
    float* ssd_gram = nullptr;
    size_t ssd_gram_cap = 0;   // floats
    std::vector<float*> ssd_gram_retired;
};

namespace lssm {

// Compute units of the current device (queried once per process).
uint32_t num_cus();

// thread-local error message (lssm_last_error)
int set_error(int code, const char* fmt, ...);
void clear_error();

// Bits of lssm_ctx::status.
constexpr uint32_t STATUS_BAD_TOKEN = 1u;      // a token id outside [0, vocab) reached the embedding
constexpr uint32_t STATUS_WAIT_TIMEOUT = 2u;   // a cross-workgroup wait gave up (not co-resident)

// After enqueueing an op: report launch errors; outside a batch, also wait and
// report asynchronous kernel failures and the device status word.
int finish(lssm_ctx* ctx, const char* what);
// Wait for the context's stream; report a HIP error or a status bit set by a
// kernel since the last check (and clear it).
int sync_and_check(lssm_ctx* ctx, const char* what);

// Dynamic LDS of the GEMV x staging (fp32 rows); static + dynamic stays <= 64 KiB.
constexpr size_t GEMV_LDS_BYTES = 60 * 1024;

inline size_t dtype_size(int act) { return act == LSSM_F32 ? 4 : 2; }
inline bool valid_act(int act) { return act == LSSM_F16 || act == LSSM_BF16 || act == LSSM_F32; }
inline bool valid_wfmt(int f) {
    return f == LSSM_W_DENSE || f == LSSM_W_Q4_B32 || f == LSSM_W_Q4_G64 || f == LSSM_W_Q8_G32;
}
inline uint32_t wfmt_group(int f) {
    return f == LSSM_W_Q4_G64 ? 64u : (f == LSSM_W_DENSE ? 0u : 32u);
}

#define LSSM_CHECK_CTX(ctx)                                                 \
    do {                                                                    \
        if (!(ctx)) return ::lssm::set_error(LSSM_EINVAL, "null lssm_ctx"); \
        ::lssm::clear_error();                                              \
    } while (0)

#define LSSM_REQUIRE(cond, ...)                                             \
    do {                                                                    \
        if (!(cond)) return ::lssm::set_error(LSSM_EINVAL, __VA_ARGS__);    \
    } while (0)

// ---------------------------------------------------------------------------
// Launchers (defined in the .hip files).  All return hipError_t of the launch.
// Row strides are in elements.
// ---------------------------------------------------------------------------
hipError_t launch_rmsnorm(hipStream_t s, const void* x, uint32_t x_stride, const void* w, void* y,
                          uint32_t y_stride, uint32_t rows, uint32_t dim, float eps, int act);
hipError_t launch_gated_rmsnorm(hipStream_t s, const void* z, uint32_t z_stride, const void* y,
                                uint32_t y_stride, const void* w, void* out, uint32_t rows,
                                uint32_t dim, float eps, int act);
hipError_t launch_silu(hipStream_t s, const void* x, void* y, uint32_t n, int act);
hipError_t launch_add(hipStream_t s, void* y, const void* x, uint32_t n, int act);
hipError_t launch_silu_gated(hipStream_t s, const void* x, const void* g, void* y, uint32_t n,
                             int act);
hipError_t launch_split_silu(hipStream_t s, const void* xBC, void* x, void* B, void* C,
                             uint32_t rows, uint32_t d_inner, uint32_t GN, int act);
// hist (one sequence only): its conv state [D][K] as launch_conv1d_seed left
// it after the sequence's earlier tokens; rows before x are read from there
// instead of the zero padding (a prefill continued from an earlier part)
hipError_t launch_conv1d(hipStream_t s, const void* x, uint32_t x_stride, const void* w,
                         const void* bias, void* y, uint32_t y_stride, uint32_t B, uint32_t L,
                         uint32_t D, uint32_t K, int act, bool silu, const void* hist = nullptr);
hipError_t launch_conv1d_update(hipStream_t s, const void* x_new, void* state, const void* w,
                                const void* bias, void* y, uint32_t B, uint32_t D, uint32_t K,
                                int act);
hipError_t launch_conv1d_update_silu(hipStream_t s, const void* x_new, uint32_t x_stride,
                                     void* state, const void* w, const void* bias, void* y,
                                     uint32_t y_stride, uint32_t B, uint32_t D, uint32_t K, int act);
hipError_t launch_conv1d_keep_last(hipStream_t s, void* state, uint32_t n_windows, uint32_t K,
                                   int act);
hipError_t launch_conv1d_seed(hipStream_t s, const void* xBC, uint32_t x_stride, void* state,
                              uint32_t B, uint32_t L, uint32_t D, uint32_t K, int act);
// seq (optional): a step counter the kernel advances by one (the tag of the
// fused decode launch's words).
// An id outside [0, vocab) gives a zero row and sets STATUS_BAD_TOKEN in *status.
hipError_t launch_embed(hipStream_t s, const void* table, const int32_t* ids, void* out,
                        uint32_t n, uint32_t d_model, uint32_t vocab, int act, uint32_t* status,
                        uint32_t* seq = nullptr);
hipError_t launch_argmax(hipStream_t s, const void* logits, int32_t* ids, uint32_t rows,
                         uint32_t vocab, int act, void* scratch);
// ids[0] = the first index of the maximum over *nblk partials (pv, pi)
hipError_t launch_argmax_final(hipStream_t s, const float* pv, const int* pi, const uint32_t* nblk,
                               int32_t* ids);

// appends next[0..B) as row *pos of log [cap][B] and advances *pos (B <= 64)
hipError_t launch_id_log(hipStream_t s, const int32_t* next, uint32_t B, int32_t* log, uint32_t cap,
                         uint32_t* pos);

// GEMV (M <= 4): optional RMSNorm prologue over each x row (norm_w != nullptr).
struct GemvArgs {
    const void* x;
    uint32_t x_stride;
    const void* w;
    const void* s;
    void* y;
    uint32_t y_stride;
    const void* res;
    const void* norm_w;
    float eps;
    uint32_t M, N, K;
    int wfmt, act, epi;
    // x rows as launch_mma_pack wrote them (norm_w applied), or null; used by
    // the MFMA decode GEMV, which then copies instead of normalising
    const void* xpack = nullptr;
    // with xpack in fragment order: xpack holds r(x norm_w) without the
    // rows' 1 / rms, which the GEMV forms from their partial sums of squares
    // of x ([rows][nparts], added in order) and applies to its fp32 sums;
    // null: xpack is normalised
    const float* xpart = nullptr;
    uint32_t nparts = 0;
    // epi == LSSM_EPI_ADD, single-pass MFMA GEMV only (gemv_mmx_parts): the
    // output rows h also as r(h ynorm_w) in fragment order for the next GEMV
    // (yfrag, ceil(M / 16) * 16 rows of N) and each row's sum of squares of h
    // over every 16 columns (ypart, [rows][N / 16]); null: y only
    void* yfrag = nullptr;
    float* ypart = nullptr;
    const void* ynorm_w = nullptr;
};
hipError_t launch_gemv(hipStream_t s, const GemvArgs& a);
// One row of logits (dense weights, epi none) and its greedy id: the GEMV's
// blocks write the logits and each block's (max, first index) into scratch,
// then one block reduces them into ids[0].  hipErrorNotSupported: the shape
// or scratch does not allow it (the caller runs launch_gemv + launch_argmax).
hipError_t launch_gemv_argmax(hipStream_t s, const GemvArgs& a, int32_t* ids, void* scratch,
                              size_t scratch_bytes);
// Rows of x one GEMV launch can take for this K / format (0 = none), with
// 16-byte aligned operands / with any alignment.
int gemv_max_rows(uint32_t K, int wfmt, int act);
int gemv_lds_rows(uint32_t K, int wfmt, int act);

hipError_t launch_dequant(hipStream_t s, const void* w, const void* sc, float* out, uint32_t N,
                          uint32_t K, int wfmt);

// MFMA GEMM for fp16 / bf16 activations, K % 64 == 0.
struct GemmArgs {
    const void* x;
    uint32_t x_stride;
    const void* w;
    const void* s;
    void* y;
    uint32_t y_stride;
    const void* res;
    uint32_t M, N, K;
    int wfmt, act, epi;
    int round_dequant;   // gemm_simple only: 1 = GEMM semantics, 0 = exact (GEMV)
    // prefill GEMM, optional: fp32 workspace of ws_floats floats; a grid of
    // few tiles then splits K into slices whose sums a second launch adds
    float* ws = nullptr;
    size_t ws_floats = 0;
    // prefill GEMM, optional: each output row's sums are scaled by
    // row_scale[row] before the epilogue (the RMSNorm's 1 / rms of an input
    // stored as r(x w)); null: no scale
    const float* row_scale = nullptr;
    // prefill GEMM, optional: outputs of columns n < silu_cols are r(silu(v))
    // (SiLU with the hardware exp and reciprocal) instead of r(v); 0: none
    uint32_t silu_cols = 0;
    // prefill GEMM with the residual add, optional (where gemm_norm_fold_takes
    // says so): the next RMSNorm's input folded into the epilogue.  Besides
    // y = r(res + r(v)) it writes y2 = r(y norm_w) (row stride y_stride) and
    // each row's sum of y^2 over every 128 columns to
    // y2_part[n / 128][M]; the GEMM that reads y2 then scales its sums by the
    // row's 1 / rms (row_scale, from launch_rms_from_parts)
    void* y2 = nullptr;
    const void* y2_w = nullptr;
    float* y2_part = nullptr;
};
// Whether launch_gemm runs a (with y2 set) through the epilogue that writes y2
// and y2_part: bf16 / f16, the residual add, M > 128 without a K split,
// N % 128 == 0, 16-byte aligned rows.  launch_gemm refuses y2 elsewhere.
bool gemm_norm_fold_takes(const GemmArgs& a);
hipError_t launch_gemm(hipStream_t s, const GemmArgs& a);
// Workspace the engine gives launch_gemm for its split-K slices (floats).
// The 130M prefill of 2048 tokens (config 3) runs its out_proj in four slices
// plus the sum: 2.60 -> 2.45 ms for the whole prefill; the same GEMM alone
// through lssm_linear (no workspace) measures 23.9 us unsplit against 26.5 us
// split, so the generic entry keeps the single launch.
constexpr size_t GEMM_WS_FLOATS = (size_t)8 << 20;   // 32 MiB
// Simple fp32 (or any dtype) reference-layout GEMM used for F32 activations.
hipError_t launch_gemm_simple(hipStream_t s, const GemmArgs& a);

// SSD.  Strides are row strides in elements of the [.., L, ...] tensors.
struct SsdArgs {
    const void* X;  uint32_t x_stride;   // row = one token: H*P elements (packed)
    const void* B;  uint32_t b_stride;   // row = one token: G*N
    const void* C;  uint32_t c_stride;
    const void* dt; uint32_t dt_stride;  // row = one token: H
    const void* dt_bias;
    const void* A_log;
    const void* D;
    void* Y;        uint32_t y_stride;
    float* state;
    uint32_t batch, L, H, P, N, G, chunk;
    float dt_min, dt_max;
    uint32_t has_D;
    int act;
    // optional gate (decode engine): Y = r(silu(z) * r(y)); z row stride
    const void* z;  uint32_t z_stride;
    // chunked scan, optional: scratch of ssd_gram_floats(batch, L, G) floats for
    // the chunks' C B^T Gram tiles, computed once per (sequence, chunk, group)
    // and shared by the group's heads (null: every head computes its own)
    float* gram = nullptr;
    // chunked scan, optional: workspace of ssd_seg_floats() floats with which
    // a grid of fewer blocks than the chip holds splits every sequence into
    // segments of chunks that run in parallel (null: one serial walk per
    // sequence, head and column block)
    float* seg = nullptr;
    // set by the launcher: segments per sequence and chunks per segment
    uint32_t nseg = 1, seg_chunks = 0;
    // decode step, bf16 with gate, H * P a multiple of 128 (ssd_step_parts):
    // Y rows also as r(Y ynorm_w) in the single-pass MFMA GEMV's fragment
    // order (yfrag, ceil(batch / 16) * 16 rows) and each row's sum of squares
    // of Y over every 32 elements (ypart, [rows][H P / 32]); null: Y only
    void* yfrag = nullptr;
    float* ypart = nullptr;
    const void* ynorm_w = nullptr;
    // chunked scan, optional (where ssd_chunked_gate_parts says it applies):
    // the gated RMSNorm's gate and weight fused into the Y stores,
    //   Y = r(g gnorm_w),  g = r(silu(z) r(y)),  z = a.z (row stride z_stride),
    // and every token's sum of g^2 over each block's columns into
    // gpart[part][batch L] (part = h * (P / PB) + pb, ssd_chunked_gate_parts(a) of them);
    // the 1 / rms scale is then applied by the GEMM that reads Y
    const void* gnorm_w = nullptr;
    float* gpart = nullptr;
    // z already holds r(silu(z)) (the projection's GEMM applied it), so
    // g = r(z r(y)); the fused gate is taken only then
    bool z_silu = false;
};
hipError_t launch_ssd_step(hipStream_t s, const SsdArgs& a);
// Partials per row a decode step with SsdArgs::yfrag writes (H P / 32), or 0
// when it cannot.
uint32_t ssd_step_parts(uint32_t H, uint32_t P, uint32_t N, int act);
hipError_t launch_ssd_chunked(hipStream_t s, const SsdArgs& a);
// Partial sums of squares per row that launch_ssd_chunked writes when a.gpart
// is set, or 0 where it cannot fuse the gate (not the MFMA walk).
uint32_t ssd_chunked_gate_parts(const SsdArgs& a);
// rs[row] = 1 / sqrt(sum of part[0 .. nparts)[row] / dim + eps), part[k] a
// column of `rows` floats
hipError_t launch_rms_from_parts(hipStream_t s, const float* part, uint32_t nparts, uint32_t rows,
                                 uint32_t dim, float eps, float* rs);
inline size_t ssd_gram_floats(uint32_t batch, uint32_t L, uint32_t G) {
    return (size_t)batch * ((L + 63) / 64) * G * 64 * 64;
}
// Segment workspace: the states of [batch][segment][H][P][N] (fp32) and the
// segments' log-decays [batch][segment][H]; the launcher takes only as many
// segments as fit.
constexpr size_t SSD_SEG_STATE_FLOATS = (size_t)512 * 64 * 128;   // 16 MiB
constexpr size_t SSD_SEG_DECAY_FLOATS = 4096;
inline size_t ssd_seg_floats() { return SSD_SEG_STATE_FLOATS + SSD_SEG_DECAY_FLOATS; }

hipError_t launch_inproj_fused(hipStream_t s, const void* normed, const void* W_in,
                               const void* W_conv, const void* conv_b, void* proj_z, void* ssd_x,
                               void* ssd_B, void* ssd_C, void* proj_dt, void* proj_xBC,
                               lssm_fused_inproj_dims d);

// Engine decode in_proj: GEMV with RMSNorm prologue whose epilogue routes rows
// to z / (conv update + SiLU -> xbc_act) / dt.
struct InprojDecodeArgs {
    GemvArgs g;           // y unused; res unused
    uint32_t d_inner, xbc, H, dconv;
    void* conv_state;     // [B, xbc, dconv] for this layer
    const void* conv_w;   // [xbc, dconv]
    const void* conv_b;   // [xbc]
    void* z;              // [B, d_inner]
    void* xbc_act;        // [B, xbc]
    void* dt;             // [B, H]
};
hipError_t launch_inproj_decode(hipStream_t s, const InprojDecodeArgs& a);

// Engine decode at batch 1: launch_inproj_decode's rows, published as tagged
// words, and the layer's SSD step + SiLU(z) gate (ssd_step_kernel's
// arithmetic) in the same launch; z / xbc_act / dt of `a` are not written.
// Returns false (launching nothing) when the shape, format, alignment or grid
// is not one it takes; err holds the launch result.
struct SsdFuseArgs {
    uint64_t* xfer;          // [proj] tagged words of this layer (zeroed once)
    const uint32_t* seq;     // step tag in device memory, advanced once per decode
                             // step (launch_embed); null: `tag` below
    uint32_t tag;
    float* state;            // [H, P, N] fp32
    const void* A_log;
    const void* dt_bias;
    const void* D;           // may be null
    void* y;                 // [d_inner]
    uint32_t P, N, G;
    float dt_min, dt_max;
    uint32_t* status;        // STATUS_WAIT_TIMEOUT when a wait gives up (that item's
                             // state is then left as it was, its outputs NaN)
    uint32_t wait_skew = 0;  // 1: the SSD items wait for a tag that is never published,
                             // so every bounded wait gives up (LSSM_DEBUG_STALE_WAIT)
};
bool launch_inproj_ssd_decode(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseArgs& f, hipError_t& err);
// The whole mixer of a layer at batch 1 in one launch: launch_inproj_ssd_decode
// with the gated SSD outputs as tagged words in `yx`, then the gated-RMSNorm +
// out_proj + residual add of the separate out_proj launch (bit-identical to
// it), hidden rewritten in place (`hidden` must be the in_proj input).  Same
// weight format for both projections; returns false (launching nothing) for
// shapes it is not built for.
struct OutprojFuseArgs {
    const void* w;           // out_proj [N, d_inner]
    const void* s;
    const void* norm_w;      // mixer norm weight [d_inner]
    float eps;
    void* hidden;            // [N] residual in, hidden out
    uint32_t* yx;            // [d_inner] tagged words of this layer: value | (tag mod 2^16) << 16
    uint32_t N;              // d_model
};
bool launch_layer_decode(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseArgs& f, const OutprojFuseArgs& o,
                         hipError_t& err);

// MFMA GEMV for decode batches (gemv_mma.hip): 2..64 rows, GEMV rule, RMSNorm
// prologue when norm_w is set.  Returns false (launching nothing) when the
// shape, format or alignment is not one it takes; err holds the launch result.
bool launch_gemv_mma(hipStream_t s, const GemvArgs& a, hipError_t& err);
bool launch_inproj_decode_mma(hipStream_t s, const InprojDecodeArgs& a, hipError_t& err);
// Engine decode at batch 2..16 with x packed in fragment order with partial
// sums (a.g.xpack, a.g.xpart): launch_inproj_decode_mma's rows published as
// tagged words, then the layer's SSD step + SiLU(z) gate with the outputs of
// launch_ssd_step's fragment variant (y, r(y ynorm_w) in yfrag, sums of y^2 in
// ypart), in one launch; z / xbc_act / dt of `a` are not written.  Returns
// false (launching nothing) for shapes, formats or grids it does not take.
struct SsdFuseBArgs {
    uint64_t* xfer;          // [M][proj] tagged words of this layer (zeroed once)
    const uint32_t* seq;     // step tag in device memory, advanced once per decode step
    float* state;            // [M][H][P][N] fp32
    const void* A_log;
    const void* dt_bias;
    const void* D;           // may be null
    void* y;                 // [M][d_inner]
    void* yfrag;             // r(y ynorm_w) in the single-pass GEMV's fragment order
    float* ypart;            // [M][H P / 32]
    const void* ynorm_w;
    uint32_t P, N, G;
    float dt_min, dt_max;
    uint32_t* status;        // STATUS_WAIT_TIMEOUT when a wait gives up
    uint32_t wait_skew = 0;  // 1: wait for a tag that is never published
};
bool launch_inproj_ssd_decode_mma(hipStream_t s, const InprojDecodeArgs& a, const SsdFuseBArgs& f,
                                  hipError_t& err);
// Whether a decode batch of M rows runs in one MFMA launch (16-byte aligned
// operands assumed; otherwise the launchers fall back to gemv1 launches).
bool gemv_mma_takes(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act);
// RMSNorm of M rows of x (K, 16-bit act), rounded and packed in the MFMA
// decode GEMV's staging order for `wfmt`, into out ([M][K / 2] dwords): one
// pass for all blocks of the GEMV launch that follows (GemvArgs::xpack).
hipError_t launch_mma_pack(hipStream_t s, const void* x, uint32_t x_stride, const void* norm_w,
                           float eps, uint32_t M, uint32_t K, int wfmt, int act, void* out,
                           bool frag = false, float* part = nullptr);
// (with frag and part set, the rows are written as r(x norm_w), without
// 1 / rms, and row m's sum of squares goes to part[4 m], zeros to part[4 m +
// 1 .. 4 m + 3]: four partials a row, for the GEMV that scales its sums by
// 1 / rms (GemvArgs::xpart); rows up to ceil(M / 16) * 16)
// The MFMA decode GEMV takes (M, N, K) in its single-pass form, which reads x
// packed in fragment order (launch_mma_pack with frag = true; the buffer then
// holds ceil(M / 16) * 16 rows).
bool gemv_mmx_takes(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act);
// Partials per row (N / 16) the single-pass MFMA GEMV writes for (M, N, K)
// with GemvArgs::yfrag, or 0 when it cannot (another plan, or a count the
// GEMV that reads them does not take).
uint32_t gemv_mmx_parts(uint32_t M, uint32_t N, uint32_t K, int wfmt, int act);
// Most partial sums of squares a row the single-pass MFMA GEMV reads.
constexpr uint32_t GEMV_MAX_XPARTS = 256;

}  // namespace lssm

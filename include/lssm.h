/*
 * lssm.h — C ABI of the MI355X (gfx950) Mamba-2 inference backend.
 *
 * This is the drop-in boundary that replaces the Metal backend of lite-ssm
 * (src/backend/metal/ops.mm and the shaders/ directory).  Every entry point takes plain
 * device pointers and sizes; nothing here names a torch or Metal type.
 *
 *   - Each reference dispatcher `MetalOps::<op>` (include/lite_ssm/ops.hpp:99-235)
 *     has a same-named `lssm_<op>` entry below with the same argument meaning.
 *     A MetalOps (handle, byte_offset) pair becomes one pointer, handle + offset.
 *   - The generic entries (`lssm_linear`, `lssm_ssd_chunked`, ...) add what the
 *     reference cannot express: a batch dimension, bf16/fp32 activations, and
 *     the Q4_G64 / Q8_G32 weight formats.  The reference-named entries are thin
 *     wrappers over them with batch 1, fp16 activations and INT4_B32 weights.
 *   - The engine entries (`lssm_engine_*`) run the whole per-layer op sequence
 *     of Mamba2Model::run_block (src/model/mamba2_block.cpp:51-290) with fused
 *     kernels, device-side embedding and argmax, and HIP-graph replay.
 *
 * Error model: every call returns an `int` status (LSSM_OK == 0).  On failure a
 * thread-local message is available from lssm_last_error(); the C++ shim
 * (include/lite_ssm/ops.hpp) rethrows it as std::runtime_error, mirroring the
 * reference's throw sites (ops.mm:39-45, 83-85, 96-98, 107-110, 144-147).
 *
 * Execution model: every op is enqueued on the stream owned (or borrowed) by
 * the lssm_ctx.  Outside a batch an op is synchronous (launch + stream sync +
 * error check), like the reference's one-shot command buffer (ops.mm:131-148).
 * Inside lssm_begin_batch / lssm_commit_and_wait ops only enqueue
 * (ops.mm:82-112).
 */
#ifndef LSSM_H
#define LSSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------- */
/* Status, dtypes, formats                                                    */
/* ------------------------------------------------------------------------- */
enum {
    LSSM_OK        = 0,
    LSSM_EINVAL    = 1,  /* bad argument / dimension precondition            */
    LSSM_EDEVICE   = 2,  /* HIP runtime or kernel failure                    */
    LSSM_ESTATE    = 3,  /* batch misuse (begin twice, commit without begin) */
    LSSM_ENOTFOUND = 4   /* unknown kernel name or tensor name              */
};

/* Activation dtypes.  Codes match the .ssm dtype codes
 * (include/lite_ssm/ssm_format.hpp:29-41): F16 = 0, BF16 = 1, F32 = 2. */
typedef enum { LSSM_F16 = 0, LSSM_BF16 = 1, LSSM_F32 = 2 } lssm_dtype;

/* Weight formats of a (N x K) row-major linear weight.
 *   DENSE  : N*K elements of the activation dtype.
 *   Q4_B32 : the reference DTYPE_INT4_B32 (ssm_format.hpp:36-43, 64-69):
 *            [N*K/2 packed nibbles][N*K/32 fp16 scales]; low nibble = even k.
 *   Q4_G64 : same layout, 64-element groups  -> [N*K/2][N*K/64 fp16].
 *   Q8_G32 : int8 two's complement, 32-element groups -> [N*K][N*K/32 fp16].
 * Q4_G64 and Q8_G32 are this build's extension codes (7 and 8). */
typedef enum {
    LSSM_W_DENSE  = 0,
    LSSM_W_Q4_B32 = 6,
    LSSM_W_Q4_G64 = 7,
    LSSM_W_Q8_G32 = 8
} lssm_wfmt;

/* Epilogue applied to a linear output before the single rounding store.
 *   NONE : y = r(acc)
 *   SILU : y = r(silu(acc))
 *   ADD  : y = r(residual + r(acc))   (out_proj + residual add, activations.metal:24-32)
 * r() rounds to the activation dtype. */
typedef enum { LSSM_EPI_NONE = 0, LSSM_EPI_SILU = 1, LSSM_EPI_ADD = 2 } lssm_epilogue;

typedef struct lssm_ctx lssm_ctx;

/* ------------------------------------------------------------------------- */
/* Dims structs: field-for-field the reference's (ops.hpp:30-55, 193-202)     */
/* ------------------------------------------------------------------------- */
typedef struct { uint32_t M, N, K; } lssm_linear_dims;                 /* LinearDims    */
typedef struct { uint32_t rows, dim; float eps; } lssm_rmsnorm_dims;   /* RMSNormDims   */
typedef struct { uint32_t N, K; float eps; } lssm_rms_linear_dims;     /* RMSLinearDims */
typedef struct { uint32_t B, L, D, K; } lssm_conv1d_dims;              /* Conv1dDims    */
typedef struct {                                                       /* SSDDims       */
    uint32_t L, H, P, N, n_groups, chunk_size;
    float dt_min, dt_max;
    uint32_t has_D;
} lssm_ssd_dims;
typedef struct {                                                       /* SSDStepDims   */
    uint32_t H, P, N, n_groups;
    float dt_min, dt_max;
    uint32_t has_D;
} lssm_ssd_step_dims;
typedef struct {                                        /* MetalOps::FusedInProjDims */
    uint32_t L, d_model, d_inner, d_state, n_groups, n_heads, d_conv, proj_dim;
} lssm_fused_inproj_dims;

/* ------------------------------------------------------------------------- */
/* Context, batching, introspection                                           */
/* ------------------------------------------------------------------------- */
const char* lssm_last_error(void);

/* `stream` = an existing hipStream_t to borrow, or NULL to create one.
 * Replaces MetalOps::MetalOps() (ops.mm:62) and the queue singleton
 * (metal_context.mm:25-70). */
int lssm_ctx_create(lssm_ctx** out, void* stream);
int lssm_ctx_destroy(lssm_ctx* ctx);
int lssm_ctx_stream(lssm_ctx* ctx, void** stream_out);

int lssm_begin_batch(lssm_ctx* ctx);       /* MetalOps::begin_batch   ops.hpp:91 */
int lssm_commit_and_wait(lssm_ctx* ctx);   /* MetalOps::commit_and_wait ops.hpp:92 */
int lssm_batch_active(lssm_ctx* ctx);      /* MetalOps::batch_active  ops.hpp:93 */
int lssm_sync(lssm_ctx* ctx);              /* stream sync + error check          */

/* Every synchronisation point of a context (lssm_sync, lssm_commit_and_wait,
 * and any op outside a batch) also reads a device status word that kernels
 * set for conditions they cannot report otherwise, and clears it:
 *   - a token id outside [0, vocab) reached the embedding (ids live in device
 *     memory, so the check of mamba2_model.cpp:129-131 runs there):
 *     LSSM_EINVAL, "Mamba2Model::embed: token_id out of range";
 *   - a bounded cross-workgroup wait of a fused decode launch gave up (its
 *     workgroups were not all resident at once): LSSM_EDEVICE; the affected
 *     outputs are NaN and their SSD state is left as it was, but the conv
 *     state has advanced by the step's token (the window shift happens in the
 *     in_proj epilogue, before any wait), so the step must not be retried on
 *     the same state.
 *   Both conditions in one step report LSSM_EINVAL with both texts.
 *
 * Failure-injection switches for the tests of these paths (no counterpart in
 * the reference; 0 = off, the default).  LSSM_DEBUG_STALE_WAIT makes the SSD
 * items of lssm_inproj_ssd_decode wait for a tag that no workgroup publishes,
 * so every bounded wait gives up and the kernel still exits normally. */
#define LSSM_DEBUG_STALE_WAIT 1u
int lssm_ctx_set_debug(lssm_ctx* ctx, uint32_t flags);

/* MetalOps::metallib_loaded / has_pipeline / metallib_path (ops.hpp:66-74). */
int lssm_library_loaded(void);
int lssm_has_kernel(const char* name);
const char* lssm_library_path(void);
int lssm_kernel_count(void);
const char* lssm_kernel_name(int i);

/* Device memory plumbing (DeviceBuffer bodies, metal_buffer.mm:107-143).
 * lssm_malloc: HBM (DeviceBuffer's storage, and UnifiedBuffer's copy of the
 * weights).  lssm_malloc_host: pinned, coherent host memory that kernels
 * read and write in place over PCIe, for callers that want one address on
 * both sides; release it with lssm_free_host. */
int lssm_malloc(void** out, size_t nbytes);
int lssm_malloc_host(void** out, size_t nbytes);
int lssm_free(void* p);
int lssm_free_host(void* p);
int lssm_memcpy_h2d(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes);
int lssm_memcpy_d2h(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes);
int lssm_memcpy_d2d(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes);
int lssm_memset(lssm_ctx* ctx, void* dst, int value, size_t nbytes);

/* ------------------------------------------------------------------------- */
/* Reference-named ops (fp16 activations, batch 1): one per MetalOps method    */
/* ------------------------------------------------------------------------- */
/* ops.hpp:99-102 */
int lssm_rmsnorm_f16(lssm_ctx* ctx, const void* x, const void* w, void* y,
                     lssm_rmsnorm_dims dims);
/* ops.hpp:104-107 */
int lssm_linear_f16_gemv(lssm_ctx* ctx, const void* x, const void* w, void* y,
                         lssm_linear_dims dims);
/* ops.hpp:109-112 */
int lssm_linear_silu_f16_gemv(lssm_ctx* ctx, const void* x, const void* w, void* y,
                              lssm_linear_dims dims);
/* ops.hpp:114-118 */
int lssm_rmsnorm_linear_f16_gemv(lssm_ctx* ctx, const void* x, const void* w_norm,
                                 const void* w, void* y, lssm_rms_linear_dims dims);
/* ops.hpp:120-123 */
int lssm_linear_f16_gemm(lssm_ctx* ctx, const void* x, const void* w, void* y,
                         lssm_linear_dims dims);
/* ops.hpp:125-128 */
int lssm_linear_silu_f16_gemm(lssm_ctx* ctx, const void* x, const void* w, void* y,
                              lssm_linear_dims dims);
/* ops.hpp:135-139 */
int lssm_linear_int4_gemv(lssm_ctx* ctx, const void* x, const void* w_packed,
                          const void* w_scales, void* y, lssm_linear_dims dims);
/* ops.hpp:141-145 */
int lssm_linear_int4_gemm(lssm_ctx* ctx, const void* x, const void* w_packed,
                          const void* w_scales, void* y, lssm_linear_dims dims);
/* ops.hpp:147-149 */
int lssm_silu_f16(lssm_ctx* ctx, const void* x, void* y, uint32_t n);
/* ops.hpp:151-153 */
int lssm_add_inplace_f16(lssm_ctx* ctx, void* y, const void* x, uint32_t n);
/* ops.hpp:158-163 */
int lssm_split_silu_xBC_f16(lssm_ctx* ctx, const void* xBC, void* x_out, void* B_out,
                            void* C_out, uint32_t L, uint32_t d_inner, uint32_t d_state,
                            uint32_t n_groups);
/* ops.hpp:165-168 */
int lssm_silu_gated_f16(lssm_ctx* ctx, const void* x, const void* gate, void* y, uint32_t n);
/* ops.hpp:170-174 */
int lssm_causal_conv1d_f16(lssm_ctx* ctx, const void* x, const void* w, const void* bias,
                           void* y, lssm_conv1d_dims dims);
/* ops.hpp:176-181 */
int lssm_causal_conv1d_update_f16(lssm_ctx* ctx, const void* x_new, void* state,
                                  const void* w, const void* bias, void* y,
                                  lssm_conv1d_dims dims);
/* ops.hpp:186-188 */
int lssm_seed_conv_state_f16(lssm_ctx* ctx, const void* xBC, void* state,
                             uint32_t L, uint32_t D, uint32_t K);
/* ops.hpp:203-213 */
int lssm_inproj_fused_f16(lssm_ctx* ctx, const void* normed, const void* W_in,
                          const void* W_conv, const void* conv_b, void* proj_z,
                          void* ssd_x, void* ssd_B, void* ssd_C, void* proj_dt,
                          void* proj_xBC, lssm_fused_inproj_dims dims);
/* ops.hpp:215-224 */
int lssm_ssd_chunked_f16(lssm_ctx* ctx, const void* X, const void* B, const void* C,
                         const void* dt_raw, const void* dt_bias, const void* A_log,
                         const void* D_skip, void* Y, float* state_io, lssm_ssd_dims dims);
/* ops.hpp:226-235 */
int lssm_ssd_step_f16(lssm_ctx* ctx, const void* x, const void* B, const void* C,
                      const void* dt_raw, const void* dt_bias, const void* A_log,
                      const void* D_skip, float* state, void* y, lssm_ssd_step_dims dims);

/* ------------------------------------------------------------------------- */
/* Generic ops (batch / dtype / format aware)                                 */
/* ------------------------------------------------------------------------- */
/* y[rows,dim] = r(x * w * rsqrt(mean(x^2) + eps))            norm.metal:52-79 */
int lssm_rmsnorm(lssm_ctx* ctx, const void* x, const void* w, void* y,
                 uint32_t rows, uint32_t dim, float eps, lssm_dtype act);

/* Y[M,N] = epi(X[M,K] . deq(W)[N,K]^T).  `w_scales` is ignored for DENSE.
 * `residual` is read only for EPI_ADD and may alias `y` (in-place residual).
 * M <= 4 runs the GEMV kernel (fp32 dequant, linear.metal:440-474 semantics);
 * larger M runs the MFMA GEMM, whose dequantized operand is rounded to the
 * activation dtype (linear.metal:538 semantics).  x_stride/y_stride are row
 * strides in elements (0 = packed). */
int lssm_linear(lssm_ctx* ctx, const void* x, uint32_t x_stride,
                const void* w, const void* w_scales,
                void* y, uint32_t y_stride, const void* residual,
                uint32_t M, uint32_t N, uint32_t K,
                lssm_wfmt wfmt, lssm_dtype act, lssm_epilogue epi);

/* Decode linear with the RMSNorm prologue, for 1..64 rows (one token of each
 * of `rows` sequences): y = epi(r(RMSNorm(x, norm_w, eps)) . deq(W)^T) with
 * the GEMV rule at every row count (exact dequantization, linear.metal:440-474),
 * as the reference decodes each sequence (mamba2_block.cpp:240-262: rmsnorm ->
 * linear gemv -> add_inplace; the engine's out_proj step).  `residual` may
 * alias `y` (EPI_ADD).  Rows are packed (stride K in, N out). */
int lssm_norm_linear_decode(lssm_ctx* ctx, const void* x, const void* norm_w, float eps,
                            const void* w, const void* w_scales, void* y, const void* residual,
                            uint32_t rows, uint32_t N, uint32_t K, lssm_wfmt wfmt,
                            lssm_dtype act, lssm_epilogue epi);

/* Bit-exact dequantization of a whole (N x K) weight into fp32 (debug/parity). */
int lssm_dequant(lssm_ctx* ctx, const void* w, const void* w_scales, float* out,
                 uint32_t N, uint32_t K, lssm_wfmt wfmt);

int lssm_silu(lssm_ctx* ctx, const void* x, void* y, uint32_t n, lssm_dtype act);
int lssm_add_inplace(lssm_ctx* ctx, void* y, const void* x, uint32_t n, lssm_dtype act);
int lssm_silu_gated(lssm_ctx* ctx, const void* x, const void* gate, void* y, uint32_t n,
                    lssm_dtype act);
int lssm_split_silu_xbc(lssm_ctx* ctx, const void* xBC, void* x_out, void* B_out,
                        void* C_out, uint32_t rows, uint32_t d_inner, uint32_t d_state,
                        uint32_t n_groups, lssm_dtype act);

/* Depthwise causal conv, x/y [B, L, D], w [D, K], bias [D], zero left pad. */
int lssm_conv1d(lssm_ctx* ctx, const void* x, const void* w, const void* bias, void* y,
                uint32_t B, uint32_t L, uint32_t D, uint32_t K, lssm_dtype act);
/* One decode step: x_new [B, D], state [B, D, K] (oldest first) updated in place. */
int lssm_conv1d_update(lssm_ctx* ctx, const void* x_new, void* state, const void* w,
                       const void* bias, void* y, uint32_t B, uint32_t D, uint32_t K,
                       lssm_dtype act);
/* state[b, d, k] = xBC[b, L-K+k, d] (0 where L-K+k < 0). */
int lssm_conv1d_seed(lssm_ctx* ctx, const void* xBC, void* state, uint32_t B, uint32_t L,
                     uint32_t D, uint32_t K, lssm_dtype act);

/* out = r(rmsnorm(r(silu(z) * y), w))  — gate-then-norm (mamba2_block.cpp:230-238). */
int lssm_gated_rmsnorm(lssm_ctx* ctx, const void* z, const void* y, const void* w,
                       void* out, uint32_t rows, uint32_t dim, float eps, lssm_dtype act);

/* Chunked SSD prefill over `batch` independent sequences of length dims.L.
 * X/Y [batch, L, H, P]; B/C [batch, L, G, N]; dt_raw [batch, L, H];
 * dt_bias/A_log/D [H] (act dtype); state [batch, H, P, N] fp32 in/out. */
int lssm_ssd_chunked(lssm_ctx* ctx, const void* X, const void* B, const void* C,
                     const void* dt_raw, const void* dt_bias, const void* A_log,
                     const void* D_skip, void* Y, float* state, uint32_t batch,
                     lssm_ssd_dims dims, lssm_dtype act);
/* One decode step for `batch` sequences: x [batch, H, P], B/C [batch, G, N],
 * dt_raw [batch, H], state [batch, H, P, N] fp32 updated in place. */
int lssm_ssd_step(lssm_ctx* ctx, const void* x, const void* B, const void* C,
                  const void* dt_raw, const void* dt_bias, const void* A_log,
                  const void* D_skip, float* state, void* y, uint32_t batch,
                  lssm_ssd_step_dims dims, lssm_dtype act);

/* Fused decode in_proj for batch <= 64 rows (the engine's first kernel of a
 * layer): normed = r(RMSNorm(hidden, norm_w)); proj = r(normed . deq(W)^T) over
 * all [z | xBC | dt] rows; z and dt rows are stored, each xBC row goes through
 * the conv-window update (conv1d.metal:108-137) and r(SiLU(r(conv))) into
 * xbc_act.  Same arithmetic as rmsnorm_f16 -> 3 x linear gemv ->
 * causal_conv1d_update_f16 -> split_silu_xBC_f16 (mamba2_block.cpp:84-177).
 * conv_state [batch, xBC_dim, d_conv]; z [batch, d_inner];
 * xbc_act [batch, xBC_dim]; dt [batch, n_heads]. */
int lssm_inproj_decode(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                       const void* w_scales, void* conv_state, const void* conv_w,
                       const void* conv_b, void* z, void* xbc_act, void* dt, uint32_t batch,
                       uint32_t d_model, uint32_t d_inner, uint32_t d_state, uint32_t n_groups,
                       uint32_t n_heads, uint32_t d_conv, float eps, lssm_wfmt wfmt,
                       lssm_dtype act);

/* Batch-1 decode of one layer's mixer input in ONE launch: lssm_inproj_decode
 * (batch 1) followed by the SSD step (lssm_ssd_step, ssd_step.metal:33-77) and
 * the SiLU(z) gate, y = r(silu(z) * r(C.S' + D x)).  The projection rows travel
 * between the launch's workgroups as 64-bit words (value | tag << 32) in
 * `xfer` ([d_inner + xBC_dim + n_heads] words, zeroed before its first use);
 * `tag` must differ from the tag of the previous call on the same `xfer`
 * (e.g. a step counter from 1).  ssd_state [n_heads, d_head, d_state] fp32 is
 * updated in place, conv_state as in lssm_inproj_decode; y [d_inner].
 * Takes d_state 128, d_head a multiple of 32, d_conv 4, fp16 / bf16, int4-g64
 * (or int8-g32 with fp16) weights, and grids of at most one workgroup per CU;
 * other shapes return LSSM_EINVAL (nothing runs).  No counterpart in the
 * reference, whose decode runs these ops as separate kernels
 * (mamba2_block.cpp:84-290). */
int lssm_inproj_ssd_decode(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                           const void* w_scales, void* conv_state, const void* conv_w,
                           const void* conv_b, const void* dt_bias, const void* A_log,
                           const void* D_skip, float* ssd_state, void* y, uint64_t* xfer,
                           uint32_t tag, uint32_t d_model, uint32_t d_inner, uint32_t d_state,
                           uint32_t n_groups, uint32_t n_heads, uint32_t d_head, uint32_t d_conv,
                           float eps, lssm_wfmt wfmt, lssm_dtype act);

/* lssm_inproj_ssd_decode that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops).  The projection's tagged words
 * and the step tag live in a static device array of the library (512 KiB +
 * 256 B, held by each GPU the library runs on until the process ends; zero at
 * load), and the tag is advanced on the device before each launch, so the
 * caller keeps no tag.  Shapes whose d_inner + xBC_dim + n_heads
 * exceeds 65536 projection rows are refused (LSSM_EINVAL), as are those the
 * fused launch does not take.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two threads) race on it. */
int lssm_inproj_ssd_decode_noalloc(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                                   const void* w_scales, void* conv_state, const void* conv_w,
                                   const void* conv_b, const void* dt_bias, const void* A_log,
                                   const void* D_skip, float* ssd_state, void* y, uint32_t d_model,
                                   uint32_t d_inner, uint32_t d_state, uint32_t n_groups, uint32_t n_heads,
                                   uint32_t d_head, uint32_t d_conv, float eps, lssm_wfmt wfmt,
                                   lssm_dtype act);

/* Batch-1 decode of one layer's whole mixer in ONE launch (in place on
 * `hidden` [d_model]): lssm_inproj_ssd_decode, then r(gated RMSNorm(y)) (the
 * mixer norm, norm.metal:52-79), out_proj and the residual add, hidden =
 * r(hidden + r(y_n . deq(W_out)^T)): bit-identical to lssm_inproj_ssd_decode ->
 * lssm_norm_linear_decode(..., EPI_ADD).  `xfer` holds d_inner + xBC_dim +
 * n_heads + d_inner 64-bit words (projection rows, then the gated SSD outputs
 * as 32-bit words carrying the tag modulo 2^16), zeroed before first use;
 * `tag` must differ from the previous call's tag on the same `xfer` modulo
 * 2^16 (a step counter does).  Both
 * projections use `wfmt`.  Takes the shapes of lssm_inproj_ssd_decode whose
 * (d_model, d_inner) it is built for: int4-g64 (2560, 5120) and (2048, 2048),
 * int8-g32 fp16 (768, 1536); others return LSSM_EINVAL (nothing runs).  No
 * counterpart in the reference (mamba2_block.cpp:84-290 runs these as
 * separate kernels). */
int lssm_mixer_decode(lssm_ctx* ctx, void* hidden, const void* norm_w, const void* in_w,
                      const void* in_scales, void* conv_state, const void* conv_w,
                      const void* conv_b, const void* dt_bias, const void* A_log,
                      const void* D_skip, float* ssd_state, const void* mixer_norm_w,
                      const void* out_w, const void* out_scales, uint64_t* xfer, uint32_t tag,
                      uint32_t d_model, uint32_t d_inner, uint32_t d_state, uint32_t n_groups,
                      uint32_t n_heads, uint32_t d_head, uint32_t d_conv, float eps,
                      lssm_wfmt wfmt, lssm_dtype act);

/* hidden[i, :] = table[ids[i], :]  (Mamba2Model::embed, mamba2_model.cpp:128-137). */
int lssm_embed(lssm_ctx* ctx, const void* table, const int32_t* ids, void* out,
               uint32_t n, uint32_t d_model, uint32_t vocab, lssm_dtype act);
/* ids[r] = first index of the max of logits[r, :]  (sampler.cpp:13-21). */
int lssm_argmax(lssm_ctx* ctx, const void* logits, int32_t* ids, uint32_t rows,
                uint32_t vocab, lssm_dtype act);

/* ------------------------------------------------------------------------- */
/* Engine: whole-model prefill / decode (configs 3-5)                         */
/* ------------------------------------------------------------------------- */
typedef struct {
    uint32_t d_model, n_layer, d_state, d_conv, expand, vocab_size;
    uint32_t n_heads, d_head, chunk_size, n_groups;
    uint32_t act;        /* lssm_dtype of activations and dense / 1-D params   */
    uint32_t wfmt;       /* lssm_wfmt of in_proj / out_proj                     */
} lssm_model_config;

/* Device pointers of one layer's tensors (names as in the .ssm file,
 * mamba2_model.cpp:62-116).  in_proj rows are [z | xBC | dt]. */
typedef struct {
    const void* norm_w;        /* [d_model]                     */
    const void* in_proj_w;     /* packed (or dense) [proj_dim, d_model] */
    const void* in_proj_s;     /* fp16 scales or NULL           */
    const void* conv1d_w;      /* [xBC_dim, d_conv]             */
    const void* conv1d_b;      /* [xBC_dim]                     */
    const void* dt_bias;       /* [n_heads]                     */
    const void* A_log;         /* [n_heads]                     */
    const void* D;             /* [n_heads]                     */
    const void* mixer_norm_w;  /* [d_inner]                     */
    const void* out_proj_w;    /* [d_model, d_inner]            */
    const void* out_proj_s;
} lssm_layer_weights;

typedef struct lssm_engine lssm_engine;

/* `layers` has cfg->n_layer entries; embed is [vocab, d_model], lm_head may
 * equal embed (tied).  The engine keeps the pointers (caller owns memory). */
int lssm_engine_create(lssm_engine** out, lssm_ctx* ctx, const lssm_model_config* cfg,
                       const void* embed, const void* norm_f, const void* lm_head,
                       const lssm_layer_weights* layers,
                       uint32_t max_batch, uint32_t max_seq);
int lssm_engine_destroy(lssm_engine* e);
/* Zero conv + SSD state of all sequences (Mamba2State::reset, state.cpp:49-51). */
int lssm_engine_reset(lssm_engine* e);
/* Prefill `batch` sequences of `L` token ids each (device int32 [batch, L]).
 * Writes last-position fp-act logits to the logits buffer and greedy ids to
 * `next_ids` (device int32 [batch]). */
int lssm_engine_prefill(lssm_engine* e, const int32_t* ids, uint32_t batch, uint32_t L,
                        int32_t* next_ids);
/* One decode step for `batch` sequences: reads ids (device int32 [batch]),
 * writes logits and greedy next ids (device, may alias ids). */
int lssm_engine_decode(lssm_engine* e, const int32_t* ids, uint32_t batch, int32_t* next_ids);
/* Capture `lssm_engine_decode(ids, batch, next_ids)` into a HIP graph (replaces
 * any earlier capture) and replay it `steps` times back to back. */
int lssm_engine_decode_graph(lssm_engine* e, const int32_t* ids, uint32_t batch,
                             int32_t* next_ids, uint32_t steps);
/* Device pointers to engine buffers (valid until destroy). */
int lssm_engine_logits(lssm_engine* e, void** logits);          /* [max_batch, vocab] act */
/* Parity hook, no counterpart in the reference (it is for layer-by-layer
 * comparisons against a CPU restatement of run_block).  With `buf` set, each
 * later lssm_engine_prefill / lssm_engine_decode copies the hidden rows
 * entering every layer, and the rows after the last layer, into `buf` as
 * [n_layer + 1][rows][d_model] in the activation dtype (rows = batch * L for a
 * prefill, batch for a decode step); a call whose rows do not fit `bytes` is
 * refused (LSSM_EINVAL).  buf = NULL turns it off.  Not combinable with
 * lssm_engine_decode_graph. */
int lssm_engine_set_trace(lssm_engine* e, void* buf, uint64_t bytes);
/* Greedy-id history, the counterpart of the id vector generate() returns
 * (runtime/inference.cpp:55-67).  With `buf` set, every later decode step
 * (lssm_engine_decode and each step replayed by lssm_engine_decode_graph)
 * appends its `batch` greedy ids as the next row of `buf` (device int32
 * [cap_steps][batch]); steps past cap_steps are not stored.  Setting it
 * restarts at row 0 and drops captured decode graphs; buf = NULL turns it
 * off.  Off by default: it adds one small kernel per step. */
int lssm_engine_set_id_log(lssm_engine* e, int32_t* buf, uint32_t cap_steps);
int lssm_engine_state(lssm_engine* e, void** conv_state, void** ssd_state);
/* conv_state: [n_layer, max_batch, xBC_dim, d_conv] act; ssd: [n_layer, max_batch, H, P, N] f32 */
/* Layers of the last decode step (eager or captured) whose SSD step ran inside
 * the in_proj launch (ssd_fused), and of those, layers whose whole mixer
 * (in_proj .. SSD step .. out_proj + residual) ran as one launch (mixer_fused).
 * Batch 1 only; the environment variable LSSM_FUSED_SSD=0 at engine creation
 * turns both off.  Either pointer may be null.  No counterpart in the
 * reference, whose decode runs every op as its own kernel. */
int lssm_engine_fused_layers(lssm_engine* e, uint32_t* ssd_fused, uint32_t* mixer_fused);

/* ------------------------------------------------------------------------- */
/* .ssm weight files                                                          */
/* ------------------------------------------------------------------------- */
/* The on-disk format of include/lite_ssm/ssm_format.hpp: a 96-byte header,
 * n_tensors index entries (32-byte prefix, u64 shape[rank], name bytes, padded
 * to 8), payloads at 64-byte aligned absolute offsets, all little-endian.
 * Tensor dtype codes 0-6 are the reference's (ssm_format.hpp:29-41); 7 and 8
 * are this build's block formats, laid out like DTYPE_INT4_B32 (packed values
 * of the whole tensor, then its fp16 scales):
 *   LSSM_DTYPE_Q4_G64: [numel/2 nibble bytes][numel/64 fp16 scales]
 *   LSSM_DTYPE_Q8_G32: [numel int8 bytes]    [numel/32 fp16 scales]        */
enum {
    LSSM_DTYPE_F16 = 0, LSSM_DTYPE_BF16 = 1, LSSM_DTYPE_F32 = 2, LSSM_DTYPE_I8 = 3,
    LSSM_DTYPE_U8 = 4, LSSM_DTYPE_I32 = 5, LSSM_DTYPE_INT4_B32 = 6,
    LSSM_DTYPE_Q4_G64 = 7, LSSM_DTYPE_Q8_G32 = 8
};
#define LSSM_SSM_MAX_RANK 4   /* TENSOR_MAX_RANK (tensor.hpp:21) */

/* FileHeader (ssm_format.hpp:73-110) without magic and reserved words, plus
 * the file size.  The writer reads only the hyperparameter fields. */
typedef struct {
    uint32_t version, header_size, n_tensors;
    uint64_t index_offset, data_offset, file_size;
    uint32_t d_model, n_layer, d_state, d_conv, expand, vocab_size;
    uint32_t n_heads, d_head, chunk_size, default_dtype, n_groups, norm_before_gate;
} lssm_ssm_header;

/* One index entry (lite_ssm::Tensor, tensor.hpp:23-36). */
typedef struct {
    uint32_t dtype, rank;
    uint64_t shape[LSSM_SSM_MAX_RANK];  /* unused dims are 0 */
    uint64_t offset;                    /* absolute byte offset in the file */
    uint64_t nbytes;
    const void* host;                   /* payload inside the read-only mapping */
} lssm_ssm_tensor;

typedef struct lssm_ssm lssm_ssm;

/* Payload bytes of `numel` elements of `dtype`: dtype_packed_nbytes
 * (ssm_format.hpp:45-69) with codes 7 and 8 added; 0 for an unknown code. */
uint64_t lssm_ssm_packed_nbytes(uint32_t dtype, uint64_t numel);

/* Map `path` read-only and validate header and index with the checks and
 * messages of SSMFile::SSMFile (src/core/ssm_loader.cpp:46-138): size, magic,
 * version, header_size, offsets, rank, in-bounds shape / name / payload, packed
 * size, duplicate names, index overrunning data_offset.  LSSM_EINVAL on a bad
 * file, LSSM_EDEVICE (errno text) when it cannot be opened or mapped. */
int lssm_ssm_open(lssm_ssm** out, const char* path);
/* Unmaps the file and frees its HBM copy (lssm_ssm_upload). */
int lssm_ssm_close(lssm_ssm* f);
/* Header fields; n_groups 0 reads as 1 (ssm_loader.cpp:40). */
int lssm_ssm_get_header(const lssm_ssm* f, lssm_ssm_header* h);
/* Entry i in file order; its name (no NUL in the file) is copied into `name`
 * with a terminating NUL and must fit in `name_cap` bytes. */
int lssm_ssm_tensor_at(const lssm_ssm* f, uint32_t i, char* name, size_t name_cap,
                       lssm_ssm_tensor* t);
/* SSMFile::find / at (ssm_loader.cpp:141-157): LSSM_ENOTFOUND with the
 * message "SSMFile: no tensor named '<name>'" when absent. */
int lssm_ssm_find(const lssm_ssm* f, const char* name, lssm_ssm_tensor* t);
/* Copy the whole file into one HBM allocation, once (the UnifiedBuffer of
 * metal_buffer.mm:37-67, which wraps the mapping): a tensor's device address
 * is *device_base + its offset, the reference's (handle, byte offset) pair.
 * Later calls return the same copy.  Staged through pinned host buffers on the
 * context's stream; returns when the copy is complete. */
int lssm_ssm_upload(lssm_ssm* f, lssm_ctx* ctx, void** device_base);
/* Mamba2Model's weight lookups (mamba2_model.cpp:62-116) against a copy of
 * the file at `device_base` (the pointer lssm_ssm_upload returned): fills
 * `cfg` (act from the dtype of backbone.norm_f.weight, wfmt from the dtype of
 * in_proj), the addresses device_base + offset of embeddings, norm_f and
 * lm_head (lm_head.weight when present, else the embeddings) and `layers`
 * (cfg->n_layer entries, at most n_layers_cap; block-format scales follow the
 * packed values), ready for lssm_engine_create.  Every tensor's dtype, shape
 * and size is checked against what the engine reads; the reference's messages
 * for a missing tensor and for in_proj / conv1d dimension mismatches are kept. */
int lssm_ssm_model(const lssm_ssm* f, const void* device_base, lssm_model_config* cfg,
                   const void** embed, const void** norm_f, const void** lm_head,
                   lssm_layer_weights* layers, uint32_t n_layers_cap);

/* Streaming writer (the write path of tools/ssm_format.py): declare every
 * tensor, then put payloads in any order; the index is written at the first
 * put (or at finish) and no declaration is accepted after that.  Tensors
 * never put read as zeros.  After a failed call the writer keeps its first
 * error; finish returns it, deletes the partial file and frees the writer. */
typedef struct lssm_ssm_writer lssm_ssm_writer;
int lssm_ssm_writer_create(lssm_ssm_writer** out, const char* path, const lssm_ssm_header* hp);
int lssm_ssm_writer_declare(lssm_ssm_writer* w, const char* name, uint32_t dtype, uint32_t rank,
                            const uint64_t* shape);
int lssm_ssm_writer_put(lssm_ssm_writer* w, const char* name, const void* data, uint64_t nbytes);
int lssm_ssm_writer_finish(lssm_ssm_writer* w);

/* Quantize a row-major fp32 [N, K] weight to `wfmt` (Q4_B32, Q4_G64 or Q8_G32)
 * with the exporter's recipe (tools/export_mamba2.py:68-103): per group,
 * scale = max(|w|, 1e-12) / qmax in fp32, q = round-half-even(w / scale)
 * clamped to [qmin, qmax], scale stored fp16; int4 low nibble = even k.
 * `packed` gets N*K/2 (int4) or N*K (int8) bytes, `scales` N*K/G fp16 bits. */
int lssm_quantize(const float* w, uint32_t N, uint32_t K, uint32_t wfmt, uint8_t* packed,
                  uint16_t* scales);

/* Write a random-initialised Mamba-2 model of shape `cfg` (cfg->act: dtype of
 * embeddings, norms, conv and the per-head parameters; cfg->wfmt: format of
 * in_proj / out_proj) to `path`, with the reference exporter's tensor names and
 * order and a tied lm_head (no lm_head.weight).  Values: linears N(0, 0.02)
 * rounded to fp16 then quantized; embeddings N(0, 0.02); norms N(1, 0.1);
 * conv weight N(0, 0.3), bias N(0, 0.1); dt_bias = softplus^-1(dt) with dt
 * log-uniform in [1e-3, 1e-1]; A_log = log(1 + 15u); D N(1, 0.1).  Normals
 * come from std::mt19937_64 streams keyed by (seed, tensor, block) through the
 * Box-Muller transform in fp64, so the file depends only on cfg and seed.
 * No counterpart in the reference, which exports trained checkpoints. */
int lssm_ssm_write_random(const char* path, const lssm_model_config* cfg, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif /* LSSM_H */

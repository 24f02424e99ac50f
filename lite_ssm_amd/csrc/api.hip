// api.hip — the C-ABI op entry points.
//
// Reference-named entries (lssm_<op>_f16 ...) keep the preconditions and error
// texts of the MetalOps dispatchers (ops.mm:175-619) and forward to the
// generic entries with fp16 activations and batch 1.  Every entry validates
// shapes and alignment on the host before launching, so that no kernel is
// launched on a shape it does not support.
#include <algorithm>
#include <cstring>
#include <mutex>

#include "internal.hpp"

using namespace lssm;

namespace {

inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// GEMV fast-path requirements (gemv.hip): K a multiple of the 16-byte chunk,
// 16-byte aligned weight rows, one x row fits the fp32 LDS staging.
bool gemv_ok(const void* w, uint32_t K, int wfmt, int act) {
    if (!al16(w)) return false;
    if (gemv_lds_rows(K, wfmt, act) < 1) return false;
    switch (wfmt) {
        case LSSM_W_Q4_B32: return K % 32 == 0;
        case LSSM_W_Q4_G64: return K % 64 == 0;
        case LSSM_W_Q8_G32: return K % 32 == 0;
        default: return K % (16 / dtype_size(act)) == 0;
    }
}

bool gemm_ok(const void* x, uint32_t x_stride, const void* w, uint32_t K, int act) {
    return act != LSSM_F32 && K % 64 == 0 && x_stride % 8 == 0 && al16(x) && al16(w);
}

int check_fmt_k(uint32_t K, int wfmt, const void* s) {
    LSSM_REQUIRE(valid_wfmt(wfmt), "linear: unknown weight format %d", wfmt);
    if (wfmt != LSSM_W_DENSE) {
        const uint32_t G = wfmt_group(wfmt);
        LSSM_REQUIRE(K % G == 0, "linear: K must be a multiple of %u for this weight format", G);
        LSSM_REQUIRE(s != nullptr, "linear: quantized weights need a scales pointer");
    }
    return LSSM_OK;
}

// Shared core of lssm_linear and the reference GEMV/GEMM entries.
// mode: 0 = auto (M <= 4 -> GEMV semantics, else GEMM), 1 = GEMV, 2 = GEMM.
int linear_core(lssm_ctx* ctx, const void* x, uint32_t xs, const void* w, const void* s, void* y,
                uint32_t ys, const void* res, uint32_t M, uint32_t N, uint32_t K, int wfmt, int act,
                int epi, int mode, const char* name) {
    LSSM_REQUIRE(valid_act(act), "%s: unknown activation dtype %d", name, act);
    if (int rc = check_fmt_k(K, wfmt, s)) return rc;
    LSSM_REQUIRE(epi == LSSM_EPI_NONE || epi == LSSM_EPI_SILU || epi == LSSM_EPI_ADD,
                 "%s: unknown epilogue %d", name, epi);
    LSSM_REQUIRE(epi != LSSM_EPI_ADD || res != nullptr, "%s: EPI_ADD needs a residual", name);
    if (M == 0 || N == 0) return LSSM_OK;
    LSSM_REQUIRE(x && w && y && K > 0, "%s: null pointer or K == 0", name);
    if (xs == 0) xs = K;
    if (ys == 0) ys = N;
    LSSM_REQUIRE(xs >= K && ys >= N, "%s: row stride smaller than the row", name);
    const bool gemv = (mode == 1) || (mode == 0 && M <= 4);
    hipError_t e;
    if (gemv && gemv_ok(w, K, wfmt, act)) {
        GemvArgs g{x, xs, w, s, y, ys, res, nullptr, 0.0f, M, N, K, wfmt, act, epi};
        e = launch_gemv(ctx->stream, g);
    } else if (!gemv && gemm_ok(x, xs, w, K, act)) {
        GemmArgs g{x, xs, w, s, y, ys, res, M, N, K, wfmt, act, epi, 1};
        e = launch_gemm(ctx->stream, g);
    } else {
        GemmArgs g{x, xs, w, s, y, ys, res, M, N, K, wfmt, act, epi, gemv ? 0 : 1};
        e = launch_gemm_simple(ctx->stream, g);
    }
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "%s: %s", name, hipGetErrorString(e));
    return finish(ctx, name);
}

int ssd_common_checks(const lssm_ssd_dims& d, const char* name) {
    LSSM_REQUIRE(d.H > 0 && d.P > 0 && d.N > 0, "%s: H, P, N must be > 0", name);
    LSSM_REQUIRE(d.n_groups > 0 && d.H % d.n_groups == 0, "%s: H must be a multiple of n_groups", name);
    LSSM_REQUIRE(d.chunk_size >= 1 && d.chunk_size <= 64, "%s: chunk_size must be in [1, 64]", name);
    LSSM_REQUIRE(d.N <= 256, "%s: N must be <= 256", name);
    return LSSM_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// Generic entries
// ---------------------------------------------------------------------------
int lssm_rmsnorm(lssm_ctx* ctx, const void* x, const void* w, void* y, uint32_t rows, uint32_t dim,
                 float eps, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "rmsnorm: unknown dtype");
    LSSM_REQUIRE(dim > 0 || rows == 0, "rmsnorm: dim must be > 0");
    hipError_t e = launch_rmsnorm(ctx->stream, x, dim, w, y, dim, rows, dim, eps, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "rmsnorm: %s", hipGetErrorString(e));
    return finish(ctx, "rmsnorm");
}

int lssm_linear(lssm_ctx* ctx, const void* x, uint32_t x_stride, const void* w, const void* w_scales,
                void* y, uint32_t y_stride, const void* residual, uint32_t M, uint32_t N, uint32_t K,
                lssm_wfmt wfmt, lssm_dtype act, lssm_epilogue epi) {
    LSSM_CHECK_CTX(ctx);
    return linear_core(ctx, x, x_stride, w, w_scales, y, y_stride, residual, M, N, K, wfmt, act, epi,
                       0, "linear");
}

int lssm_norm_linear_decode(lssm_ctx* ctx, const void* x, const void* norm_w, float eps,
                            const void* w, const void* w_scales, void* y, const void* residual,
                            uint32_t rows, uint32_t N, uint32_t K, lssm_wfmt wfmt,
                            lssm_dtype act, lssm_epilogue epi) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "norm_linear_decode: unknown dtype");
    if (int rc = check_fmt_k(K, wfmt, w_scales)) return rc;
    LSSM_REQUIRE(epi == LSSM_EPI_NONE || epi == LSSM_EPI_SILU || epi == LSSM_EPI_ADD,
                 "norm_linear_decode: unknown epilogue %d", (int)epi);
    LSSM_REQUIRE(epi != LSSM_EPI_ADD || residual != nullptr, "norm_linear_decode: EPI_ADD needs a residual");
    LSSM_REQUIRE(rows <= 64, "norm_linear_decode: rows must be <= 64");
    if (rows == 0 || N == 0) return LSSM_OK;
    LSSM_REQUIRE(x && norm_w && w && y, "norm_linear_decode: null pointer");
    LSSM_REQUIRE(gemv_ok(w, K, wfmt, act), "norm_linear_decode: unsupported K / weight alignment");
    GemvArgs g{x, K, w, w_scales, y, N, residual, norm_w, eps, rows, N, K, wfmt, act, epi};
    hipError_t e = launch_gemv(ctx->stream, g);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "norm_linear_decode: %s", hipGetErrorString(e));
    return finish(ctx, "norm_linear_decode");
}

int lssm_dequant(lssm_ctx* ctx, const void* w, const void* w_scales, float* out, uint32_t N,
                 uint32_t K, lssm_wfmt wfmt) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(wfmt != LSSM_W_DENSE && valid_wfmt(wfmt), "dequant: quantized format required");
    LSSM_REQUIRE(K % wfmt_group(wfmt) == 0, "dequant: K must be a multiple of the group size");
    hipError_t e = launch_dequant(ctx->stream, w, w_scales, out, N, K, wfmt);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "dequant: %s", hipGetErrorString(e));
    return finish(ctx, "dequant");
}

int lssm_silu(lssm_ctx* ctx, const void* x, void* y, uint32_t n, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "silu: unknown dtype");
    hipError_t e = launch_silu(ctx->stream, x, y, n, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "silu: %s", hipGetErrorString(e));
    return finish(ctx, "silu");
}

int lssm_add_inplace(lssm_ctx* ctx, void* y, const void* x, uint32_t n, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "add_inplace: unknown dtype");
    hipError_t e = launch_add(ctx->stream, y, x, n, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "add_inplace: %s", hipGetErrorString(e));
    return finish(ctx, "add_inplace");
}

int lssm_silu_gated(lssm_ctx* ctx, const void* x, const void* gate, void* y, uint32_t n,
                    lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "silu_gated: unknown dtype");
    hipError_t e = launch_silu_gated(ctx->stream, x, gate, y, n, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "silu_gated: %s", hipGetErrorString(e));
    return finish(ctx, "silu_gated");
}

int lssm_split_silu_xbc(lssm_ctx* ctx, const void* xBC, void* x_out, void* B_out, void* C_out,
                        uint32_t rows, uint32_t d_inner, uint32_t d_state, uint32_t n_groups,
                        lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "split_silu_xBC: unknown dtype");
    hipError_t e = launch_split_silu(ctx->stream, xBC, x_out, B_out, C_out, rows, d_inner,
                                     n_groups * d_state, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "split_silu_xBC: %s", hipGetErrorString(e));
    return finish(ctx, "split_silu_xBC");
}

int lssm_conv1d(lssm_ctx* ctx, const void* x, const void* w, const void* bias, void* y, uint32_t B,
                uint32_t L, uint32_t D, uint32_t K, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "causal_conv1d: unknown dtype");
    LSSM_REQUIRE(K >= 1, "causal_conv1d: kernel width must be >= 1");
    LSSM_REQUIRE(L <= 65535 && B <= 65535, "causal_conv1d: L and B must be <= 65535");
    hipError_t e = launch_conv1d(ctx->stream, x, D, w, bias, y, D, B, L, D, K, act, false);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "causal_conv1d: %s", hipGetErrorString(e));
    return finish(ctx, "causal_conv1d");
}

int lssm_conv1d_update(lssm_ctx* ctx, const void* x_new, void* state, const void* w,
                       const void* bias, void* y, uint32_t B, uint32_t D, uint32_t K, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "causal_conv1d_update: unknown dtype");
    LSSM_REQUIRE(K >= 1, "causal_conv1d_update: kernel width must be >= 1");
    LSSM_REQUIRE(B <= 65535, "causal_conv1d_update: B must be <= 65535");
    hipError_t e = launch_conv1d_update(ctx->stream, x_new, state, w, bias, y, B, D, K, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "causal_conv1d_update: %s", hipGetErrorString(e));
    return finish(ctx, "causal_conv1d_update");
}

int lssm_conv1d_seed(lssm_ctx* ctx, const void* xBC, void* state, uint32_t B, uint32_t L, uint32_t D,
                     uint32_t K, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "seed_conv_state: unknown dtype");
    LSSM_REQUIRE(B <= 65535, "seed_conv_state: B must be <= 65535");
    hipError_t e = launch_conv1d_seed(ctx->stream, xBC, D, state, B, L, D, K, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "seed_conv_state: %s", hipGetErrorString(e));
    return finish(ctx, "seed_conv_state");
}

int lssm_gated_rmsnorm(lssm_ctx* ctx, const void* z, const void* y, const void* w, void* out,
                       uint32_t rows, uint32_t dim, float eps, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "gated_rmsnorm: unknown dtype");
    LSSM_REQUIRE(dim > 0 || rows == 0, "gated_rmsnorm: dim must be > 0");
    hipError_t e = launch_gated_rmsnorm(ctx->stream, z, dim, y, dim, w, out, rows, dim, eps, act);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "gated_rmsnorm: %s", hipGetErrorString(e));
    return finish(ctx, "gated_rmsnorm");
}

int lssm_ssd_chunked(lssm_ctx* ctx, const void* X, const void* B, const void* C, const void* dt_raw,
                     const void* dt_bias, const void* A_log, const void* D_skip, void* Y, float* state,
                     uint32_t batch, lssm_ssd_dims d, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "ssd_chunked: unknown dtype");
    if (int rc = ssd_common_checks(d, "ssd_chunked")) return rc;
    LSSM_REQUIRE(batch <= 65535, "ssd_chunked: batch must be <= 65535");
    LSSM_REQUIRE(!d.has_D || D_skip, "ssd_chunked: has_D set but D is null");
    if (batch == 0 || d.L == 0) return LSSM_OK;
    const uint32_t GN = d.n_groups * d.N;
    SsdArgs a{X, d.H * d.P, B, GN, C, GN, dt_raw, d.H, dt_bias, A_log, D_skip, Y, d.H * d.P, state,
              batch, d.L, d.H, d.P, d.N, d.n_groups, d.chunk_size, d.dt_min, d.dt_max, d.has_D, act,
              nullptr, 0};
    // The context's workspaces: the segment workspace (allocated on first
    // use) and the Gram tiles of the MFMA scan (grown on demand).  Neither is
    // allocated while the stream is being captured; the scan then runs
    // without the ones that do not exist yet (unsegmented, or each head
    // forming its own C B^T).  A captured launch may keep either address, so
    // neither is freed before lssm_ctx_destroy: a grown-out Gram buffer is
    // retired, not freed.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(ctx->stream, &cap);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "ssd_chunked: %s", hipGetErrorString(e));
    if (cap == hipStreamCaptureStatusNone) {
        if (!ctx->ssd_seg) {
            e = hipMalloc((void**)&ctx->ssd_seg, ssd_seg_floats() * sizeof(float));
            if (e != hipSuccess) {
                ctx->ssd_seg = nullptr;
                return set_error(LSSM_EDEVICE, "ssd_chunked: segment workspace: %s", hipGetErrorString(e));
            }
        }
        const size_t gf = ssd_gram_floats(batch, d.L, d.n_groups);
        if (act != LSSM_F32 && ctx->ssd_gram_cap < gf) {
            const size_t want = std::max(gf, 2 * ctx->ssd_gram_cap);
            float* p = nullptr;
            e = hipMalloc((void**)&p, want * sizeof(float));
            if (e != hipSuccess)
                return set_error(LSSM_EDEVICE, "ssd_chunked: Gram workspace: %s", hipGetErrorString(e));
            if (ctx->ssd_gram) ctx->ssd_gram_retired.push_back(ctx->ssd_gram);
            ctx->ssd_gram = p;
            ctx->ssd_gram_cap = want;
        }
    }
    a.seg = ctx->ssd_seg;
    if (act != LSSM_F32 && ctx->ssd_gram_cap >= ssd_gram_floats(batch, d.L, d.n_groups)) a.gram = ctx->ssd_gram;
    e = launch_ssd_chunked(ctx->stream, a);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "ssd_chunked: %s", hipGetErrorString(e));
    return finish(ctx, "ssd_chunked");
}

int lssm_ssd_step(lssm_ctx* ctx, const void* x, const void* B, const void* C, const void* dt_raw,
                  const void* dt_bias, const void* A_log, const void* D_skip, float* state, void* y,
                  uint32_t batch, lssm_ssd_step_dims d, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "ssd_step: unknown dtype");
    LSSM_REQUIRE(d.H > 0 && d.P > 0 && d.N > 0, "ssd_step: H, P, N must be > 0");
    LSSM_REQUIRE(d.P <= 1024, "ssd_step: P must be <= 1024");
    LSSM_REQUIRE(d.n_groups > 0 && d.H % d.n_groups == 0, "ssd_step: H must be a multiple of n_groups");
    LSSM_REQUIRE(batch <= 65535, "ssd_step: batch must be <= 65535");
    LSSM_REQUIRE(!d.has_D || D_skip, "ssd_step: has_D set but D is null");
    if (batch == 0) return LSSM_OK;
    const uint32_t GN = d.n_groups * d.N;
    SsdArgs a{x, d.H * d.P, B, GN, C, GN, dt_raw, d.H, dt_bias, A_log, D_skip, y, d.H * d.P, state,
              batch, 1, d.H, d.P, d.N, d.n_groups, 1, d.dt_min, d.dt_max, d.has_D, act, nullptr, 0};
    hipError_t e = launch_ssd_step(ctx->stream, a);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "ssd_step: %s", hipGetErrorString(e));
    return finish(ctx, "ssd_step");
}

int lssm_inproj_decode(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                       const void* w_scales, void* conv_state, const void* conv_w,
                       const void* conv_b, void* z, void* xbc_act, void* dt, uint32_t batch,
                       uint32_t d_model, uint32_t d_inner, uint32_t d_state, uint32_t n_groups,
                       uint32_t n_heads, uint32_t d_conv, float eps, lssm_wfmt wfmt,
                       lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "inproj_decode: unknown dtype");
    if (int rc = check_fmt_k(d_model, wfmt, w_scales)) return rc;
    LSSM_REQUIRE(batch >= 1 && batch <= 64, "inproj_decode: batch must be in [1, 64]");
    LSSM_REQUIRE(d_conv >= 1, "inproj_decode: d_conv must be >= 1");
    LSSM_REQUIRE((uintptr_t)conv_state % 8 == 0 && (uintptr_t)conv_w % 8 == 0,
                 "inproj_decode: conv_state and conv_w must be 8-byte aligned");
    LSSM_REQUIRE(gemv_ok(w, d_model, wfmt, act), "inproj_decode: unsupported d_model / weight alignment");
    LSSM_REQUIRE(gemv_max_rows(d_model, wfmt, act) >= 1, "inproj_decode: d_model too large");
    const uint32_t xbc = d_inner + 2u * n_groups * d_state;
    InprojDecodeArgs a;
    a.g = GemvArgs{hidden, d_model, w, w_scales, nullptr, 0, nullptr, norm_w, eps, batch,
                   d_inner + xbc + n_heads, d_model, wfmt, act, LSSM_EPI_NONE};
    a.d_inner = d_inner;
    a.xbc = xbc;
    a.H = n_heads;
    a.dconv = d_conv;
    a.conv_state = conv_state;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.z = z;
    a.xbc_act = xbc_act;
    a.dt = dt;
    hipError_t e = launch_inproj_decode(ctx->stream, a);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "inproj_decode: %s", hipGetErrorString(e));
    return finish(ctx, "inproj_decode");
}

int lssm_inproj_ssd_decode(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                           const void* w_scales, void* conv_state, const void* conv_w,
                           const void* conv_b, const void* dt_bias, const void* A_log,
                           const void* D_skip, float* ssd_state, void* y, uint64_t* xfer,
                           uint32_t tag, uint32_t d_model, uint32_t d_inner, uint32_t d_state,
                           uint32_t n_groups, uint32_t n_heads, uint32_t d_head, uint32_t d_conv,
                           float eps, lssm_wfmt wfmt, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "inproj_ssd_decode: unknown dtype");
    if (int rc = check_fmt_k(d_model, wfmt, w_scales)) return rc;
    LSSM_REQUIRE(xfer && ssd_state && y && norm_w && A_log && dt_bias, "inproj_ssd_decode: null pointer");
    LSSM_REQUIRE(n_heads >= 1 && n_groups >= 1 && d_inner == n_heads * d_head,
                 "inproj_ssd_decode: d_inner must equal n_heads * d_head");
    const uint32_t xbc = d_inner + 2u * n_groups * d_state;
    InprojDecodeArgs a;
    a.g = GemvArgs{hidden, d_model, w, w_scales, nullptr, 0, nullptr, norm_w, eps, 1u,
                   d_inner + xbc + n_heads, d_model, wfmt, act, LSSM_EPI_NONE};
    a.d_inner = d_inner;
    a.xbc = xbc;
    a.H = n_heads;
    a.dconv = d_conv;
    a.conv_state = conv_state;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.z = nullptr;
    a.xbc_act = nullptr;
    a.dt = nullptr;
    const SsdFuseArgs f{xfer, nullptr, tag, ssd_state, A_log, dt_bias, D_skip, y, d_head, d_state, n_groups,
                        1e-6f, 1e6f, ctx->status, (ctx->debug & LSSM_DEBUG_STALE_WAIT) ? 1u : 0u};
    hipError_t e = hipSuccess;
    if (!launch_inproj_ssd_decode(ctx->stream, a, f, e))
        return set_error(LSSM_EINVAL, "inproj_ssd_decode: shape, format, alignment or grid not supported by the fused launch");
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "inproj_ssd_decode: %s", hipGetErrorString(e));
    return finish(ctx, "inproj_ssd_decode");
}

// ---------------------------------------------------------------------------
// lssm_inproj_ssd_decode without a caller workspace and without allocating:
// the projection's tagged words and the step tag live in `scratch`, a static
// device array (zero at load, so no word carries a tag before its first use).
// Its device address is looked up once per device with hipGetSymbolAddress;
// host code uses only that address, never the array's name.  A one-thread
// kernel advances the tag on the device before each fused launch, so every
// call runs with a new tag and the host keeps no counter.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t NOALLOC_WORDS = 1u << 16;                 // projection rows it can carry
constexpr size_t NOALLOC_BYTES = NOALLOC_WORDS * 8 + 256;  // words + the tag (512 KiB + 256 B)
__device__ __align__(256) uint64_t scratch[NOALLOC_BYTES / 8];
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// This device's copy of `scratch` (the device must be current); null + error
// text on failure.
void* scratch_of(int dev) {
    if (dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

__global__ void advance_tag_kernel(uint32_t* seq) {
    if (threadIdx.x == 0) *seq += 1u;
}
}  // namespace

int lssm_mixer_decode(lssm_ctx* ctx, void* hidden, const void* norm_w, const void* in_w,
                      const void* in_scales, void* conv_state, const void* conv_w,
                      const void* conv_b, const void* dt_bias, const void* A_log,
                      const void* D_skip, float* ssd_state, const void* mixer_norm_w,
                      const void* out_w, const void* out_scales, uint64_t* xfer, uint32_t tag,
                      uint32_t d_model, uint32_t d_inner, uint32_t d_state, uint32_t n_groups,
                      uint32_t n_heads, uint32_t d_head, uint32_t d_conv, float eps,
                      lssm_wfmt wfmt, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "mixer_decode: unknown dtype");
    if (int rc = check_fmt_k(d_model, wfmt, in_scales)) return rc;
    if (int rc = check_fmt_k(d_inner, wfmt, out_scales)) return rc;
    LSSM_REQUIRE(hidden && xfer && ssd_state && norm_w && mixer_norm_w && A_log && dt_bias && out_w,
                 "mixer_decode: null pointer");
    LSSM_REQUIRE(n_heads >= 1 && n_groups >= 1 && d_inner == n_heads * d_head,
                 "mixer_decode: d_inner must equal n_heads * d_head");
    const uint32_t xbc = d_inner + 2u * n_groups * d_state, proj = d_inner + xbc + n_heads;
    InprojDecodeArgs a;
    a.g = GemvArgs{hidden, d_model, in_w, in_scales, nullptr, 0, nullptr, norm_w, eps, 1u, proj, d_model,
                   wfmt, act, LSSM_EPI_NONE};
    a.d_inner = d_inner;
    a.xbc = xbc;
    a.H = n_heads;
    a.dconv = d_conv;
    a.conv_state = conv_state;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.z = nullptr;
    a.xbc_act = nullptr;
    a.dt = nullptr;
    const SsdFuseArgs f{xfer, nullptr, tag, ssd_state, A_log, dt_bias, D_skip, nullptr, d_head, d_state, n_groups,
                        1e-6f, 1e6f, ctx->status};
    const OutprojFuseArgs o{out_w, out_scales, mixer_norm_w, eps, hidden, reinterpret_cast<uint32_t*>(xfer + proj), d_model};
    hipError_t e = hipSuccess;
    if (!launch_layer_decode(ctx->stream, a, f, o, e))
        return set_error(LSSM_EINVAL, "mixer_decode: shape, format, alignment or grid not supported by the fused launch");
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "mixer_decode: %s", hipGetErrorString(e));
    return finish(ctx, "mixer_decode");
}

int lssm_inproj_ssd_decode_noalloc(lssm_ctx* ctx, const void* hidden, const void* norm_w, const void* w,
                                   const void* w_scales, void* conv_state, const void* conv_w,
                                   const void* conv_b, const void* dt_bias, const void* A_log,
                                   const void* D_skip, float* ssd_state, void* y, uint32_t d_model,
                                   uint32_t d_inner, uint32_t d_state, uint32_t n_groups, uint32_t n_heads,
                                   uint32_t d_head, uint32_t d_conv, float eps, lssm_wfmt wfmt,
                                   lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "inproj_ssd_decode_noalloc: unknown dtype");
    if (int rc = check_fmt_k(d_model, wfmt, w_scales)) return rc;
    LSSM_REQUIRE(ssd_state && y && norm_w && A_log && dt_bias, "inproj_ssd_decode_noalloc: null pointer");
    LSSM_REQUIRE(n_heads >= 1 && n_groups >= 1 && d_inner == n_heads * d_head,
                 "inproj_ssd_decode_noalloc: d_inner must equal n_heads * d_head");
    const uint32_t xbc = d_inner + 2u * n_groups * d_state;
    const size_t proj = (size_t)d_inner + xbc + n_heads;
    LSSM_REQUIRE(proj <= NOALLOC_WORDS,
                 "inproj_ssd_decode_noalloc: %zu projection rows exceed the static scratch of %zu rows", proj,
                 NOALLOC_WORDS);
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
        return set_error(LSSM_EINVAL, "inproj_ssd_decode_noalloc: the context's device must be current");
    char* base = (char*)scratch_of(dev);
    if (!base) return set_error(LSSM_EDEVICE, "inproj_ssd_decode_noalloc: hipGetSymbolAddress(scratch) failed");
    uint64_t* words = reinterpret_cast<uint64_t*>(base);
    uint32_t* seq = reinterpret_cast<uint32_t*>(base + NOALLOC_WORDS * 8);
    InprojDecodeArgs a;
    a.g = GemvArgs{hidden, d_model, w, w_scales, nullptr, 0, nullptr, norm_w, eps, 1u, (uint32_t)proj, d_model,
                   wfmt, act, LSSM_EPI_NONE};
    a.d_inner = d_inner;
    a.xbc = xbc;
    a.H = n_heads;
    a.dconv = d_conv;
    a.conv_state = conv_state;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.z = nullptr;
    a.xbc_act = nullptr;
    a.dt = nullptr;
    const SsdFuseArgs f{words, seq, 0u, ssd_state, A_log, dt_bias, D_skip, y, d_head, d_state, n_groups,
                        1e-6f, 1e6f, ctx->status, 0u};
    advance_tag_kernel<<<1, 64, 0, ctx->stream>>>(seq);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "inproj_ssd_decode_noalloc: %s", hipGetErrorString(e));
    if (!launch_inproj_ssd_decode(ctx->stream, a, f, e))
        return set_error(LSSM_EINVAL,
                         "inproj_ssd_decode_noalloc: shape, format, alignment or grid not supported by the fused "
                         "launch (the tag was advanced; the state was not touched)");
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "inproj_ssd_decode_noalloc: %s", hipGetErrorString(e));
    return finish(ctx, "inproj_ssd_decode_noalloc");
}

int lssm_embed(lssm_ctx* ctx, const void* table, const int32_t* ids, void* out, uint32_t n,
               uint32_t d_model, uint32_t vocab, lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "embed: unknown dtype");
    hipError_t e = launch_embed(ctx->stream, table, ids, out, n, d_model, vocab, act, ctx->status);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "embed: %s", hipGetErrorString(e));
    return finish(ctx, "embed");
}

int lssm_argmax(lssm_ctx* ctx, const void* logits, int32_t* ids, uint32_t rows, uint32_t vocab,
                lssm_dtype act) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(valid_act(act), "argmax: unknown dtype");
    LSSM_REQUIRE(vocab > 0 || rows == 0, "argmax: empty logits");
    LSSM_REQUIRE(rows <= 65535, "argmax: rows must be <= 65535");
    hipError_t e = launch_argmax(ctx->stream, logits, ids, rows, vocab, act, nullptr);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "argmax: %s", hipGetErrorString(e));
    return finish(ctx, "argmax");
}

// ---------------------------------------------------------------------------
// Reference-named entries (fp16, batch 1)
// ---------------------------------------------------------------------------
int lssm_rmsnorm_f16(lssm_ctx* ctx, const void* x, const void* w, void* y, lssm_rmsnorm_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.dim % 4 == 0, "rmsnorm_f16: dim must be a multiple of 4");   // ops.mm:179-181
    return lssm_rmsnorm(ctx, x, w, y, d.rows, d.dim, d.eps, LSSM_F16);
}

int lssm_linear_f16_gemv(lssm_ctx* ctx, const void* x, const void* w, void* y, lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.M == 1, "dispatch_gemv: M must be 1");                      // ops.mm:207-212
    LSSM_REQUIRE(d.K % 4 == 0, "dispatch_gemv: K must be a multiple of 4");
    return linear_core(ctx, x, 0, w, nullptr, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_DENSE, LSSM_F16,
                       LSSM_EPI_NONE, 1, "linear_f16_gemv");
}

int lssm_linear_silu_f16_gemv(lssm_ctx* ctx, const void* x, const void* w, void* y,
                              lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.M == 1, "dispatch_gemv: M must be 1");
    LSSM_REQUIRE(d.K % 4 == 0, "dispatch_gemv: K must be a multiple of 4");
    return linear_core(ctx, x, 0, w, nullptr, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_DENSE, LSSM_F16,
                       LSSM_EPI_SILU, 1, "linear_silu_f16_gemv");
}

// linear.metal:148-204: RMSNorm staged (rounded to half) then GEMV.
int lssm_rmsnorm_linear_f16_gemv(lssm_ctx* ctx, const void* x, const void* w_norm, const void* w,
                                 void* y, lssm_rms_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.K % 4 == 0, "rmsnorm_linear_f16_gemv: K must be a multiple of 4");  // ops.mm:251-253
    if (d.N == 0) return LSSM_OK;
    if (gemv_ok(w, d.K, LSSM_W_DENSE, LSSM_F16)) {
        GemvArgs g{x, d.K, w, nullptr, y, d.N, nullptr, w_norm, d.eps, 1, d.N, d.K, LSSM_W_DENSE,
                   LSSM_F16, LSSM_EPI_NONE};
        hipError_t e = launch_gemv(ctx->stream, g);
        if (e != hipSuccess) return set_error(LSSM_EDEVICE, "rmsnorm_linear_f16_gemv: %s", hipGetErrorString(e));
        return finish(ctx, "rmsnorm_linear_f16_gemv");
    }
    return set_error(LSSM_EINVAL, "rmsnorm_linear_f16_gemv: K must be a multiple of 8 and <= 16384 "
                                  "with a 16-byte aligned weight");
}

int lssm_linear_f16_gemm(lssm_ctx* ctx, const void* x, const void* w, void* y, lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    return linear_core(ctx, x, 0, w, nullptr, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_DENSE, LSSM_F16,
                       LSSM_EPI_NONE, 2, "linear_f16_gemm");
}

int lssm_linear_silu_f16_gemm(lssm_ctx* ctx, const void* x, const void* w, void* y,
                              lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    return linear_core(ctx, x, 0, w, nullptr, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_DENSE, LSSM_F16,
                       LSSM_EPI_SILU, 2, "linear_silu_f16_gemm");
}

int lssm_linear_int4_gemv(lssm_ctx* ctx, const void* x, const void* w_packed, const void* w_scales,
                          void* y, lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.M == 1, "linear_int4_gemv: M must be 1");                   // ops.mm:323-324
    LSSM_REQUIRE(d.K % 32 == 0, "linear_int4_gemv: K must be a multiple of 32");
    return linear_core(ctx, x, 0, w_packed, w_scales, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_Q4_B32,
                       LSSM_F16, LSSM_EPI_NONE, 1, "linear_int4_gemv");
}

int lssm_linear_int4_gemm(lssm_ctx* ctx, const void* x, const void* w_packed, const void* w_scales,
                          void* y, lssm_linear_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.K % 32 == 0, "linear_int4_gemm: K must be a multiple of 32");  // ops.mm:347
    return linear_core(ctx, x, 0, w_packed, w_scales, y, 0, nullptr, d.M, d.N, d.K, LSSM_W_Q4_B32,
                       LSSM_F16, LSSM_EPI_NONE, 2, "linear_int4_gemm");
}

int lssm_silu_f16(lssm_ctx* ctx, const void* x, void* y, uint32_t n) {
    return lssm_silu(ctx, x, y, n, LSSM_F16);
}

int lssm_add_inplace_f16(lssm_ctx* ctx, void* y, const void* x, uint32_t n) {
    return lssm_add_inplace(ctx, y, x, n, LSSM_F16);
}

int lssm_split_silu_xBC_f16(lssm_ctx* ctx, const void* xBC, void* x_out, void* B_out, void* C_out,
                            uint32_t L, uint32_t d_inner, uint32_t d_state, uint32_t n_groups) {
    return lssm_split_silu_xbc(ctx, xBC, x_out, B_out, C_out, L, d_inner, d_state, n_groups, LSSM_F16);
}

int lssm_silu_gated_f16(lssm_ctx* ctx, const void* x, const void* gate, void* y, uint32_t n) {
    return lssm_silu_gated(ctx, x, gate, y, n, LSSM_F16);
}

int lssm_causal_conv1d_f16(lssm_ctx* ctx, const void* x, const void* w, const void* bias, void* y,
                           lssm_conv1d_dims d) {
    return lssm_conv1d(ctx, x, w, bias, y, d.B, d.L, d.D, d.K, LSSM_F16);
}

int lssm_causal_conv1d_update_f16(lssm_ctx* ctx, const void* x_new, void* state, const void* w,
                                  const void* bias, void* y, lssm_conv1d_dims d) {
    return lssm_conv1d_update(ctx, x_new, state, w, bias, y, d.B, d.D, d.K, LSSM_F16);
}

int lssm_seed_conv_state_f16(lssm_ctx* ctx, const void* xBC, void* state, uint32_t L, uint32_t D,
                             uint32_t K) {
    return lssm_conv1d_seed(ctx, xBC, state, 1, L, D, K, LSSM_F16);
}

int lssm_inproj_fused_f16(lssm_ctx* ctx, const void* normed, const void* W_in, const void* W_conv,
                          const void* conv_b, void* proj_z, void* ssd_x, void* ssd_B, void* ssd_C,
                          void* proj_dt, void* proj_xBC, lssm_fused_inproj_dims d) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(d.L <= 16, "inproj_fused_f16: L must be <= 16");            // fused.metal:20-22
    const uint32_t xbc = d.d_inner + 2u * d.n_groups * d.d_state;
    LSSM_REQUIRE(d.proj_dim == d.d_inner + xbc + d.n_heads,
                 "inproj_fused_f16: proj_dim must be d_inner + xBC_dim + n_heads");
    hipError_t e = launch_inproj_fused(ctx->stream, normed, W_in, W_conv, conv_b, proj_z, ssd_x, ssd_B,
                                       ssd_C, proj_dt, proj_xBC, d);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "inproj_fused_f16: %s", hipGetErrorString(e));
    return finish(ctx, "inproj_fused_f16");
}

int lssm_ssd_chunked_f16(lssm_ctx* ctx, const void* X, const void* B, const void* C,
                         const void* dt_raw, const void* dt_bias, const void* A_log,
                         const void* D_skip, void* Y, float* state_io, lssm_ssd_dims d) {
    return lssm_ssd_chunked(ctx, X, B, C, dt_raw, dt_bias, A_log, D_skip, Y, state_io, 1, d, LSSM_F16);
}

int lssm_ssd_step_f16(lssm_ctx* ctx, const void* x, const void* B, const void* C, const void* dt_raw,
                      const void* dt_bias, const void* A_log, const void* D_skip, float* state,
                      void* y, lssm_ssd_step_dims d) {
    return lssm_ssd_step(ctx, x, B, C, dt_raw, dt_bias, A_log, D_skip, state, y, 1, d, LSSM_F16);
}

}  // extern "C"

// ctx.hip — context, batching, errors, memory and kernel introspection.
//
// Replaces the Metal device/queue singletons (metal_context.mm:25-70), the
// kernel registry (kernel_registry.mm:19-93) and MetalOps' batch lifecycle
// (ops.mm:62-149).  One lssm_ctx owns (or borrows) one HIP stream; there is no
// global mutable state besides the thread-local error string.
#include <dlfcn.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "internal.hpp"

namespace lssm {

static thread_local std::string g_err;

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

void clear_error() { g_err.clear(); }

int sync_and_check(lssm_ctx* ctx, const char* what) {
    hipError_t e = hipMemcpyAsync(ctx->status_host, ctx->status, sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "%s failed: %s", what, hipGetErrorString(e));
    const uint32_t st = *ctx->status_host;
    if (st == 0) return LSSM_OK;
    // clear for the next check (a plain copy: no memset node can end up in a
    // captured graph from here, and the word is only written by kernels)
    *ctx->status_host = 0;
    e = hipMemcpyAsync(ctx->status, ctx->status_host, sizeof(uint32_t), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "%s failed: %s", what, hipGetErrorString(e));
    // The fused decode launch shifts each conv window in its in_proj epilogue,
    // before any SSD item waits, so a timed-out step has advanced the conv
    // state by its token while leaving the waiting items' SSD state alone.
    const char* wait_msg =
        "a cross-workgroup wait timed out (the launch's workgroups were not all resident at once); "
        "the affected outputs are NaN and their SSD state was not updated, but the conv state did "
        "advance by this step's token";
    // mamba2_model.cpp:129-131 throws std::out_of_range with this text
    if ((st & STATUS_BAD_TOKEN) && (st & STATUS_WAIT_TIMEOUT))
        return set_error(LSSM_EINVAL, "Mamba2Model::embed: token_id out of range (%s); also: %s", what,
                         wait_msg);
    if (st & STATUS_BAD_TOKEN)
        return set_error(LSSM_EINVAL, "Mamba2Model::embed: token_id out of range (%s)", what);
    return set_error(LSSM_EDEVICE, "%s: %s", what, wait_msg);
}

int finish(lssm_ctx* ctx, const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(LSSM_EDEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
    if (!ctx->batch) return sync_and_check(ctx, what);
    return LSSM_OK;
}

__global__ void lite_ssm_common_noop() {}

// Compute units of the current device (queried once per process).
uint32_t num_cus() {
    static const uint32_t n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return 256u;
        return (uint32_t)cus;
    }();
    return n;
}

}  // namespace lssm

using namespace lssm;

extern "C" {

const char* lssm_last_error(void) { return g_err.c_str(); }

int lssm_ctx_create(lssm_ctx** out, void* stream) {
    clear_error();
    if (!out) return set_error(LSSM_EINVAL, "lssm_ctx_create: null out");
    auto* c = new lssm_ctx();
    hipError_t e = hipGetDevice(&c->device);
    if (e != hipSuccess) {
        delete c;
        return set_error(LSSM_EDEVICE, "lssm_ctx_create: no HIP device: %s", hipGetErrorString(e));
    }
    if (stream) {
        c->stream = (hipStream_t)stream;
    } else {
        // default priority only: streams of different priorities are not used anywhere
        e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            return set_error(LSSM_EDEVICE, "lssm_ctx_create: %s", hipGetErrorString(e));
        }
        c->own_stream = true;
    }
    e = hipMalloc((void**)&c->status, 256);
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->status_host, 256, hipHostMallocDefault);
    if (e == hipSuccess) {
        *c->status_host = 0;
        e = hipMemcpyAsync(c->status, c->status_host, sizeof(uint32_t), hipMemcpyHostToDevice, c->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        if (c->status) (void)hipFree(c->status);
        if (c->status_host) (void)hipHostFree(c->status_host);
        if (c->own_stream) (void)hipStreamDestroy(c->stream);
        delete c;
        return set_error(LSSM_EDEVICE, "lssm_ctx_create: status word: %s", hipGetErrorString(e));
    }
    *out = c;
    return LSSM_OK;
}

int lssm_ctx_destroy(lssm_ctx* ctx) {
    clear_error();
    if (!ctx) return LSSM_OK;
    // An uncommitted batch is dropped after the queued work drains (ops.mm:64-68).
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(ctx->status);
    (void)hipHostFree(ctx->status_host);
    if (ctx->ssd_seg) (void)hipFree(ctx->ssd_seg);
    if (ctx->ssd_gram) (void)hipFree(ctx->ssd_gram);
    for (float* p : ctx->ssd_gram_retired) (void)hipFree(p);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return LSSM_OK;
}

int lssm_ctx_stream(lssm_ctx* ctx, void** stream_out) {
    LSSM_CHECK_CTX(ctx);
    if (!stream_out) return set_error(LSSM_EINVAL, "lssm_ctx_stream: null out");
    *stream_out = (void*)ctx->stream;
    return LSSM_OK;
}

int lssm_begin_batch(lssm_ctx* ctx) {
    LSSM_CHECK_CTX(ctx);
    if (ctx->batch)
        return set_error(LSSM_ESTATE, "MetalOps: begin_batch called while batch already active");
    ctx->batch = true;
    return LSSM_OK;
}

int lssm_commit_and_wait(lssm_ctx* ctx) {
    LSSM_CHECK_CTX(ctx);
    if (!ctx->batch)
        return set_error(LSSM_ESTATE, "MetalOps: commit_and_wait without an active batch");
    ctx->batch = false;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(LSSM_EDEVICE, "HIP: forward batch failed: %s", hipGetErrorString(e));
    return sync_and_check(ctx, "HIP: forward batch");
}

int lssm_batch_active(lssm_ctx* ctx) { return (ctx && ctx->batch) ? 1 : 0; }

int lssm_sync(lssm_ctx* ctx) {
    LSSM_CHECK_CTX(ctx);
    return sync_and_check(ctx, "lssm_sync");
}

int lssm_ctx_set_debug(lssm_ctx* ctx, uint32_t flags) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE((flags & ~LSSM_DEBUG_STALE_WAIT) == 0, "lssm_ctx_set_debug: unknown flag");
    ctx->debug = flags;
    return LSSM_OK;
}

// ---------------------------------------------------------------------------
// Introspection.  The 19 names are the reference's kernel entry points
// (shaders/*.metal, listed by tests/test_metal_ops.cpp:31-49 plus
// split_silu_xBC_f16 and add_inplace_f16); the rest are this build's generic
// and fused kernels.
// ---------------------------------------------------------------------------
static const char* const kKernelNames[] = {
    "lite_ssm_common_noop",
    "rmsnorm_f16",
    "linear_f16_gemv",
    "linear_silu_f16_gemv",
    "rmsnorm_linear_f16_gemv",
    "linear_f16_gemm",
    "linear_silu_f16_gemm",
    "linear_int4_gemv",
    "linear_int4_gemm",
    "silu_f16",
    "add_inplace_f16",
    "split_silu_xBC_f16",
    "silu_gated_f16",
    "causal_conv1d_f16",
    "causal_conv1d_update_f16",
    "seed_conv_state_f16",
    "inproj_fused_f16",
    "ssd_chunked_f16",
    "ssd_step_f16",
    // generic / fused
    "rmsnorm",
    "gated_rmsnorm",
    "linear_gemv_q",
    "linear_gemm_mfma",
    "dequant",
    "conv1d",
    "conv1d_update",
    "conv1d_seed",
    "ssd_chunked_mfma",
    "ssd_step_gate",
    "inproj_decode",
    "embed",
    "argmax",
};

int lssm_kernel_count(void) { return (int)(sizeof(kKernelNames) / sizeof(kKernelNames[0])); }

const char* lssm_kernel_name(int i) {
    if (i < 0 || i >= lssm_kernel_count()) return nullptr;
    return kKernelNames[i];
}

int lssm_has_kernel(const char* name) {
    if (!name) return 0;
    for (int i = 0; i < lssm_kernel_count(); ++i)
        if (std::strcmp(kKernelNames[i], name) == 0) return 1;
    return 0;
}

// True iff a HIP device is present and this library's code object has a
// kernel for it (the metallib-loaded probe, ops.mm:157-161).
int lssm_library_loaded(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&lssm::lite_ssm_common_noop)) != hipSuccess)
        return 0;
    return 1;
}

const char* lssm_library_path(void) {
    static std::string path;
    if (path.empty()) {
        Dl_info info;
        if (dladdr(reinterpret_cast<void*>(&lssm_library_path), &info) && info.dli_fname)
            path = info.dli_fname;
    }
    return path.c_str();
}

// ---------------------------------------------------------------------------
// Memory
// ---------------------------------------------------------------------------
int lssm_malloc(void** out, size_t nbytes) {
    clear_error();
    if (!out) return set_error(LSSM_EINVAL, "lssm_malloc: null out");
    *out = nullptr;
    if (nbytes == 0) return LSSM_OK;
    hipError_t e = hipMalloc(out, nbytes);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_malloc(%zu): %s", nbytes, hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_malloc_host(void** out, size_t nbytes) {
    clear_error();
    if (!out) return set_error(LSSM_EINVAL, "lssm_malloc_host: null out");
    *out = nullptr;
    if (nbytes == 0) return LSSM_OK;
    // Default flags: coherent, mapped into every device's address space, so
    // the same pointer is used by host code and by kernels.
    hipError_t e = hipHostMalloc(out, nbytes, hipHostMallocDefault);
    if (e != hipSuccess)
        return set_error(LSSM_EDEVICE, "lssm_malloc_host(%zu): %s", nbytes, hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_free(void* p) {
    clear_error();
    if (!p) return LSSM_OK;
    hipError_t e = hipFree(p);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_free: %s", hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_free_host(void* p) {
    clear_error();
    if (!p) return LSSM_OK;
    hipError_t e = hipHostFree(p);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_free_host: %s", hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_memcpy_h2d(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes) {
    LSSM_CHECK_CTX(ctx);
    if (nbytes == 0) return LSSM_OK;
    hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_memcpy_h2d: %s", hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_memcpy_d2h(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes) {
    LSSM_CHECK_CTX(ctx);
    if (nbytes == 0) return LSSM_OK;
    hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_memcpy_d2h: %s", hipGetErrorString(e));
    return LSSM_OK;
}

int lssm_memcpy_d2d(lssm_ctx* ctx, void* dst, const void* src, size_t nbytes) {
    LSSM_CHECK_CTX(ctx);
    if (nbytes == 0) return LSSM_OK;
    hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_memcpy_d2d: %s", hipGetErrorString(e));
    return finish(ctx, "lssm_memcpy_d2d");
}

int lssm_memset(lssm_ctx* ctx, void* dst, int value, size_t nbytes) {
    LSSM_CHECK_CTX(ctx);
    if (nbytes == 0) return LSSM_OK;
    hipError_t e = hipMemsetAsync(dst, value, nbytes, ctx->stream);
    if (e != hipSuccess) return set_error(LSSM_EDEVICE, "lssm_memset: %s", hipGetErrorString(e));
    return finish(ctx, "lssm_memset");
}

}  // extern "C"

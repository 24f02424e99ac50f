// ops.cpp — lite_ssm::MetalOps served by the HIP kernels of liblssm_hip.so.
//
// Interface: include/lite_ssm/ops.hpp (reference include/lite_ssm/ops.hpp:30-244).
// Each method resolves (handle, byte offset) to a device address and calls the
// matching C entry point of include/lssm.h; a non-zero status is rethrown as
// std::runtime_error carrying lssm_last_error(), whose text for argument
// errors is the reference's own (src/backend/metal/ops.mm:175-620).  The
// stream is created on the first op or batch, so a MetalOps can be built and
// queried (metallib_loaded) on a machine without a GPU, as the reference's
// tests/test_metal_ops.cpp:20-27 expects.

#include "lite_ssm/ops.hpp"
#include "lssm.h"
#include "mirror.hpp"

#include <cstdint>
#include <stdexcept>
#include <string>

namespace lite_ssm {

struct MetalOps::Impl {
    lssm_ctx*   ctx = nullptr;
    std::string path;

    lssm_ctx* get() {
        if (!ctx && lssm_ctx_create(&ctx, nullptr) != LSSM_OK) {
            ctx = nullptr;
            throw std::runtime_error(std::string("MetalOps: ") + lssm_last_error());
        }
        return ctx;
    }
};

namespace {

inline void check(int rc) {
    if (rc != LSSM_OK) throw std::runtime_error(lssm_last_error());
}

template <class P>
inline P* at(MetalBufferHandle h, std::size_t off) {
    return h ? reinterpret_cast<P*>(static_cast<std::uint8_t*>(h) + off) : nullptr;
}
// every buffer an op names is brought up to date on the device first (the
// host's writes uploaded, its host view invalidated: allocator.cpp)
inline const void* cv(MetalBufferHandle h, std::size_t off) {
    detail::mirror_sync_for_device(h);
    return at<const void>(h, off);
}
inline void* mv(MetalBufferHandle h, std::size_t off) {
    detail::mirror_sync_for_device(h);
    return at<void>(h, off);
}
inline float* fv(MetalBufferHandle h, std::size_t off) {
    detail::mirror_sync_for_device(h);
    return at<float>(h, off);
}

}  // namespace

MetalOps::MetalOps() : impl_(std::make_unique<Impl>()) {}

MetalOps::~MetalOps() {
    // An open batch is dropped: its queued work finishes on the stream first.
    if (impl_->ctx) lssm_ctx_destroy(impl_->ctx);
}

bool MetalOps::metallib_loaded() const { return lssm_library_loaded() != 0; }

bool MetalOps::has_pipeline(std::string_view name) {
    if (!lssm_library_loaded()) return false;
    return lssm_has_kernel(std::string(name).c_str()) != 0;
}

const std::string& MetalOps::metallib_path() const {
    if (impl_->path.empty()) impl_->path = lssm_library_path();
    return impl_->path;
}

void MetalOps::begin_batch() { check(lssm_begin_batch(impl_->get())); }
void MetalOps::commit_and_wait() { check(lssm_commit_and_wait(impl_->get())); }
bool MetalOps::batch_active() const { return impl_->ctx && lssm_batch_active(impl_->ctx) == 1; }

// ---------------------------------------------------------------------------
// ops.mm:175-231
void MetalOps::rmsnorm_f16(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                           std::size_t w_off, MetalBufferHandle y, std::size_t y_off,
                           RMSNormDims d) {
    check(lssm_rmsnorm_f16(impl_->get(), cv(x, x_off), cv(w, w_off), mv(y, y_off),
                           lssm_rmsnorm_dims{d.rows, d.dim, d.eps}));
}

// ops.mm:232-245
void MetalOps::linear_f16_gemv(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                               std::size_t w_off, MetalBufferHandle y, std::size_t y_off,
                               LinearDims d) {
    check(lssm_linear_f16_gemv(impl_->get(), cv(x, x_off), cv(w, w_off), mv(y, y_off),
                               lssm_linear_dims{d.M, d.N, d.K}));
}

void MetalOps::linear_silu_f16_gemv(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                                    std::size_t w_off, MetalBufferHandle y, std::size_t y_off,
                                    LinearDims d) {
    check(lssm_linear_silu_f16_gemv(impl_->get(), cv(x, x_off), cv(w, w_off), mv(y, y_off),
                                    lssm_linear_dims{d.M, d.N, d.K}));
}

// ops.mm:246-300
void MetalOps::rmsnorm_linear_f16_gemv(MetalBufferHandle x, std::size_t x_off,
                                       MetalBufferHandle w_norm, std::size_t w_norm_off,
                                       MetalBufferHandle w, std::size_t w_off,
                                       MetalBufferHandle y, std::size_t y_off, RMSLinearDims d) {
    check(lssm_rmsnorm_linear_f16_gemv(impl_->get(), cv(x, x_off), cv(w_norm, w_norm_off),
                                       cv(w, w_off), mv(y, y_off),
                                       lssm_rms_linear_dims{d.N, d.K, d.eps}));
}

// ops.mm:301-317
void MetalOps::linear_f16_gemm(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                               std::size_t w_off, MetalBufferHandle y, std::size_t y_off,
                               LinearDims d) {
    check(lssm_linear_f16_gemm(impl_->get(), cv(x, x_off), cv(w, w_off), mv(y, y_off),
                               lssm_linear_dims{d.M, d.N, d.K}));
}

void MetalOps::linear_silu_f16_gemm(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                                    std::size_t w_off, MetalBufferHandle y, std::size_t y_off,
                                    LinearDims d) {
    check(lssm_linear_silu_f16_gemm(impl_->get(), cv(x, x_off), cv(w, w_off), mv(y, y_off),
                                    lssm_linear_dims{d.M, d.N, d.K}));
}

// ops.mm:318-367
void MetalOps::linear_int4_gemv(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                                std::size_t w_packed_off, MetalBufferHandle w_scl,
                                std::size_t w_scales_off, MetalBufferHandle y, std::size_t y_off,
                                LinearDims d) {
    check(lssm_linear_int4_gemv(impl_->get(), cv(x, x_off), cv(w, w_packed_off),
                                cv(w_scl, w_scales_off), mv(y, y_off),
                                lssm_linear_dims{d.M, d.N, d.K}));
}

void MetalOps::linear_int4_gemm(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                                std::size_t w_packed_off, MetalBufferHandle w_scl,
                                std::size_t w_scales_off, MetalBufferHandle y, std::size_t y_off,
                                LinearDims d) {
    check(lssm_linear_int4_gemm(impl_->get(), cv(x, x_off), cv(w, w_packed_off),
                                cv(w_scl, w_scales_off), mv(y, y_off),
                                lssm_linear_dims{d.M, d.N, d.K}));
}

// ops.mm:368-443
void MetalOps::silu_f16(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle y,
                        std::size_t y_off, uint32_t n) {
    check(lssm_silu_f16(impl_->get(), cv(x, x_off), mv(y, y_off), n));
}

void MetalOps::add_inplace_f16(MetalBufferHandle y, std::size_t y_off, MetalBufferHandle x,
                               std::size_t x_off, uint32_t n) {
    check(lssm_add_inplace_f16(impl_->get(), mv(y, y_off), cv(x, x_off), n));
}

void MetalOps::split_silu_xBC_f16(MetalBufferHandle xBC, std::size_t xBC_off,
                                  MetalBufferHandle x_out, std::size_t x_off,
                                  MetalBufferHandle B_out, std::size_t B_off,
                                  MetalBufferHandle C_out, std::size_t C_off, uint32_t L,
                                  uint32_t d_inner, uint32_t d_state, uint32_t n_groups) {
    check(lssm_split_silu_xBC_f16(impl_->get(), cv(xBC, xBC_off), mv(x_out, x_off),
                                  mv(B_out, B_off), mv(C_out, C_off), L, d_inner, d_state,
                                  n_groups));
}

void MetalOps::silu_gated_f16(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle gate,
                              std::size_t gate_off, MetalBufferHandle y, std::size_t y_off,
                              uint32_t n) {
    check(lssm_silu_gated_f16(impl_->get(), cv(x, x_off), cv(gate, gate_off), mv(y, y_off), n));
}

// ops.mm:444-507
void MetalOps::causal_conv1d_f16(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle w,
                                 std::size_t w_off, MetalBufferHandle bias, std::size_t bias_off,
                                 MetalBufferHandle y, std::size_t y_off, Conv1dDims d) {
    check(lssm_causal_conv1d_f16(impl_->get(), cv(x, x_off), cv(w, w_off), cv(bias, bias_off),
                                 mv(y, y_off), lssm_conv1d_dims{d.B, d.L, d.D, d.K}));
}

void MetalOps::causal_conv1d_update_f16(MetalBufferHandle x_new, std::size_t x_off,
                                        MetalBufferHandle state, std::size_t state_off,
                                        MetalBufferHandle w, std::size_t w_off,
                                        MetalBufferHandle bias, std::size_t bias_off,
                                        MetalBufferHandle y, std::size_t y_off, Conv1dDims d) {
    check(lssm_causal_conv1d_update_f16(impl_->get(), cv(x_new, x_off), mv(state, state_off),
                                        cv(w, w_off), cv(bias, bias_off), mv(y, y_off),
                                        lssm_conv1d_dims{d.B, d.L, d.D, d.K}));
}

void MetalOps::seed_conv_state_f16(MetalBufferHandle xBC, std::size_t xBC_off,
                                   MetalBufferHandle state, std::size_t state_off, uint32_t L,
                                   uint32_t D, uint32_t K) {
    check(lssm_seed_conv_state_f16(impl_->get(), cv(xBC, xBC_off), mv(state, state_off), L, D, K));
}

// ops.mm:508-547
void MetalOps::inproj_fused_f16(MetalBufferHandle normed, std::size_t normed_off,
                                MetalBufferHandle W_in, std::size_t w_in_off,
                                MetalBufferHandle W_conv, std::size_t w_conv_off,
                                MetalBufferHandle conv_b, std::size_t conv_b_off,
                                MetalBufferHandle proj_z, std::size_t z_off,
                                MetalBufferHandle ssd_x, std::size_t x_off,
                                MetalBufferHandle ssd_B, std::size_t b_off,
                                MetalBufferHandle ssd_C, std::size_t c_off,
                                MetalBufferHandle proj_dt, std::size_t dt_off,
                                MetalBufferHandle proj_xBC, std::size_t xBC_off,
                                FusedInProjDims d) {
    check(lssm_inproj_fused_f16(
        impl_->get(), cv(normed, normed_off), cv(W_in, w_in_off), cv(W_conv, w_conv_off),
        cv(conv_b, conv_b_off), mv(proj_z, z_off), mv(ssd_x, x_off), mv(ssd_B, b_off),
        mv(ssd_C, c_off), mv(proj_dt, dt_off), mv(proj_xBC, xBC_off),
        lssm_fused_inproj_dims{d.L, d.d_model, d.d_inner, d.d_state, d.n_groups, d.n_heads,
                               d.d_conv, d.proj_dim}));
}

// ops.mm:548-588
void MetalOps::ssd_chunked_f16(MetalBufferHandle X, std::size_t X_off, MetalBufferHandle B,
                               std::size_t B_off, MetalBufferHandle C, std::size_t C_off,
                               MetalBufferHandle dt_raw, std::size_t dt_off,
                               MetalBufferHandle dt_bias, std::size_t db_off,
                               MetalBufferHandle A_log, std::size_t A_off,
                               MetalBufferHandle D_skip, std::size_t D_off, MetalBufferHandle Y,
                               std::size_t Y_off, MetalBufferHandle state_io, std::size_t S_off,
                               SSDDims d) {
    check(lssm_ssd_chunked_f16(
        impl_->get(), cv(X, X_off), cv(B, B_off), cv(C, C_off), cv(dt_raw, dt_off),
        cv(dt_bias, db_off), cv(A_log, A_off), cv(D_skip, D_off), mv(Y, Y_off),
        fv(state_io, S_off),
        lssm_ssd_dims{d.L, d.H, d.P, d.N, d.n_groups, d.chunk_size, d.dt_min, d.dt_max, d.has_D}));
}

// ops.mm:589-620
void MetalOps::ssd_step_f16(MetalBufferHandle x, std::size_t x_off, MetalBufferHandle B,
                            std::size_t B_off, MetalBufferHandle C, std::size_t C_off,
                            MetalBufferHandle dt_raw, std::size_t dt_off,
                            MetalBufferHandle dt_bias, std::size_t db_off,
                            MetalBufferHandle A_log, std::size_t A_off, MetalBufferHandle D_skip,
                            std::size_t D_off, MetalBufferHandle state, std::size_t S_off,
                            MetalBufferHandle y, std::size_t y_off, SSDStepDims d) {
    check(lssm_ssd_step_f16(
        impl_->get(), cv(x, x_off), cv(B, B_off), cv(C, C_off), cv(dt_raw, dt_off),
        cv(dt_bias, db_off), cv(A_log, A_off), cv(D_skip, D_off), fv(state, S_off),
        mv(y, y_off),
        lssm_ssd_step_dims{d.H, d.P, d.N, d.n_groups, d.dt_min, d.dt_max, d.has_D}));
}

}  // namespace lite_ssm

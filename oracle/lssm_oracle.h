/*
 * lssm_oracle.h — CPU restatement of lite-ssm's Metal kernels (TEST INFRASTRUCTURE).
 *
 * This library is the parity oracle and the timed CPU baseline.  It is never
 * part of the product path: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it, and only as a checker.
 *
 * Conventions (restated from shaders/common.metal:4-9):
 *   - activations are stored in the activation dtype (fp16 in the reference;
 *     bf16 / fp32 are this build's extensions); all math is fp32;
 *   - every reduction (dot products, sums of squares, the A*dt cumsum) is
 *     accumulated in double here, i.e. the exact value the reference's fp32
 *     reductions approximate in some unspecified order;
 *   - r(v) = round-to-nearest-even into the activation dtype, applied at the
 *     same points where the reference stores a `half`.
 *
 * Every function cites the reference file:line it restates.
 */
#ifndef LSSM_ORACLE_H
#define LSSM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/lssm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* scalar conversions (RNE); bit-level, no compiler half type needed */
uint16_t orc_f2h(float f);
float    orc_h2f(uint16_t h);
uint16_t orc_f2b(float f);
float    orc_b2f(uint16_t b);
void     orc_f32_to_act(const float* in, void* out, size_t n, int dt);
void     orc_act_to_f32(const void* in, float* out, size_t n, int dt);

/* weight format helpers */
size_t orc_wfmt_group(int wfmt);                 /* elements per scale group      */
size_t orc_packed_nbytes(int wfmt, size_t N, size_t K, int act); /* whole tensor */
void   orc_dequant(const void* w, const void* s, float* out, uint32_t N, uint32_t K,
                   int wfmt, int act);
/* symmetric per-group absmax quantizer (tools/export_mamba2.py:68-103 generalised):
 * w_f32 [N,K] -> packed [..] + fp16 scales [N*K/group] */
void   orc_quantize(const float* w, uint32_t N, uint32_t K, int wfmt, uint8_t* packed,
                    uint16_t* scales);

/* kernels */
void orc_rmsnorm(const void* x, const void* w, void* y, uint32_t rows, uint32_t dim,
                 float eps, int act);
void orc_linear(const void* x, uint32_t x_stride, const void* w, const void* s, void* y,
                uint32_t y_stride, const void* residual, uint32_t M, uint32_t N, uint32_t K,
                int wfmt, int act, int epi, int round_dequant);
void orc_silu(const void* x, void* y, uint32_t n, int act);
void orc_add_inplace(void* y, const void* x, uint32_t n, int act);
void orc_silu_gated(const void* x, const void* gate, void* y, uint32_t n, int act);
void orc_split_silu_xbc(const void* xBC, void* x, void* B, void* C, uint32_t rows,
                        uint32_t d_inner, uint32_t d_state, uint32_t n_groups, int act);
void orc_conv1d(const void* x, const void* w, const void* bias, void* y, uint32_t B,
                uint32_t L, uint32_t D, uint32_t K, int act);
void orc_conv1d_update(const void* x_new, void* state, const void* w, const void* bias,
                       void* y, uint32_t B, uint32_t D, uint32_t K, int act);
void orc_conv1d_seed(const void* xBC, void* state, uint32_t B, uint32_t L, uint32_t D,
                     uint32_t K, int act);
void orc_gated_rmsnorm(const void* z, const void* y, const void* w, void* out,
                       uint32_t rows, uint32_t dim, float eps, int act);
void orc_inproj_fused(const void* normed, const void* W_in, const void* W_conv,
                      const void* conv_b, void* proj_z, void* ssd_x, void* ssd_B,
                      void* ssd_C, void* proj_dt, void* proj_xBC,
                      lssm_fused_inproj_dims d, int act);
void orc_ssd_chunked(const void* X, const void* B, const void* C, const void* dt_raw,
                     const void* dt_bias, const void* A_log, const void* D_skip, void* Y,
                     float* state, uint32_t batch, lssm_ssd_dims d, int act);
void orc_ssd_step(const void* x, const void* B, const void* C, const void* dt_raw,
                  const void* dt_bias, const void* A_log, const void* D_skip, float* state,
                  void* y, uint32_t batch, lssm_ssd_step_dims d, int act);
void orc_embed(const void* table, const int32_t* ids, void* out, uint32_t n,
               uint32_t d_model, int act);
void orc_argmax(const void* logits, int32_t* ids, uint32_t rows, uint32_t vocab, int act);

/* whole model (Mamba2Model::forward_prefill / forward_step / compute_logits,
 * mamba2_block.cpp:51-327, mamba2_model.cpp:144-175) on host pointers.
 * conv_state [n_layer, batch, xBC_dim, d_conv] act; ssd_state [n_layer, batch, H, P, N] f32.
 * logits [batch, vocab] act. */
typedef struct {
    lssm_model_config cfg;
    const void* embed;
    const void* norm_f;
    const void* lm_head;
    const lssm_layer_weights* layers;
} orc_model;

void orc_model_prefill(const orc_model* m, void* conv_state, float* ssd_state,
                       const int32_t* ids, uint32_t batch, uint32_t L, void* logits);
void orc_model_decode(const orc_model* m, void* conv_state, float* ssd_state,
                      const int32_t* ids, uint32_t batch, void* logits);
/* One layer (Mamba2Model::run_block, mamba2_block.cpp:51-290) on caller rows:
 * hidden [batch * L, d_model] act is updated in place, the layer's slabs of
 * conv_state / ssd_state ([n_layer, batch, ...]) too.  decode = 1: one token per
 * sequence (L == 1, conv update + SSD step). */
void orc_model_block(const orc_model* m, uint32_t li, void* hidden, void* conv_state, float* ssd_state,
                     uint32_t batch, uint32_t L, int decode);
/* norm_f + lm_head of `rows` hidden rows (mamba2_model.cpp:144-175) -> logits [rows, vocab]. */
void orc_model_logits(const orc_model* m, const void* rows_h, uint32_t rows, void* logits);

int orc_num_threads(void);
void orc_set_num_threads(int n);
/* summation of the linears: 0 = double (default), 1 = float32 */
void orc_set_accum(int f32);
int orc_accum(void);

#ifdef __cplusplus
}
#endif
#endif

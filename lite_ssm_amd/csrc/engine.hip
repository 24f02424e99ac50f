// engine.hip — whole-model Mamba-2 prefill / decode on one GPU.
//
// Runs the op sequence of Mamba2Model::run_block (mamba2_block.cpp:51-290),
// forward_prefill / forward_step (:296-327) and compute_logits
// (mamba2_model.cpp:144-175), generalised to a batch of sequences, with:
//   - decode fused to 3 kernels per layer for batch <= 4:
//       [RMSNorm + in_proj GEMV + conv update + SiLU split]
//       [SSD step + SiLU(z) gate]
//       [gated RMSNorm + out_proj GEMV + residual add]
//     (batch > 4 runs the MFMA GEMM with separate norm / conv kernels);
//   - prefill on the MFMA GEMM and the MFMA chunked scan;
//   - embedding gather and greedy argmax on the device, so a decode step has
//     no host round trip and can be captured once into a HIP graph.
// Every intermediate is rounded at the same points as the reference's
// unfused kernels.
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "internal.hpp"

using namespace lssm;

namespace {
constexpr float RMS_EPS = 1e-5f;   // mamba2_block.cpp:45
constexpr float DT_MIN = 1e-6f;    // mamba2_block.cpp:43
constexpr float DT_MAX = 1e6f;     // mamba2_block.cpp:44
}  // namespace

struct lssm_engine {
    lssm_ctx* ctx = nullptr;
    lssm_model_config cfg{};
    uint32_t d_model = 0, d_inner = 0, xbc = 0, proj = 0, H = 0, P = 0, N = 0, G = 0, K = 0,
             vocab = 0, GN = 0;
    int act = 0, wfmt = 0;
    size_t es = 2;
    const void* embed = nullptr;
    const void* norm_f = nullptr;
    const void* lm_head = nullptr;
    std::vector<lssm_layer_weights> layers;
    uint32_t max_batch = 0, max_seq = 0;

    std::vector<void*> allocs;
    // prefill buffers [max_batch * max_seq, ...]
    void* hidden = nullptr;
    void* normed = nullptr;
    void* projb = nullptr;
    void* xbc_act = nullptr;
    void* ys = nullptr;
    void* gn = nullptr;
    // decode buffers [max_batch, ...]
    void* d_hidden = nullptr;
    void* d_normed = nullptr;
    void* d_proj = nullptr;
    void* d_z = nullptr;
    void* d_xbc = nullptr;
    void* d_dt = nullptr;
    void* d_g = nullptr;
    void* d_gn = nullptr;      // also the packed x rows of the MFMA decode GEMV (launch_mma_pack)
    void* logits = nullptr;
    // short fp16 prefills (1 < L <= 16, dense fp16 weights): the fused in_proj
    // + conv + SiLU split's outputs [max_batch * 16, .] (mamba2_block.cpp:98)
    void* f_z = nullptr;
    void* f_x = nullptr;
    void* f_B = nullptr;
    void* f_C = nullptr;
    void* f_dt = nullptr;
    void* f_xbc = nullptr;
    bool short_fused() const { return act == LSSM_F16 && wfmt == LSSM_W_DENSE; }
    void* conv_state = nullptr;
    float* ssd_state = nullptr;
    void* argmax_scratch = nullptr;
    size_t argmax_scratch_bytes = 0;
    // batch-1 greedy id from the lm_head launch's per-block partials
    // (LSSM_FUSED_ARGMAX=0: the two-pass argmax over the stored logits)
    bool fuse_argmax = true;
    float* gram = nullptr;     // prefill: the chunks' C B^T tiles, shared by a group's heads
    float* seg = nullptr;      // prefill: the chunked scan's segment workspace
    // prefill: the split-K slices of GEMMs whose grid leaves most CUs idle
    float* gemm_ws = nullptr;
    // prefill: the gated RMSNorm fused into the chunked scan's Y stores (which
    // then hold r(g w), g = r(silu(z) r(y))) with each row's sums of g^2 per
    // scan block (gpart) and 1 / rms per row (g_rs), applied by out_proj to
    // its fp32 sums; where the scan cannot fuse it, the separate gated
    // RMSNorm runs.  LSSM_FUSED_GATED_NORM=0 at creation turns it off.
    float* gpart = nullptr;
    float* g_rs = nullptr;
    bool fuse_gated_norm = true;
    // prefill: the next layer's pre-mixer RMSNorm folded into out_proj's
    // epilogue, which then also writes normed = r(h w) and each row's sums of
    // h^2 per 128 columns (hpart); 1 / rms per row (h_rs) is applied by the
    // next in_proj to its fp32 sums.  Where the GEMM cannot fold it (and for
    // the first layer) the separate RMSNorm runs.  Off by default (measured no
    // faster at 4 x 4096: the epilogue's extra stores and the row scale cost
    // what the norm pass did); LSSM_FOLD_PRE_NORM=1 at creation turns it on.
    float* hpart = nullptr;
    float* h_rs = nullptr;
    bool fold_pre_norm = false;
    // prefill of a batch of long sequences as two halves, the second on a
    // stream of the engine's own (default priority) forked from and joined to
    // the context's by events, each half with its own segment and split-K
    // workspace: while one half's latency-bound chunked scan leaves CUs idle,
    // the other half's GEMMs take them (2.7B at 4 x 4096: 109.4 -> 106.9 ms).
    // LSSM_SPLIT_PREFILL=0 at creation keeps one stream.
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    // one long sequence: its two halves in time, the second on that stream a
    // layer behind, each of its layers after the first half's scan of the
    // layer (the SSD state and conv window it continues from): one event a
    // layer (8B at 1 x 8192: 111.5 -> 106.4 ms)
    std::vector<hipEvent_t> ev_layer;
    float* seg2 = nullptr;
    float* gemm_ws2 = nullptr;
    bool split_prefill = true;
    // batch-1 decode: in_proj, the SSD step (and out_proj) in one launch
    // (tagged words of each layer's projection and gated SSD output; the tag
    // is a count the embedding advances on every step that uses tagged
    // words, so consecutive uses of a word carry different tags).  Both are zeroed once at creation
    // and never reset apart.  On by default when the SSD step has work items
    // (32 state rows each) for at least half the CUs: the 2.7B shape (160
    // items) decodes at 1131 tok/s fused against 1095 in three launches, the
    // 130M int8 fp16 shape (48 items, the rest of the launch's workgroups idle
    // while they wait) at 4221 against 4404.  LSSM_FUSED_SSD=0 / 1 at creation
    // turns it off / on.
    uint64_t* xfer = nullptr;
    uint32_t* seq = nullptr;
    bool fuse_ssd = true;
    // decode batches of 3..16 on the normalise-on-load path: the SSD step in
    // the in_proj launch likewise (launch_inproj_ssd_decode_mma), with the
    // rows' words in xfer_b ([n_layer][xfer_b_rows][proj]); the tag then
    // advances on those steps too.  Bit-identical, but slower than the
    // separate SSD step launch (2.7B batch 4: 17.6 against 8.8 + 6.7 us; batch
    // 16: 38.8 against 9.8 + 16.1 us): one workgroup per CU keeps too little
    // state traffic in flight, where the separate launch runs thousands of
    // small ones.  Off by default; LSSM_FUSED_SSD_B=1 at creation turns it on.
    uint64_t* xfer_b = nullptr;
    uint32_t xfer_b_rows = 0;
    bool fuse_ssd_b = false;
    // decode batches from this many rows pack x once per linear (launch_mma_pack);
    // LSSM_PACK_MIN_ROWS at creation overrides it; parts_min_rows is the same
    // for the normalise-on-load path below (LSSM_PARTS_MIN_ROWS)
    uint32_t pack_min_rows = 8;
    uint32_t parts_min_rows = 3;
    // packed decode batches whose two linears both take the single-pass MFMA
    // GEMV (and the partial counts it reads): out_proj also writes r(h w),
    // w the next layer's norm weight, in that GEMV's fragment order with each
    // row's sums of squares of h over every 16 columns (h_frag, h_part), the
    // SSD step r(y w') likewise over every 32 (g_frag, g_part), and the
    // linears scale their fp32 sums by the rows' 1 / rms, so no pack launch
    // runs after the first layer's in_proj (which packs r(x w) likewise).
    // LSSM_NOPACK at creation: 0 = off; 2 = a pack launch of r(x w) with one
    // partial a row before every linear (the GEMV's scaling on its own)
    int nopack = 1;
    void* h_frag = nullptr;
    void* g_frag = nullptr;
    float* h_part = nullptr;
    float* g_part = nullptr;
    // LSSM_FUSED_MIXER=1: out_proj in the same launch too (bit-identical; on
    // the 2.7B shape it measures ~3 % slower than a separate out_proj launch:
    // its two waits on other workgroups' words cost more than one kernel
    // boundary), so it is off by default
    bool fuse_mixer = false;
    mutable uint32_t fused_layers = 0;   // of the last decode step issued: SSD in the in_proj launch
    mutable uint32_t mixer_layers = 0;   //   the whole mixer (+ out_proj) in one launch
    size_t xfer_words() const { return (size_t)proj + d_inner; }   // per layer: [z|xBC|dt] + gated y

    // parity hook (lssm_engine_set_trace): hidden rows entering each layer
    // and after the last one, [n_layer + 1][rows][d_model], or null
    void* trace = nullptr;
    size_t trace_cap = 0;
    // greedy-id history (lssm_engine_set_id_log): every decode step, eager or
    // graph-replayed, appends its ids as row seq[1] of id_log [id_log_cap][batch]
    int32_t* id_log = nullptr;
    uint32_t id_log_cap = 0;
    size_t trace_bytes(uint32_t rows) const { return (size_t)(cfg.n_layer + 1) * rows * d_model * es; }
    hipError_t trace_rows(uint32_t slot, const void* h, uint32_t rows) const {
        if (!trace) return hipSuccess;
        const size_t n = (size_t)rows * d_model * es;
        return hipMemcpyAsync((char*)trace + (size_t)slot * n, h, n, hipMemcpyDeviceToDevice, st());
    }

    // decode graphs of one step and of graph_unroll steps in a row (each
    // graph launch costs a gap of ~8 us before its first kernel; steps are
    // replayed unroll at a time, the rest one at a time).  2.7B batch 1: 1130
    // tok/s at one step per launch, 1137 at 4, 1138 at 8; batch 8: 4497,
    // 4511, 4435 (8-step graphs of the batched path measure slower).
    // LSSM_GRAPH_UNROLL at creation overrides the count (1: one step a launch).
    hipGraph_t graph[2] = {nullptr, nullptr};
    hipGraphExec_t graph_exec[2] = {nullptr, nullptr};
    uint32_t graph_unroll = 4;
    const int32_t* g_ids = nullptr;
    int32_t* g_next = nullptr;
    uint32_t g_batch = 0;
    void drop_graphs() {
        for (int i = 0; i < 2; ++i) {
            if (graph_exec[i]) (void)hipGraphExecDestroy(graph_exec[i]);
            if (graph[i]) (void)hipGraphDestroy(graph[i]);
            graph_exec[i] = nullptr;
            graph[i] = nullptr;
        }
    }

    ~lssm_engine() {
        drop_graphs();
        if (side) {
            (void)hipStreamSynchronize(side);
            (void)hipStreamDestroy(side);
        }
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_join) (void)hipEventDestroy(ev_join);
        for (hipEvent_t ev : ev_layer) (void)hipEventDestroy(ev);
        for (void* p : allocs) (void)hipFree(p);
    }

    int alloc(void** p, size_t n) {
        if (n == 0) n = 16;
        hipError_t e = hipMalloc(p, n);
        if (e != hipSuccess) return set_error(LSSM_EDEVICE, "engine: hipMalloc(%zu): %s", n, hipGetErrorString(e));
        allocs.push_back(*p);
        return LSSM_OK;
    }

    char* conv_layer(uint32_t li) const {
        return (char*)conv_state + (size_t)li * max_batch * xbc * K * es;
    }
    float* ssd_layer(uint32_t li) const { return ssd_state + (size_t)li * max_batch * H * P * N; }

    hipStream_t st() const { return ctx->stream; }

    // Decode-side linear (one token per sequence): quantized weights keep the
    // GEMV rule at any batch, as the reference's decode (mamba2_block.cpp:111,
    // 248: decode || L == 1 -> gemv) does per sequence; dense weights take the
    // GEMM kernels above 4 rows (the same arithmetic).
    hipError_t linear(const void* x, uint32_t xs, const void* w, const void* s, void* y, uint32_t ysd,
                      const void* res, uint32_t M, uint32_t Nn, uint32_t Kk, int fmt, int epi) const {
        if (M <= 4 || fmt != LSSM_W_DENSE) {
            GemvArgs g{x, xs, w, s, y, ysd, res, nullptr, 0.0f, M, Nn, Kk, fmt, act, epi};
            return launch_gemv(st(), g);
        }
        GemmArgs g{x, xs, w, s, y, ysd, res, M, Nn, Kk, fmt, act, epi, 1};
        if (act == LSSM_F32) return launch_gemm_simple(st(), g);
        return launch_gemm(st(), g);
    }

    // Logits of `rows` hidden rows (row stride xs) -> logits, then argmax.
    hipError_t logits_argmax(const void* x, uint32_t xs, uint32_t rows, int32_t* next) const {
        hipError_t e;
        if (rows <= 4 && gemv_max_rows(d_model, LSSM_W_DENSE, act) >= 1) {
            GemvArgs g{x, xs, lm_head, nullptr, logits, vocab, nullptr, norm_f, RMS_EPS, rows, vocab,
                       d_model, LSSM_W_DENSE, act, LSSM_EPI_NONE};
            // one row: the argmax's first pass folded into the lm_head launch
            if (rows == 1 && fuse_argmax) {
                e = launch_gemv_argmax(st(), g, next, argmax_scratch, argmax_scratch_bytes);
                if (e != hipErrorNotSupported) return e;
            }
            e = launch_gemv(st(), g);
        } else {
            e = launch_rmsnorm(st(), x, xs, norm_f, d_normed, d_model, rows, d_model, RMS_EPS, act);
            if (e == hipSuccess)
                e = linear(d_normed, d_model, lm_head, nullptr, logits, vocab, nullptr, rows, vocab,
                           d_model, LSSM_W_DENSE, LSSM_EPI_NONE);
        }
        if (e == hipSuccess) e = launch_argmax(st(), logits, next, rows, vocab, act, argmax_scratch);
        return e;
    }

    // One decode step: ids -> next (all on device).  mamba2_block.cpp:317-327.
    hipError_t decode(const int32_t* ids, uint32_t B, int32_t* next) const {
        // fused RMSNorm + linear kernels: the VALU GEMV up to 4 rows, the MFMA
        // GEMV for decode batches of the shapes it takes
        const bool fused_in = (B <= 4 && (int)B <= gemv_max_rows(d_model, wfmt, act)) ||
                              (B >= 2 && gemv_mma_takes(B, proj, d_model, wfmt, act));
        const bool fused_out = (B <= 4 && gemv_max_rows(d_inner, wfmt, act) >= 1) ||
                               (B >= 2 && gemv_mma_takes(B, d_model, d_inner, wfmt, act));
        // x is normalised and packed once per linear (into d_gn) instead of by
        // every block of the MFMA GEMV, whose staging is issue-bound: from 8
        // rows (below that the extra launch costs what it saves), or from 3
        // when both linears take the single-pass kernel with its partial sums
        // of squares (frag_parts: one pack launch per step, not per linear;
        // 2.7B at batch 4: 2573 against 2454 tok/s, batch 6: 3548 against 3230)
        const bool mmx_in = d_model % 128 == 0 && gemv_mmx_takes(B, proj, d_model, wfmt, act);
        const bool mmx_out = d_inner % 128 == 0 && gemv_mmx_takes(B, d_model, d_inner, wfmt, act);
        const uint32_t np_h = gemv_mmx_parts(B, d_model, d_inner, wfmt, act);
        const uint32_t np_g = ssd_step_parts(H, P, N, act);
        const bool parts_ok = mmx_in && mmx_out && np_h != 0 && np_g != 0;
        const uint32_t PACK_MIN_ROWS = nopack != 0 && parts_ok ? parts_min_rows : pack_min_rows;
        const bool pack_in = B >= PACK_MIN_ROWS && d_model % 128 == 0 && gemv_mma_takes(B, proj, d_model, wfmt, act);
        const bool pack_out = B >= PACK_MIN_ROWS && d_inner % 128 == 0 &&
                              gemv_mma_takes(B, d_model, d_inner, wfmt, act);
        // packed in the single-pass kernel's fragment order when it takes the call
        const bool frag_in = pack_in && mmx_in;
        const bool frag_out = pack_out && mmx_out;
        // x = r(x w) in fragment order with partial sums of squares (nopack)
        const bool frag_parts = nopack == 1 && frag_in && frag_out && parts_ok;
        const bool raw_pack = nopack == 2 && frag_in && frag_out;
        // the batched in_proj + SSD launch (its launcher checks the rest)
        const bool fuse_b = fuse_ssd_b && frag_parts && B >= 2 && B <= xfer_b_rows;
        // the step tag advances on the steps that use tagged words (batch 1
        // fused, or fuse_b): every use of a word then finds an older tag
        hipError_t e = launch_embed(st(), embed, ids, d_hidden, B, d_model, vocab, act, ctx->status,
                                    (fuse_ssd && B == 1) || fuse_b ? seq : nullptr);
        fused_layers = 0;
        mixer_layers = 0;
        if (e == hipSuccess) e = trace_rows(0, d_hidden, B);
        for (uint32_t li = 0; li < cfg.n_layer && e == hipSuccess; ++li) {
            if (li > 0) e = trace_rows(li, d_hidden, B);
            if (e != hipSuccess) break;
            const lssm_layer_weights& w = layers[li];
            char* cs = conv_layer(li);
            bool ssd_done = false;   // the SSD step ran inside the in_proj launch
            bool out_done = false;   //   and out_proj too
            if (fused_in) {
                InprojDecodeArgs a;
                a.g = GemvArgs{d_hidden, d_model, w.in_proj_w, w.in_proj_s, nullptr, 0, nullptr,
                               w.norm_w, RMS_EPS, B, proj, d_model, wfmt, act, LSSM_EPI_NONE};
                a.d_inner = d_inner;
                a.xbc = xbc;
                a.H = H;
                a.dconv = K;
                a.conv_state = cs;
                a.conv_w = w.conv1d_w;
                a.conv_b = w.conv1d_b;
                a.z = d_z;
                a.xbc_act = d_xbc;
                a.dt = d_dt;
                if (B == 1 && fuse_ssd) {
                    uint64_t* lx = xfer + (size_t)li * xfer_words();
                    const SsdFuseArgs f{lx, seq, 0u, ssd_layer(li), w.A_log, w.dt_bias, w.D,
                                        d_g, P, N, G, DT_MIN, DT_MAX, ctx->status};
                    if (fused_out && fuse_mixer) {
                        const OutprojFuseArgs o{w.out_proj_w, w.out_proj_s, w.mixer_norm_w, RMS_EPS, d_hidden,
                                                reinterpret_cast<uint32_t*>(lx + proj), d_model};
                        out_done = ssd_done = launch_layer_decode(st(), a, f, o, e);
                    }
                    if (!ssd_done) ssd_done = launch_inproj_ssd_decode(st(), a, f, e);
                    fused_layers += ssd_done ? 1u : 0u;
                    mixer_layers += out_done ? 1u : 0u;
                }
                if (!ssd_done && pack_in) {
                    if (frag_parts && li > 0) {
                        a.g.xpack = h_frag;                    // the previous out_proj's
                        a.g.xpart = h_part;
                        a.g.nparts = np_h;
                    } else {
                        // (the first layer of frag_parts packs r(x w) too: every
                        // linear then rounds at the same point)
                        const bool raw = raw_pack || frag_parts;
                        e = launch_mma_pack(st(), d_hidden, d_model, w.norm_w, RMS_EPS, B, d_model, wfmt, act,
                                            d_gn, frag_in, raw ? h_part : nullptr);
                        a.g.xpack = d_gn;
                        if (raw) {
                            a.g.xpart = h_part;
                            a.g.nparts = 4;
                        }
                    }
                }
                if (!ssd_done && e == hipSuccess && fuse_b) {
                    const SsdFuseBArgs fb{xfer_b + (size_t)li * xfer_b_rows * proj, seq, ssd_layer(li), w.A_log,
                                          w.dt_bias, w.D, d_g, g_frag, g_part, w.mixer_norm_w, P, N, G,
                                          DT_MIN, DT_MAX, ctx->status};
                    ssd_done = launch_inproj_ssd_decode_mma(st(), a, fb, e);
                    fused_layers += ssd_done ? 1u : 0u;
                }
                if (!ssd_done && e == hipSuccess) e = launch_inproj_decode(st(), a);
            } else {
                e = launch_rmsnorm(st(), d_hidden, d_model, w.norm_w, d_normed, d_model, B, d_model,
                                   RMS_EPS, act);
                if (e == hipSuccess)
                    e = linear(d_normed, d_model, w.in_proj_w, w.in_proj_s, d_proj, proj, nullptr, B,
                               proj, d_model, wfmt, LSSM_EPI_NONE);
                if (e == hipSuccess)
                    e = launch_conv1d_update_silu(st(), (char*)d_proj + (size_t)d_inner * es, proj, cs,
                                                  w.conv1d_w, w.conv1d_b, d_xbc, xbc, B, xbc, K, act);
            }
            if (e != hipSuccess) break;
            // z / dt live in d_z, d_dt (fused) or inside d_proj (strided)
            const void* z = fused_in ? d_z : d_proj;
            const uint32_t zs = fused_in ? d_inner : proj;
            const void* dt = fused_in ? d_dt : (const void*)((char*)d_proj + (size_t)(d_inner + xbc) * es);
            const uint32_t dts = fused_in ? H : proj;
            SsdArgs s{d_xbc, xbc, (char*)d_xbc + (size_t)d_inner * es, xbc,
                      (char*)d_xbc + (size_t)(d_inner + GN) * es, xbc, dt, dts, w.dt_bias, w.A_log,
                      w.D, d_g, d_inner, ssd_layer(li), B, 1, H, P, N, G, 1, DT_MIN, DT_MAX, 1u, act,
                      z, zs};
            if (frag_parts) {
                s.yfrag = g_frag;
                s.ypart = g_part;
                s.ynorm_w = w.mixer_norm_w;
            }
            if (!ssd_done) e = launch_ssd_step(st(), s);
            if (e != hipSuccess) break;
            if (out_done) continue;
            if (fused_out) {
                GemvArgs g{d_g, d_inner, w.out_proj_w, w.out_proj_s, d_hidden, d_model, d_hidden,
                           w.mixer_norm_w, RMS_EPS, B, d_model, d_inner, wfmt, act, LSSM_EPI_ADD};
                if (frag_parts) {
                    g.xpack = g_frag;                          // the SSD step's
                    g.xpart = g_part;
                    g.nparts = np_g;
                    if (li + 1 < cfg.n_layer) {                // for the next in_proj
                        g.yfrag = h_frag;
                        g.ypart = h_part;
                        g.ynorm_w = layers[li + 1].norm_w;
                    }
                } else if (pack_out) {
                    e = launch_mma_pack(st(), d_g, d_inner, w.mixer_norm_w, RMS_EPS, B, d_inner, wfmt, act, d_gn,
                                        frag_out, raw_pack ? g_part : nullptr);
                    g.xpack = d_gn;
                    if (raw_pack) {
                        g.xpart = g_part;
                        g.nparts = 4;
                    }
                }
                if (e == hipSuccess) e = launch_gemv(st(), g);
            } else {
                e = launch_rmsnorm(st(), d_g, d_inner, w.mixer_norm_w, d_gn, d_inner, B, d_inner,
                                   RMS_EPS, act);
                if (e == hipSuccess)
                    e = linear(d_gn, d_inner, w.out_proj_w, w.out_proj_s, d_hidden, d_model, d_hidden,
                               B, d_model, d_inner, wfmt, LSSM_EPI_ADD);
            }
        }
        if (e == hipSuccess) e = trace_rows(cfg.n_layer, d_hidden, B);
        if (e == hipSuccess) e = logits_argmax(d_hidden, d_model, B, next);
        if (e == hipSuccess && id_log) e = launch_id_log(st(), next, B, id_log, id_log_cap, seq + 1);
        return e;
    }

    // Prefill of B sequences of L tokens (mamba2_block.cpp:296-315).  L == 1
    // follows the reference's 1-token path (GEMV, conv update, SSD step, then
    // the state seed).
    hipError_t prefill(const int32_t* ids, uint32_t B, uint32_t L, int32_t* next) const {
        if (L == 1) {
            hipError_t e = decode_layers_for_prefill1(ids, B);
            if (e == hipSuccess) e = logits_argmax(d_hidden, d_model, B, next);
            return e;
        }
        const uint32_t ck = cfg.chunk_size < L ? (cfg.chunk_size < 64 ? cfg.chunk_size : 64)
                                               : (L < 64 ? L : 64);
        // mamba2_block.cpp:97-98: a short prefill of fp16 weights takes the
        // fused in_proj + conv + SiLU split (its conv reads the unrounded
        // projection, so it rounds differently from the chain below)
        const bool fused = short_fused() && L > 1 && L <= 16;
        const uint32_t R = B * L;
        // two halves on two streams: a batch of at least 8192 rows in
        // sequences of at least 64 tokens (each half's GEMMs still fill the
        // GPU), no debug trace (it reads one stream's rows in order)
        const bool can_split = split_prefill && side && !fused && !trace && act != LSSM_F32;
        const uint32_t b0 = can_split && B >= 2 && L >= 64 && R >= 8192 ? B / 2 : 0;
        // one sequence of at least 8192 tokens: halves in time, on chunk bounds
        const uint32_t th = can_split && B == 1 && L >= 8192 && ev_layer.size() >= cfg.n_layer ? L / 2 / 64 * 64 : 0;
        hipError_t e;
        if (b0 == 0 && th == 0) {
            e = prefill_layers(ids, 0, B, L, 0, L, ck, fused, st(), seg, gemm_ws);
        } else {
            e = hipEventRecord(ev_fork, st());
            if (e == hipSuccess) e = hipStreamWaitEvent(side, ev_fork, 0);
            if (e != hipSuccess) return e;
            if (b0) {
                e = prefill_layers(ids, 0, b0, L, 0, L, ck, fused, st(), seg, gemm_ws);
                if (e == hipSuccess) e = prefill_layers(ids, b0, B - b0, L, 0, L, ck, fused, side, seg2, gemm_ws2);
            } else {
                e = prefill_layers(ids, 0, 1, L, 0, th, ck, fused, st(), seg, gemm_ws, ev_layer.data(), nullptr);
                if (e == hipSuccess)
                    e = prefill_layers(ids, 0, 1, L, th, L - th, ck, fused, side, seg2, gemm_ws2, nullptr,
                                       ev_layer.data());
            }
            // joined whatever happened, so nothing stays queued unordered on the side stream
            hipError_t j = hipEventRecord(ev_join, side);
            if (j == hipSuccess) j = hipStreamWaitEvent(st(), ev_join, 0);
            if (e == hipSuccess) e = j;
        }
        if (e == hipSuccess) e = trace_rows(cfg.n_layer, hidden, R);
        // last position of each sequence: rows (b*L + L-1), stride L*d_model
        if (e == hipSuccess)
            e = logits_argmax((const char*)hidden + (size_t)(L - 1) * d_model * es, L * d_model, B, next);
        return e;
    }

    // The layers of a prefill for tokens t0 .. t0 + L of sequences b0 .. b0 +
    // nb of the batch (sequence length Ls) on stream strm
    // (mamba2_block.cpp:296-315): rows b0 Ls + t0 .. of every row buffer, the
    // sequences' conv / SSD state and Gram tiles, and the given segment and
    // split-K workspaces.  t0 > 0 (one sequence): the prefill continues from
    // the state and conv window that tokens 0 .. t0 left, each layer after
    // the event wait[li]; rec: an event recorded after each layer's scan.
    hipError_t prefill_layers(const int32_t* ids, uint32_t b0, uint32_t nb, uint32_t Ls, uint32_t t0, uint32_t L,
                              uint32_t ck, bool fused, hipStream_t strm, float* segw, float* gws,
                              const hipEvent_t* rec = nullptr, const hipEvent_t* wait = nullptr) const {
        const uint32_t R = nb * L;
        const size_t r0 = (size_t)b0 * Ls + t0;
        char* hid = (char*)hidden + r0 * d_model * es;
        char* nrm = (char*)normed + r0 * d_model * es;
        char* prj = (char*)projb + r0 * proj * es;
        char* xba = (char*)xbc_act + r0 * xbc * es;
        char* yb = (char*)ys + r0 * d_inner * es;
        char* gnb = (char*)gn + r0 * d_inner * es;
        float* grs = g_rs + r0;
        float* hrs = h_rs + r0;
        float* hp = hpart + (size_t)(d_model / 128) * r0;     // this half's [part][nb L] block
        float* gr = gram + ((size_t)b0 * ((Ls + 63) / 64) + t0 / 64) * G * 64 * 64;
        const size_t cofs = (size_t)b0 * xbc * K * es;
        const size_t sofs = (size_t)b0 * H * P * N;
        hipError_t e = launch_embed(strm, embed, ids + r0, hid, R, d_model, vocab, act, ctx->status);
        bool normed_ready = false;   // the previous out_proj wrote nrm and hrs
        for (uint32_t li = 0; li < cfg.n_layer && e == hipSuccess; ++li) {
            const lssm_layer_weights& w = layers[li];
            e = trace_rows(li, hid, R);
            if (e == hipSuccess && !normed_ready)
                e = launch_rmsnorm(strm, hid, d_model, w.norm_w, nrm, d_model, R, d_model, RMS_EPS, act);
            // the scan of this layer; with the gated norm fused into it, in_proj
            // stores r(silu(z)) for the gate
            SsdArgs s{xba, xbc, xba + (size_t)d_inner * es, xbc, xba + (size_t)(d_inner + GN) * es, xbc,
                      prj + (size_t)(d_inner + xbc) * es, proj, w.dt_bias, w.A_log, w.D,
                      yb, d_inner, ssd_layer(li) + sofs, nb, L, H, P, N, G, ck, DT_MIN, DT_MAX, 1u, act,
                      nullptr, 0, gr, segw};
            uint32_t gparts = 0;   // the gated norm runs inside the scan (out_proj scales rows)
            if (fuse_gated_norm && !fused) {
                SsdArgs sg = s;
                sg.z = prj;                                    // z: columns 0 .. d_inner of the projection
                sg.z_stride = proj;
                sg.gnorm_w = w.mixer_norm_w;
                sg.z_silu = true;                              // in_proj stores r(silu(z)) (silu_cols)
                gparts = ssd_chunked_gate_parts(sg);
                if (gparts) {
                    s = sg;
                    s.gpart = gpart + (size_t)gparts * r0;   // this half's [part][nb L] block
                }
            }
            if (e == hipSuccess && !fused) {
                GemmArgs g{nrm, d_model, w.in_proj_w, w.in_proj_s, prj, proj, nullptr, R, proj,
                           d_model, wfmt, act, LSSM_EPI_NONE, 1};
                g.ws = gws;
                g.ws_floats = GEMM_WS_FLOATS;
                g.silu_cols = gparts ? d_inner : 0u;
                g.row_scale = normed_ready ? hrs : nullptr;
                e = (act == LSSM_F32) ? launch_gemm_simple(strm, g) : launch_gemm(strm, g);
            }
            if (e != hipSuccess) break;
            if (fused) {
                e = short_prefill_mixer(li, nb, L, ck);   // (never split)
            } else {
                const char* xbc_pre = prj + (size_t)d_inner * es;
                if (wait) e = hipStreamWaitEvent(strm, wait[li], 0);
                if (e == hipSuccess)
                    e = launch_conv1d(strm, xbc_pre, proj, w.conv1d_w, w.conv1d_b, xba, xbc, nb, L, xbc, K,
                                      act, true, t0 ? conv_layer(li) + cofs : nullptr);
                if (e == hipSuccess)
                    e = launch_conv1d_seed(strm, xbc_pre, proj, conv_layer(li) + cofs, nb, L, xbc, K, act);
                if (e == hipSuccess) {
                    e = launch_ssd_chunked(strm, s);
                    if (e == hipSuccess && gparts)
                        e = launch_rms_from_parts(strm, s.gpart, gparts, R, d_inner, RMS_EPS, grs);
                    if (e == hipSuccess && rec) e = hipEventRecord(rec[li], strm);
                }
                if (e == hipSuccess && !gparts)
                    e = launch_gated_rmsnorm(strm, prj, proj, yb, d_inner, w.mixer_norm_w, gnb, R, d_inner,
                                             RMS_EPS, act);
            }
            if (e == hipSuccess) {
                GemmArgs g{gparts ? yb : gnb, d_inner, w.out_proj_w, w.out_proj_s, hid, d_model, hid, R,
                           d_model, d_inner, wfmt, act, LSSM_EPI_ADD, 1};
                g.ws = gws;
                g.ws_floats = GEMM_WS_FLOATS;
                g.row_scale = gparts ? grs : nullptr;
                normed_ready = false;
                if (fold_pre_norm && !fused && li + 1 < cfg.n_layer) {
                    g.y2 = nrm;
                    g.y2_w = layers[li + 1].norm_w;
                    g.y2_part = hp;
                    normed_ready = gemm_norm_fold_takes(g);
                    if (!normed_ready) g.y2 = nullptr;
                }
                e = (act == LSSM_F32) ? launch_gemm_simple(strm, g) : launch_gemm(strm, g);
                if (e == hipSuccess && normed_ready)
                    e = launch_rms_from_parts(strm, hp, d_model / 128, R, d_model, RMS_EPS, hrs);
            }
        }
        return e;
    }

    // The mixer of layer li for a short fp16 prefill, per sequence as the
    // reference's batch-1 model (mamba2_block.cpp:130-148, then the seed from
    // the pre-conv projection, the chunked scan and the gated norm over the
    // fused op's outputs).  normed holds the layer's normalised input rows.
    hipError_t short_prefill_mixer(uint32_t li, uint32_t B, uint32_t L, uint32_t ck) const {
        const lssm_layer_weights& w = layers[li];
        const lssm_fused_inproj_dims fd{L, d_model, d_inner, N, G, H, K, proj};
        hipError_t e = hipSuccess;
        for (uint32_t b = 0; b < B && e == hipSuccess; ++b) {
            const size_t r0 = (size_t)b * L;
            e = launch_inproj_fused(st(), (const char*)normed + r0 * d_model * es, w.in_proj_w, w.conv1d_w,
                                    w.conv1d_b, (char*)f_z + r0 * d_inner * es, (char*)f_x + r0 * d_inner * es,
                                    (char*)f_B + r0 * GN * es, (char*)f_C + r0 * GN * es,
                                    (char*)f_dt + r0 * H * es, (char*)f_xbc + r0 * xbc * es, fd);
        }
        if (e == hipSuccess) e = launch_conv1d_seed(st(), f_xbc, xbc, conv_layer(li), B, L, xbc, K, act);
        if (e == hipSuccess) {
            SsdArgs s{f_x, d_inner, f_B, GN, f_C, GN, f_dt, H, w.dt_bias, w.A_log, w.D, ys, d_inner,
                      ssd_layer(li), B, L, H, P, N, G, ck, DT_MIN, DT_MAX, 1u, act, nullptr, 0, nullptr, seg};
            e = launch_ssd_chunked(st(), s);
        }
        if (e == hipSuccess)
            e = launch_gated_rmsnorm(st(), f_z, d_inner, ys, d_inner, w.mixer_norm_w, gn, B * L, d_inner, RMS_EPS,
                                     act);
        return e;
    }

    hipError_t decode_layers_for_prefill1(const int32_t* ids, uint32_t B) const {
        // same kernels as a decode step without logits, then the 1-row seed
        hipError_t e = launch_embed(st(), embed, ids, d_hidden, B, d_model, vocab, act, ctx->status);
        for (uint32_t li = 0; li < cfg.n_layer && e == hipSuccess; ++li) {
            const lssm_layer_weights& w = layers[li];
            e = trace_rows(li, d_hidden, B);
            if (e == hipSuccess)
                e = launch_rmsnorm(st(), d_hidden, d_model, w.norm_w, d_normed, d_model, B, d_model, RMS_EPS, act);
            if (e == hipSuccess)
                e = linear(d_normed, d_model, w.in_proj_w, w.in_proj_s, d_proj, proj, nullptr, B, proj,
                           d_model, wfmt, LSSM_EPI_NONE);
            if (e == hipSuccess)
                e = launch_conv1d_update_silu(st(), (char*)d_proj + (size_t)d_inner * es, proj,
                                              conv_layer(li), w.conv1d_w, w.conv1d_b, d_xbc, xbc, B,
                                              xbc, K, act);
            if (e == hipSuccess) e = launch_conv1d_keep_last(st(), conv_layer(li), B * xbc, K, act);
            if (e != hipSuccess) break;
            SsdArgs s{d_xbc, xbc, (char*)d_xbc + (size_t)d_inner * es, xbc,
                      (char*)d_xbc + (size_t)(d_inner + GN) * es, xbc,
                      (char*)d_proj + (size_t)(d_inner + xbc) * es, proj, w.dt_bias, w.A_log, w.D,
                      d_g, d_inner, ssd_layer(li), B, 1, H, P, N, G, 1, DT_MIN, DT_MAX, 1u, act,
                      d_proj, proj};
            e = launch_ssd_step(st(), s);
            if (e == hipSuccess)
                e = launch_rmsnorm(st(), d_g, d_inner, w.mixer_norm_w, d_gn, d_inner, B, d_inner, RMS_EPS, act);
            if (e == hipSuccess)
                e = linear(d_gn, d_inner, w.out_proj_w, w.out_proj_s, d_hidden, d_model, d_hidden, B,
                           d_model, d_inner, wfmt, LSSM_EPI_ADD);
        }
        if (e == hipSuccess) e = trace_rows(cfg.n_layer, d_hidden, B);
        return e;
    }
};

namespace {

int check_engine(lssm_engine* e) {
    if (!e) return set_error(LSSM_EINVAL, "null lssm_engine");
    clear_error();
    return LSSM_OK;
}

int engine_finish(lssm_engine* e, hipError_t err, const char* what) {
    if (err != hipSuccess) return set_error(LSSM_EDEVICE, "%s: %s", what, hipGetErrorString(err));
    return finish(e->ctx, what);
}

}  // namespace

extern "C" {

int lssm_engine_create(lssm_engine** out, lssm_ctx* ctx, const lssm_model_config* cfg,
                       const void* embed, const void* norm_f, const void* lm_head,
                       const lssm_layer_weights* layers, uint32_t max_batch, uint32_t max_seq) {
    LSSM_CHECK_CTX(ctx);
    LSSM_REQUIRE(out && cfg && embed && norm_f && layers, "engine_create: null argument");
    LSSM_REQUIRE(valid_act((int)cfg->act), "engine_create: unknown activation dtype");
    LSSM_REQUIRE(valid_wfmt((int)cfg->wfmt), "engine_create: unknown weight format");
    LSSM_REQUIRE(cfg->n_layer > 0 && cfg->d_model > 0 && cfg->expand > 0 && cfg->d_state > 0 &&
                     cfg->d_conv > 0 && cfg->n_heads > 0 && cfg->d_head > 0 && cfg->vocab_size > 0,
                 "engine_create: zero dimension in config");
    const uint32_t G = cfg->n_groups ? cfg->n_groups : 1;
    const uint32_t d_inner = cfg->expand * cfg->d_model;
    LSSM_REQUIRE(cfg->n_heads * cfg->d_head == d_inner, "engine_create: n_heads * d_head != d_inner");
    LSSM_REQUIRE(cfg->n_heads % G == 0, "engine_create: n_heads must be a multiple of n_groups");
    LSSM_REQUIRE(max_batch >= 1 && max_seq >= 1, "engine_create: max_batch and max_seq must be >= 1");
    if (cfg->wfmt != LSSM_W_DENSE) {
        const uint32_t g = wfmt_group((int)cfg->wfmt);
        LSSM_REQUIRE(cfg->d_model % g == 0 && d_inner % g == 0,
                     "engine_create: d_model and d_inner must be multiples of the group size");
    }
    LSSM_REQUIRE(cfg->d_model % 64 == 0 && d_inner % 64 == 0,
                 "engine_create: d_model and d_inner must be multiples of 64");
    LSSM_REQUIRE(cfg->d_model <= 16384 && d_inner <= 16384, "engine_create: d_model/d_inner > 16384");
    LSSM_REQUIRE(cfg->chunk_size >= 1, "engine_create: chunk_size must be >= 1");
    LSSM_REQUIRE(max_seq <= 65535, "engine_create: max_seq must be <= 65535");

    auto* e = new lssm_engine();
    e->ctx = ctx;
    e->cfg = *cfg;
    e->cfg.n_groups = G;
    e->act = (int)cfg->act;
    e->wfmt = (int)cfg->wfmt;
    e->es = dtype_size(e->act);
    e->d_model = cfg->d_model;
    e->d_inner = d_inner;
    e->G = G;
    e->N = cfg->d_state;
    e->GN = G * cfg->d_state;
    e->xbc = d_inner + 2 * e->GN;
    e->H = cfg->n_heads;
    e->P = cfg->d_head;
    e->proj = d_inner + e->xbc + e->H;
    e->K = cfg->d_conv;
    e->vocab = cfg->vocab_size;
    e->embed = embed;
    e->norm_f = norm_f;
    e->lm_head = lm_head ? lm_head : embed;   // tied lm_head (mamba2_model.cpp:75-83)
    e->layers.assign(layers, layers + cfg->n_layer);
    e->max_batch = max_batch;
    e->max_seq = max_seq;

    const size_t es = e->es;
    const size_t R = (size_t)max_batch * max_seq;
    int rc = LSSM_OK;
    auto A = [&](void** p, size_t n) {
        if (rc == LSSM_OK) rc = e->alloc(p, n);
    };
    A(&e->hidden, R * e->d_model * es);
    A(&e->normed, R * e->d_model * es);
    A(&e->projb, R * e->proj * es);
    A(&e->xbc_act, R * e->xbc * es);
    A(&e->ys, R * d_inner * es);
    A(&e->gn, R * d_inner * es);
    A(&e->d_hidden, (size_t)max_batch * e->d_model * es);
    A(&e->d_normed, (size_t)max_batch * e->d_model * es);
    A(&e->d_proj, (size_t)max_batch * e->proj * es);
    A(&e->d_z, (size_t)max_batch * d_inner * es);
    A(&e->d_xbc, (size_t)max_batch * e->xbc * es);
    A(&e->d_dt, (size_t)max_batch * e->H * es);
    A(&e->d_g, (size_t)max_batch * d_inner * es);
    // (also the packed x rows of the MFMA decode GEMV: up to the next multiple of 16 rows)
    A(&e->d_gn, (size_t)(max_batch + 15) / 16 * 16 * d_inner * es);
    A(&e->logits, (size_t)max_batch * e->vocab * es);
    A(&e->conv_state, (size_t)cfg->n_layer * max_batch * e->xbc * e->K * es);
    A((void**)&e->ssd_state, (size_t)cfg->n_layer * max_batch * e->H * e->P * e->N * sizeof(float));
    // the two-pass argmax: 128 partials per row; the lm_head's fused first
    // pass: a count and up to 1024 partials
    e->argmax_scratch_bytes = std::max((size_t)max_batch * 128 * 8, (size_t)16 + 1024 * 8);
    A(&e->argmax_scratch, e->argmax_scratch_bytes);
    A((void**)&e->gram, ssd_gram_floats(max_batch, max_seq, G) * sizeof(float));
    A((void**)&e->seg, ssd_seg_floats() * sizeof(float));
    A((void**)&e->gemm_ws, GEMM_WS_FLOATS * sizeof(float));
    A((void**)&e->gpart, R * std::max<size_t>((size_t)e->H * e->P / 32, 1) * sizeof(float));
    A((void**)&e->g_rs, R * sizeof(float));
    A((void**)&e->hpart, R * std::max<size_t>(e->d_model / 128, 1) * sizeof(float));
    A((void**)&e->h_rs, R * sizeof(float));
    if (e->short_fused()) {
        const size_t R16 = (size_t)max_batch * 16;
        A(&e->f_z, R16 * d_inner * es);
        A(&e->f_x, R16 * d_inner * es);
        A(&e->f_B, R16 * e->GN * es);
        A(&e->f_C, R16 * e->GN * es);
        A(&e->f_dt, R16 * e->H * es);
        A(&e->f_xbc, R16 * e->xbc * es);
    }
    const size_t xfer_bytes = (size_t)cfg->n_layer * e->xfer_words() * sizeof(uint64_t);
    A((void**)&e->xfer, xfer_bytes);
    if (const char* v = getenv("LSSM_FUSED_SSD_B")) e->fuse_ssd_b = v[0] != '0';
    e->xfer_b_rows = e->fuse_ssd_b && max_batch >= 3 ? std::min<uint32_t>(max_batch, 16u) : 0u;
    const size_t xfer_b_bytes = (size_t)cfg->n_layer * e->xfer_b_rows * e->proj * sizeof(uint64_t);
    if (xfer_b_bytes) A((void**)&e->xfer_b, xfer_b_bytes);
    A((void**)&e->seq, 256);
    // rows up to the next multiple of 16 (the GEMV's row tiles; rows past the
    // batch are read and their results dropped)
    const size_t R16 = (size_t)(max_batch + 15) / 16 * 16;
    const size_t hpb = R16 * std::max<size_t>(e->d_model / 16, 4) * sizeof(float);
    const size_t gpb = R16 * std::max<size_t>(d_inner / 32, 4) * sizeof(float);
    A(&e->h_frag, R16 * e->d_model * es);
    A(&e->g_frag, R16 * d_inner * es);
    A((void**)&e->h_part, hpb);
    A((void**)&e->g_part, gpb);
    if (const char* v = getenv("LSSM_SPLIT_PREFILL")) e->split_prefill = v[0] != '0';
    if ((max_batch >= 2 || max_seq >= 8192) && e->split_prefill) {
        // the second half of a split prefill: its workspaces, stream and events
        A((void**)&e->seg2, ssd_seg_floats() * sizeof(float));
        A((void**)&e->gemm_ws2, GEMM_WS_FLOATS * sizeof(float));
        if (rc == LSSM_OK) {
            hipError_t err = hipStreamCreateWithFlags(&e->side, hipStreamNonBlocking);
            if (err == hipSuccess) err = hipEventCreateWithFlags(&e->ev_fork, hipEventDisableTiming);
            if (err == hipSuccess) err = hipEventCreateWithFlags(&e->ev_join, hipEventDisableTiming);
            for (uint32_t li = 0; max_seq >= 8192 && li < cfg->n_layer && err == hipSuccess; ++li) {
                hipEvent_t ev = nullptr;
                err = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
                if (err == hipSuccess) e->ev_layer.push_back(ev);
            }
            if (err != hipSuccess) rc = set_error(LSSM_EDEVICE, "engine_create: %s", hipGetErrorString(err));
        }
    }
    if (rc == LSSM_OK) {
        hipError_t err = hipMemsetAsync(e->xfer, 0, xfer_bytes, ctx->stream);
        if (err == hipSuccess && xfer_b_bytes) err = hipMemsetAsync(e->xfer_b, 0, xfer_b_bytes, ctx->stream);
        if (err == hipSuccess) err = hipMemsetAsync(e->seq, 0, 256, ctx->stream);
        if (err == hipSuccess) err = hipMemsetAsync(e->h_frag, 0, R16 * e->d_model * es, ctx->stream);
        if (err == hipSuccess) err = hipMemsetAsync(e->g_frag, 0, R16 * d_inner * es, ctx->stream);
        if (err == hipSuccess) err = hipMemsetAsync(e->h_part, 0, hpb, ctx->stream);
        if (err == hipSuccess) err = hipMemsetAsync(e->g_part, 0, gpb, ctx->stream);
        if (err != hipSuccess) rc = set_error(LSSM_EDEVICE, "engine_create: %s", hipGetErrorString(err));
    }
    e->fuse_ssd = (uint64_t)e->H * e->P / 32 * 2 >= num_cus();
    if (const char* v = getenv("LSSM_FUSED_SSD")) e->fuse_ssd = v[0] != '0';
    if (const char* v = getenv("LSSM_FUSED_MIXER")) e->fuse_mixer = v[0] == '1';
    if (const char* v = getenv("LSSM_PACK_MIN_ROWS")) e->pack_min_rows = (uint32_t)strtoul(v, nullptr, 10);
    if (const char* v = getenv("LSSM_PARTS_MIN_ROWS")) e->parts_min_rows = (uint32_t)strtoul(v, nullptr, 10);
    if (const char* v = getenv("LSSM_GRAPH_UNROLL")) e->graph_unroll = (uint32_t)strtoul(v, nullptr, 10);
    if (const char* v = getenv("LSSM_NOPACK")) e->nopack = (int)strtol(v, nullptr, 10);
    if (const char* v = getenv("LSSM_FUSED_GATED_NORM")) e->fuse_gated_norm = v[0] != '0';
    if (const char* v = getenv("LSSM_FOLD_PRE_NORM")) e->fold_pre_norm = v[0] != '0';
    if (const char* v = getenv("LSSM_FUSED_ARGMAX")) e->fuse_argmax = v[0] != '0';
    if (rc != LSSM_OK) {
        delete e;
        return rc;
    }
    *out = e;
    return lssm_engine_reset(e);
}

int lssm_engine_destroy(lssm_engine* e) {
    clear_error();
    if (!e) return LSSM_OK;
    (void)hipStreamSynchronize(e->ctx->stream);
    delete e;
    return LSSM_OK;
}

int lssm_engine_reset(lssm_engine* e) {
    if (int rc = check_engine(e)) return rc;
    hipError_t err = hipMemsetAsync(e->conv_state, 0,
                                    (size_t)e->cfg.n_layer * e->max_batch * e->xbc * e->K * e->es,
                                    e->ctx->stream);
    if (err == hipSuccess)
        err = hipMemsetAsync(e->ssd_state, 0,
                             (size_t)e->cfg.n_layer * e->max_batch * e->H * e->P * e->N * sizeof(float),
                             e->ctx->stream);
    return engine_finish(e, err, "engine_reset");
}

int lssm_engine_prefill(lssm_engine* e, const int32_t* ids, uint32_t batch, uint32_t L,
                        int32_t* next_ids) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(L >= 1, "forward_prefill: L must be >= 1");                       // mamba2_block.cpp:300
    LSSM_REQUIRE(L <= e->max_seq, "forward_prefill: L exceeds workspace max_seq_len"); // :301-303
    LSSM_REQUIRE(batch >= 1 && batch <= e->max_batch, "forward_prefill: batch out of range");
    LSSM_REQUIRE(ids && next_ids, "forward_prefill: null ids");
    LSSM_REQUIRE(!e->trace || e->trace_bytes(L == 1 ? batch : batch * L) <= e->trace_cap,
                 "engine_prefill: trace buffer too small");
    return engine_finish(e, e->prefill(ids, batch, L, next_ids), "engine_prefill");
}

int lssm_engine_decode(lssm_engine* e, const int32_t* ids, uint32_t batch, int32_t* next_ids) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(batch >= 1 && batch <= e->max_batch, "forward_step: batch out of range");
    LSSM_REQUIRE(ids && next_ids, "forward_step: null ids");
    LSSM_REQUIRE(!e->trace || e->trace_bytes(batch) <= e->trace_cap, "engine_decode: trace buffer too small");
    return engine_finish(e, e->decode(ids, batch, next_ids), "engine_decode");
}

int lssm_engine_set_trace(lssm_engine* e, void* buf, uint64_t bytes) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(!buf || bytes > 0, "engine_set_trace: empty buffer");
    e->trace = buf;
    e->trace_cap = buf ? (size_t)bytes : 0;
    return LSSM_OK;
}

int lssm_engine_set_id_log(lssm_engine* e, int32_t* buf, uint32_t cap_steps) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(!buf || cap_steps > 0, "engine_set_id_log: empty buffer");
    e->drop_graphs();                       // captured steps hold the old setting
    e->id_log = buf;
    e->id_log_cap = buf ? cap_steps : 0;
    return engine_finish(e, hipMemsetAsync(e->seq + 1, 0, sizeof(uint32_t), e->ctx->stream),
                         "engine_set_id_log");
}

int lssm_engine_decode_graph(lssm_engine* e, const int32_t* ids, uint32_t batch, int32_t* next_ids,
                             uint32_t steps) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(!e->trace, "engine_decode_graph: not with a trace buffer set (lssm_engine_set_trace)");
    LSSM_REQUIRE(batch >= 1 && batch <= e->max_batch, "forward_step: batch out of range");
    LSSM_REQUIRE(ids && next_ids, "forward_step: null ids");
    hipStream_t s = e->ctx->stream;
    if (e->g_ids != ids || e->g_next != next_ids || e->g_batch != batch) {
        e->drop_graphs();
        e->g_ids = ids;
        e->g_next = next_ids;
        e->g_batch = batch;
    }
    // graph k of n steps, captured on first use
    auto exec = [&](int k, uint32_t n) -> int {
        if (e->graph_exec[k]) return LSSM_OK;
        if (e->graph[k]) {                                     // left by a failed instantiation
            (void)hipGraphDestroy(e->graph[k]);
            e->graph[k] = nullptr;
        }
        hipError_t err = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (err != hipSuccess) return engine_finish(e, err, "engine_decode_graph: begin capture");
        hipError_t le = hipSuccess;
        for (uint32_t i = 0; i < n && le == hipSuccess; ++i) le = e->decode(ids, batch, next_ids);
        err = hipStreamEndCapture(s, &e->graph[k]);
        if (le != hipSuccess) return engine_finish(e, le, "engine_decode_graph: capture");
        if (err != hipSuccess) return engine_finish(e, err, "engine_decode_graph: end capture");
        err = hipGraphInstantiate(&e->graph_exec[k], e->graph[k], nullptr, nullptr, 0);
        if (err != hipSuccess) return engine_finish(e, err, "engine_decode_graph: instantiate");
        return LSSM_OK;
    };
    const uint32_t U = e->graph_unroll > 1 ? e->graph_unroll : 1;
    uint32_t left = steps;
    if (U > 1 && left >= U) {
        if (int rc = exec(1, U)) return rc;
        for (; left >= U; left -= U) {
            hipError_t err = hipGraphLaunch(e->graph_exec[1], s);
            if (err != hipSuccess) return engine_finish(e, err, "engine_decode_graph: launch");
        }
    }
    if (left > 0) {
        if (int rc = exec(0, 1)) return rc;
        for (; left > 0; --left) {
            hipError_t err = hipGraphLaunch(e->graph_exec[0], s);
            if (err != hipSuccess) return engine_finish(e, err, "engine_decode_graph: launch");
        }
    }
    return finish(e->ctx, "engine_decode_graph");
}

int lssm_engine_logits(lssm_engine* e, void** logits) {
    if (int rc = check_engine(e)) return rc;
    LSSM_REQUIRE(logits, "engine_logits: null out");
    *logits = e->logits;
    return LSSM_OK;
}

int lssm_engine_fused_layers(lssm_engine* e, uint32_t* ssd_fused, uint32_t* mixer_fused) {
    if (int rc = check_engine(e)) return rc;
    if (ssd_fused) *ssd_fused = e->fused_layers;
    if (mixer_fused) *mixer_fused = e->mixer_layers;
    return LSSM_OK;
}

int lssm_engine_state(lssm_engine* e, void** conv_state, void** ssd_state) {
    if (int rc = check_engine(e)) return rc;
    if (conv_state) *conv_state = e->conv_state;
    if (ssd_state) *ssd_state = e->ssd_state;
    return LSSM_OK;
}

}  // extern "C"

"""GPU parity of every op, through the C ABI, against the CPU oracle on the
same seeded inputs (BASELINE configs 1 and 2 included at their full shapes)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import MAXREL, act_host, assert_close, dev, empty, host, max_rel, ulp_diff16

pytestmark = pytest.mark.gpu

ACTS = [O.F16, O.BF16, O.F32]
QFMTS = [O.W_Q4_B32, O.W_Q4_G64, O.W_Q8_G32]
ALL_FMTS = [O.W_DENSE] + QFMTS


def _lib():
    import lite_ssm_amd as L
    return L


def _weights(rng, N, K, wfmt, act, std=0.02):
    wf = (rng.standard_normal((N, K)) * std).astype(np.float16).astype(np.float32)
    if wfmt == O.W_DENSE:
        return O.to_act(wf, act), None
    return O.quantize(wf, wfmt)


# --------------------------------------------------------------------------- dequant
@pytest.mark.parametrize("wfmt", QFMTS)
def test_dequant_bit_exact(ctx, rng, wfmt):
    N, K = 96, 512
    w, s = _weights(rng, N, K, wfmt, O.F16, std=1.0)
    out = torch.empty(N, K, dtype=torch.float32, device="cuda")
    ctx.dequant(dev(w), dev(s), out, N, K, wfmt)
    ref = O.dequant(w, s, N, K, wfmt)
    assert np.array_equal(host(out, np.float32).view(np.uint32), ref.view(np.uint32))


# --------------------------------------------------------------------------- GEMV / GEMM
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("wfmt", ALL_FMTS)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_vs_oracle(ctx, rng, act, wfmt, M):
    L = _lib()
    N, K = 200, 768
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    y = empty((M, N), act)
    ctx.linear(dev(x), dev(w), None if s is None else dev(s), y, M, N, K, wfmt, act)
    ref = O.linear(x, w, s, M, N, K, wfmt, act)
    got = act_host(y, act)
    bound = {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-5}[act]
    assert_close(got, ref, act, bound, "gemv")
    if act == O.F16:
        assert ulp_diff16(got, ref).max() <= 2


@pytest.mark.parametrize("act", [O.F16, O.BF16])
@pytest.mark.parametrize("wfmt", ALL_FMTS)
@pytest.mark.parametrize("M", [5, 300])
def test_gemm_vs_oracle(ctx, rng, act, wfmt, M):
    N, K = 300, 1536
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    y = empty((M, N), act)
    ctx.linear(dev(x), dev(w), None if s is None else dev(s), y, M, N, K, wfmt, act)
    # GEMM semantics: dequantized weight rounded to the activation dtype (linear.metal:538)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, round_dequant=1)
    bound = {O.F16: 2e-3, O.BF16: 1.6e-2}[act]
    assert_close(act_host(y, act), ref, act, bound, "gemm")


@pytest.mark.parametrize("act", [O.F16, O.BF16])
@pytest.mark.parametrize("wfmt", ALL_FMTS)
@pytest.mark.parametrize("M", [7, 16, 40, 64])
def test_gemm_decode_batch_vs_oracle(ctx, rng, act, wfmt, M):
    """Decode batches (5 <= M <= 64): the weight-streaming GEMM, N not a
    multiple of its 16-row tile."""
    N, K = 300, 1024
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    y = empty((M, N), act)
    ctx.linear(dev(x), dev(w), None if s is None else dev(s), y, M, N, K, wfmt, act)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, round_dequant=1)
    assert_close(act_host(y, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2}[act], "gemm")


@pytest.mark.parametrize("act", [O.F16, O.BF16])
def test_gemm_decode_batch_epilogues(ctx, rng, act):
    L = _lib()
    M, N, K, wfmt = 16, 256, 512, O.W_Q4_G64
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    res = O.to_act(rng.standard_normal((M, N)), act)
    yd = dev(res)
    ctx.linear(dev(x), dev(w), dev(s), yd, M, N, K, wfmt, act, epi=L.EPI_ADD, residual=yd)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_ADD, residual=res, round_dequant=1)
    assert_close(act_host(yd, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2}[act], "add")
    ys = empty((M, N), act)
    ctx.linear(dev(x), dev(w), dev(s), ys, M, N, K, wfmt, act, epi=L.EPI_SILU)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_SILU, round_dequant=1)
    assert_close(act_host(ys, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2}[act], "silu")


@pytest.mark.parametrize("wfmt", QFMTS)
def test_gemm_wide_tiles(ctx, rng, wfmt):
    """Enough 256 x 256 tiles for the wide GEMM (>= 3 per CU on 256 CUs), with
    partial last tiles in M and N and an odd number of K steps."""
    act, M, N, K = O.BF16, 2000, 24500, 192
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    y = empty((M, N), act)
    ctx.linear(dev(x), dev(w), dev(s), y, M, N, K, wfmt, act)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, round_dequant=1)
    assert_close(act_host(y, act), ref, act, 1.6e-2, "gemm")


@pytest.mark.parametrize("wfmt", [O.W_Q4_G64, O.W_Q4_B32, O.W_Q8_G32])
def test_gemm_wide_tiles_split_tail(ctx, rng, wfmt):
    """286 wide tiles on 256 CUs (a last round of 30): the columns of the full
    round go to the wide launch and the remaining 336 (two and a partial
    128-wide tile) to a narrow one, in place with the residual epilogue as the
    engine's out_proj runs it."""
    L = _lib()
    act, M, N, K = O.BF16, 26 * 256, 2640, 192
    print(f"case: split-tail GEMM {wfmt} M {M} N {N} K {K}", flush=True)
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    res = O.to_act(rng.standard_normal((M, N)), act)
    yd = dev(res)
    ctx.linear(dev(x), dev(w), dev(s), yd, M, N, K, wfmt, act, epi=L.EPI_ADD, residual=yd)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_ADD, residual=res, round_dequant=1)
    assert_close(act_host(yd, act), ref, act, 1.6e-2, "gemm split tail")


@pytest.mark.parametrize("wfmt", [O.W_Q4_G64, O.W_Q8_G32, O.W_DENSE])
@pytest.mark.parametrize("K", [64, 192])
def test_gemm_one_and_odd_k_steps(ctx, rng, wfmt, K):
    """Large-tile GEMM with 1 and 3 K steps of 64 (the pipeline's tail paths),
    M and N one past a tile edge."""
    act, M, N = O.BF16, 257, 129
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    y = empty((M, N), act)
    ctx.linear(dev(x), dev(w), None if s is None else dev(s), y, M, N, K, wfmt, act)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, round_dequant=1)
    assert_close(act_host(y, act), ref, act, 1.6e-2, "gemm")


@pytest.mark.parametrize("act", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("M", [2, 130])
def test_linear_epilogues(ctx, rng, act, M):
    L = _lib()
    N, K, wfmt = 256, 512, O.W_Q4_G64
    x = O.to_act(rng.standard_normal((M, K)), act)
    w, s = _weights(rng, N, K, wfmt, act)
    res = O.to_act(rng.standard_normal((M, N)), act)
    yd = dev(res)                                   # in-place residual: y == residual
    ctx.linear(dev(x), dev(w), dev(s), yd, M, N, K, wfmt, act, epi=L.EPI_ADD, residual=yd)
    rd = 1 if M > 4 else 0
    ref = O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_ADD, residual=res, round_dequant=rd)
    assert_close(act_host(yd, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-5}[act], "add")
    ys = empty((M, N), act)
    ctx.linear(dev(x), dev(w), dev(s), ys, M, N, K, wfmt, act, epi=L.EPI_SILU)
    ref = O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_SILU, round_dequant=rd)
    assert_close(act_host(ys, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-5}[act], "silu")


@pytest.mark.parametrize("which", ["in_proj", "out_proj"])
def test_config2_q8g32_130m_shapes_gemv_and_gemm(ctx, rng, which):
    """130M in_proj [3352 x 768] / out_proj [768 x 1536],
    int8 group-32 fp16 scales, N(0, 0.02) weights, fp16 activations; M = 1 and 2048."""
    N, K = (3352, 768) if which == "in_proj" else (768, 1536)
    w, s = _weights(rng, N, K, O.W_Q8_G32, O.F16)
    wd, sd = dev(w), dev(s)
    for M in (1, 2048):
        x = O.to_act(rng.standard_normal((M, K)), O.F16)
        y = empty((M, N), O.F16)
        ctx.linear(dev(x), wd, sd, y, M, N, K, O.W_Q8_G32, O.F16)
        ref = O.linear(x, w, s, M, N, K, O.W_Q8_G32, O.F16, round_dequant=int(M > 4))
        assert_close(act_host(y, O.F16), ref, O.F16, 2e-3, f"config2 {which} M={M}")


def test_reference_named_linear_entries(ctx, rng):
    L = _lib()
    lib = L.lib
    N, K = 100, 256
    x1 = O.to_act(rng.standard_normal((1, K)), O.F16)
    x8 = O.to_act(rng.standard_normal((8, K)), O.F16)
    w4, s4 = _weights(rng, N, K, O.W_Q4_B32, O.F16)
    wh, _ = _weights(rng, N, K, O.W_DENSE, O.F16)
    y1, y8 = empty((1, N), O.F16), empty((8, N), O.F16)
    L.check(lib.lssm_linear_int4_gemv(ctx.h, dev(x1).data_ptr(), dev(w4).data_ptr(), dev(s4).data_ptr(),
                                      y1.data_ptr(), L.LinearDims(1, N, K)))
    assert_close(act_host(y1, O.F16), O.linear(x1, w4, s4, 1, N, K, O.W_Q4_B32, O.F16), O.F16, 2e-3)
    L.check(lib.lssm_linear_int4_gemm(ctx.h, dev(x8).data_ptr(), dev(w4).data_ptr(), dev(s4).data_ptr(),
                                      y8.data_ptr(), L.LinearDims(8, N, K)))
    assert_close(act_host(y8, O.F16), O.linear(x8, w4, s4, 8, N, K, O.W_Q4_B32, O.F16, round_dequant=1),
                 O.F16, 2e-3)
    for fn, epi in ((lib.lssm_linear_f16_gemv, O.EPI_NONE), (lib.lssm_linear_silu_f16_gemv, O.EPI_SILU)):
        L.check(fn(ctx.h, dev(x1).data_ptr(), dev(wh).data_ptr(), y1.data_ptr(), L.LinearDims(1, N, K)))
        assert_close(act_host(y1, O.F16), O.linear(x1, wh, None, 1, N, K, O.W_DENSE, O.F16, epi=epi), O.F16, 2e-3)
    for fn, epi in ((lib.lssm_linear_f16_gemm, O.EPI_NONE), (lib.lssm_linear_silu_f16_gemm, O.EPI_SILU)):
        L.check(fn(ctx.h, dev(x8).data_ptr(), dev(wh).data_ptr(), y8.data_ptr(), L.LinearDims(8, N, K)))
        assert_close(act_host(y8, O.F16), O.linear(x8, wh, None, 8, N, K, O.W_DENSE, O.F16, epi=epi), O.F16, 2e-3)
    # rmsnorm_linear_f16_gemv (linear.metal:148-204): normed rounded to half, then GEMV
    wn = O.to_act(1 + 0.1 * rng.standard_normal(K), O.F16)
    L.check(lib.lssm_rmsnorm_linear_f16_gemv(ctx.h, dev(x1).data_ptr(), dev(wn).data_ptr(),
                                             dev(wh).data_ptr(), y1.data_ptr(), L.RMSLinearDims(N, K, 1e-5)))
    ref = O.linear(O.rmsnorm(x1, wn, 1e-5, O.F16), wh, None, 1, N, K, O.W_DENSE, O.F16)
    assert_close(act_host(y1, O.F16), ref, O.F16, 2e-3)
    # preconditions keep the reference's messages (ops.mm:207-212, 323-324)
    rc = lib.lssm_linear_int4_gemv(ctx.h, dev(x8).data_ptr(), dev(w4).data_ptr(), dev(s4).data_ptr(),
                                   y8.data_ptr(), L.LinearDims(8, N, K))
    assert rc == 1 and b"M must be 1" in lib.lssm_last_error()
    rc = lib.lssm_linear_int4_gemv(ctx.h, dev(x1).data_ptr(), dev(w4).data_ptr(), dev(s4).data_ptr(),
                                   y1.data_ptr(), L.LinearDims(1, N, 250))
    assert rc == 1 and b"multiple of 32" in lib.lssm_last_error()
    rc = lib.lssm_rmsnorm_f16(ctx.h, None, None, None, L.RMSNormDims(1, 6, 1e-5))
    assert rc == 1 and b"multiple of 4" in lib.lssm_last_error()


# --------------------------------------------------------------------------- norms / activations
# dims: partial 512-element chunks (1536, 40), the 2.7B / 8B widths, and one
# past the wave-per-row kernels' limit (block-per-row kernels)
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("dim", [1536, 40, 5120, 8192, 8200])
def test_rmsnorm_and_gated(ctx, rng, act, dim):
    L = _lib()
    rows = 7
    x = O.to_act(rng.standard_normal((rows, dim)) * 2, act)
    z = O.to_act(rng.standard_normal((rows, dim)), act)
    w = O.to_act(1 + 0.1 * rng.standard_normal(dim), act)
    y = empty((rows, dim), act)
    ctx.rmsnorm(dev(x), dev(w), y, rows, dim, 1e-5, act)
    ref = O.rmsnorm(x, w, 1e-5, act)
    assert_close(act_host(y, act), ref, act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act], "rmsnorm")
    L.check(L.lib.lssm_gated_rmsnorm(ctx.h, dev(z).data_ptr(), dev(x).data_ptr(), dev(w).data_ptr(),
                                     y.data_ptr(), rows, dim, 1e-5, act))
    ref = O.gated_rmsnorm(z, x, w, 1e-5, act)
    assert_close(act_host(y, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-6}[act], "gated")


@pytest.mark.parametrize("act", ACTS)
def test_elementwise(ctx, rng, act):
    L = _lib()
    lib = L.lib
    n = 5000
    a = O.to_act(rng.standard_normal(n) * 3, act)
    b = O.to_act(rng.standard_normal(n), act)
    y = empty((n,), act)
    L.check(lib.lssm_silu(ctx.h, dev(a).data_ptr(), y.data_ptr(), n, act))
    assert_close(act_host(y, act), O.silu(a, act), act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act])
    L.check(lib.lssm_silu_gated(ctx.h, dev(a).data_ptr(), dev(b).data_ptr(), y.data_ptr(), n, act))
    assert_close(act_host(y, act), O.silu_gated(a, b, act), act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act])
    yd = dev(a)
    L.check(lib.lssm_add_inplace(ctx.h, yd.data_ptr(), dev(b).data_ptr(), n, act))
    assert np.array_equal(act_host(yd, act), O.add_inplace(a.copy(), b, act))
    rows, d_inner, N, G = 9, 256, 64, 2
    xbc = O.to_act(rng.standard_normal((rows, d_inner + 2 * G * N)) * 3, act)
    xo, Bo, Co = empty((rows, d_inner), act), empty((rows, G * N), act), empty((rows, G * N), act)
    L.check(lib.lssm_split_silu_xbc(ctx.h, dev(xbc).data_ptr(), xo.data_ptr(), Bo.data_ptr(),
                                    Co.data_ptr(), rows, d_inner, N, G, act))
    for g_, r_ in zip((xo, Bo, Co), O.split_silu_xbc(xbc, rows, d_inner, N, G, act)):
        assert_close(act_host(g_, act), r_, act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act], "split")


# --------------------------------------------------------------------------- conv
@pytest.mark.parametrize("act", ACTS)
def test_conv1d_family(ctx, rng, act):
    L = _lib()
    lib = L.lib
    B, Lq, D, K = 2, 37, 1792, 4
    x = O.to_act(rng.standard_normal((B, Lq, D)), act)
    w = O.to_act(rng.standard_normal((D, K)) * 0.5, act)
    bb = O.to_act(rng.standard_normal(D) * 0.1, act)
    y = empty((B, Lq, D), act)
    L.check(lib.lssm_conv1d(ctx.h, dev(x).data_ptr(), dev(w).data_ptr(), dev(bb).data_ptr(), y.data_ptr(),
                            B, Lq, D, K, act))
    ref = O.conv1d(x, w, bb, B, Lq, D, K, act)
    assert_close(act_host(y, act), ref, act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act], "conv1d")
    st = empty((B, D, K), act)
    L.check(lib.lssm_conv1d_seed(ctx.h, dev(x).data_ptr(), st.data_ptr(), B, Lq, D, K, act))
    seed = O.conv1d_seed(x, B, Lq, D, K, act)
    assert np.array_equal(act_host(st, act), seed)
    xn = O.to_act(rng.standard_normal((B, D)), act)
    yo = empty((B, D), act)
    L.check(lib.lssm_conv1d_update(ctx.h, dev(xn).data_ptr(), st.data_ptr(), dev(w).data_ptr(),
                                   dev(bb).data_ptr(), yo.data_ptr(), B, D, K, act))
    seed2 = seed.copy()
    yref = O.conv1d_update(xn, seed2, w, bb, B, D, K, act)
    assert np.array_equal(act_host(st, act), seed2)
    assert_close(act_host(yo, act), yref, act, {O.F16: 1e-3, O.BF16: 8e-3, O.F32: 1e-6}[act], "update")


def test_reference_conv_entries_f16(ctx, rng):
    L = _lib()
    lib = L.lib
    Lq, D, K = 12, 64, 4
    x = O.to_act(rng.standard_normal((1, Lq, D)), O.F16)
    w = O.to_act(rng.standard_normal((D, K)) * 0.5, O.F16)
    bb = O.to_act(rng.standard_normal(D) * 0.1, O.F16)
    y = empty((1, Lq, D), O.F16)
    L.check(lib.lssm_causal_conv1d_f16(ctx.h, dev(x).data_ptr(), dev(w).data_ptr(), dev(bb).data_ptr(),
                                       y.data_ptr(), L.Conv1dDims(1, Lq, D, K)))
    assert_close(act_host(y, O.F16), O.conv1d(x, w, bb, 1, Lq, D, K, O.F16), O.F16, 1e-3)
    st = empty((1, D, K), O.F16)
    L.check(lib.lssm_seed_conv_state_f16(ctx.h, dev(x).data_ptr(), st.data_ptr(), Lq, D, K))
    assert np.array_equal(act_host(st, O.F16), O.conv1d_seed(x, 1, Lq, D, K, O.F16))


# --------------------------------------------------------------------------- SSD
def _ssd_inputs(rng, batch, L, H, P, N, G, act):
    X = O.to_act(rng.standard_normal((batch, L, H, P)), act)
    B = O.to_act(rng.standard_normal((batch, L, G, N)) / np.sqrt(N), act)
    Cc = O.to_act(rng.standard_normal((batch, L, G, N)) / np.sqrt(N), act)
    dt = O.to_act(rng.normal(-2.0, 0.5, (batch, L, H)), act)        # softplus(N(-2, .5))
    dtb = O.to_act(np.zeros(H), act)
    A_log = O.to_act(rng.uniform(0, np.log(16), H), act)            # A = -exp(U(log 1, log 16))
    D = O.to_act(rng.standard_normal(H), act)
    return X, B, Cc, dt, dtb, A_log, D


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("G,H,batch", [(1, 24, 1), (8, 32, 3)])
def test_ssd_step_vs_oracle(ctx, rng, act, G, H, batch):
    L = _lib()
    P, N = 64, 128
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, 1, H, P, N, G, act)
    st = (rng.standard_normal((batch, H, P, N)) * 0.5).astype(np.float32)
    xs, Bs, Cs, dts = (np.ascontiguousarray(a[:, 0]) for a in (X, B, Cc, dt))
    sd = dev(st)
    y = empty((batch, H, P), act)
    ctx.ssd_step(dev(xs), dev(Bs), dev(Cs), dev(dts), dev(dtb), dev(A_log), dev(D), sd, y, batch,
                 L.SSDStepDims(H, P, N, G, 1e-6, 1e6, 1), act)
    s2 = st.copy()
    yr = O.ssd_step(xs, Bs, Cs, dts, dtb, A_log, D, s2, batch, H, P, N, G, act)
    assert max_rel(host(sd, np.float32), s2) < 1e-5
    assert_close(act_host(y, act), yr, act, {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-5}[act], "ssd_step")


def test_ssd_chunked_config1_fp32(ctx, rng):
    """fp32 SSD, 130M layer shape: batch 1, L 512, 24 heads x 64,
    d_state 128, 1 group, chunk 64.  max-rel 1e-3 on y and the final state."""
    L = _lib()
    act, batch, Lq, H, P, N, G = O.F32, 1, 512, 24, 64, 128, 1
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, Lq, H, P, N, G, act)
    sd = torch.zeros(batch, H, P, N, dtype=torch.float32, device="cuda")
    Y = empty((batch, Lq, H, P), act)
    ctx.ssd_chunked(dev(X), dev(B), dev(Cc), dev(dt), dev(dtb), dev(A_log), dev(D), Y, sd, batch,
                    L.SSDDims(Lq, H, P, N, G, 64, 1e-6, 1e6, 1), act)
    s2 = np.zeros((batch, H, P, N), np.float32)
    Yr = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s2, batch, Lq, H, P, N, G, 64, act)
    assert max_rel(host(Y, np.float32), Yr) < 1e-3
    assert max_rel(host(sd, np.float32), s2) < 1e-3


@pytest.mark.parametrize("batch,Lq,H,G,P", [(1, 512, 24, 1, 64), (2, 200, 8, 2, 128), (1, 40, 4, 1, 64),
                                            (3, 64, 16, 8, 64), (1, 1950, 24, 1, 64)])
def test_ssd_chunked_fp32_mfma_vs_oracle(ctx, rng, batch, Lq, H, G, P):
    """The fp32 chunked scan on v_mfma_f32_16x16x4_f32: a nonzero initial
    state, ragged last chunks, several groups and P slices, max-rel 1e-3 on y
    and the final state."""
    L = _lib()
    act, N = O.F32, 128
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, Lq, H, P, N, G, act)
    s0 = (rng.standard_normal((batch, H, P, N)) * 0.3).astype(np.float32)
    sd = dev(s0)
    Y = empty((batch, Lq, H, P), act)
    ctx.ssd_chunked(dev(X), dev(B), dev(Cc), dev(dt), dev(dtb), dev(A_log), dev(D), Y, sd, batch,
                    L.SSDDims(Lq, H, P, N, G, 64, 1e-6, 1e6, 1), act)
    s2 = s0.copy()
    Yr = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s2, batch, Lq, H, P, N, G, 64, act)
    assert max_rel(host(Y, np.float32), Yr) < 1e-3
    assert max_rel(host(sd, np.float32), s2) < 1e-3


# Grids of fewer blocks than CUs run segmented (the sequence's chunks split
# into segments that run in parallel): (1, 512, 24) one chunk per segment,
# (1, 1950, 24) two per segment and a last segment of one partial chunk.
# (4, 130, 64, 1) and P = 128 give at least one block per CU and run
# unsegmented; P = 32 takes the two-wave blocks.
@pytest.mark.parametrize("act", [O.F16, O.BF16])
@pytest.mark.parametrize("batch,Lq,H,G,P", [(1, 512, 24, 1, 64), (2, 200, 8, 2, 64), (1, 40, 4, 1, 64),
                                            (3, 64, 16, 8, 64), (4, 130, 64, 1, 64), (2, 100, 6, 2, 32),
                                            (2, 150, 128, 1, 128), (1, 1950, 24, 1, 64)])
def test_ssd_chunked_mfma_vs_oracle(ctx, rng, act, batch, Lq, H, G, P):
    L = _lib()
    N = 128
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, Lq, H, P, N, G, act)
    st = (rng.standard_normal((batch, H, P, N)) * 0.2).astype(np.float32)
    ck = min(64, Lq)
    sd = dev(st)
    Y = empty((batch, Lq, H, P), act)
    ctx.ssd_chunked(dev(X), dev(B), dev(Cc), dev(dt), dev(dtb), dev(A_log), dev(D), Y, sd, batch,
                    L.SSDDims(Lq, H, P, N, G, ck, 1e-6, 1e6, 1), act)
    s2 = st.copy()
    Yr = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s2, batch, Lq, H, P, N, G, ck, act)
    assert_close(act_host(Y, act), Yr, act, 2e-2, "ssd_chunked y")
    assert max_rel(host(sd, np.float32), s2) < 2e-2


def test_ssd_chunked_graph_survives_gram_growth(ctx, rng):
    """A graph captured around lssm_ssd_chunked records the context's Gram
    workspace; a later, larger uncaptured call grows that workspace.  The old
    buffer must stay allocated (retired until lssm_ctx_destroy), so every
    replay of the graph still gives the eager bits."""
    L = _lib()
    act, P, N, G = O.BF16, 64, 128, 1
    st = torch.cuda.Stream()
    c2 = L.Ctx(st.cuda_stream)
    try:
        def inputs(batch, Lq, H):
            X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, Lq, H, P, N, G, act)
            return [dev(a) for a in (X, B, Cc, dt, dtb, A_log, D)]

        small = (1, 192, 8)
        a = inputs(*small)
        s0 = torch.from_numpy((rng.standard_normal((1, 8, P, N)) * 0.2).astype(np.float32)).cuda()
        sd = s0.clone()
        Y = empty((1, 192, 8, P), act)
        dims = L.SSDDims(192, 8, P, N, G, 64, 1e-6, 1e6, 1)
        with torch.cuda.stream(st):
            c2.ssd_chunked(*a, Y, sd, 1, dims, act)          # allocates the workspaces
        st.synchronize()
        Ye, se = Y.clone(), sd.clone()
        g = torch.cuda.CUDAGraph()
        sd.copy_(s0)
        Y.zero_()
        torch.cuda.synchronize()
        c2.begin_batch()
        with torch.cuda.stream(st):
            g.capture_begin()
            c2.ssd_chunked(*a, Y, sd, 1, dims, act)
            g.capture_end()
        c2.commit_and_wait()
        # a larger call grows the Gram workspace
        big = inputs(4, 1024, 8)
        sb = torch.zeros(4, 8, P, N, dtype=torch.float32, device="cuda")
        Yb = empty((4, 1024, 8, P), act)
        with torch.cuda.stream(st):
            c2.ssd_chunked(*big, Yb, sb, 4, L.SSDDims(1024, 8, P, N, G, 64, 1e-6, 1e6, 1), act)
        st.synchronize()
        for _ in range(3):
            sd.copy_(s0)
            Y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(Y, Ye) and torch.equal(sd, se)
    finally:
        torch.cuda.synchronize()
        c2.close()


def test_ssd_chunked_reference_entry_and_checks(ctx, rng):
    L = _lib()
    lib = L.lib
    Lq, H, P, N = 100, 4, 64, 128
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, 1, Lq, H, P, N, 1, O.F16)
    sd = torch.zeros(1, H, P, N, dtype=torch.float32, device="cuda")
    Y = empty((1, Lq, H, P), O.F16)
    args = [dev(a).data_ptr() for a in (X, B, Cc, dt, dtb, A_log, D)]
    L.check(lib.lssm_ssd_chunked_f16(ctx.h, *args, Y.data_ptr(), sd.data_ptr(),
                                     L.SSDDims(Lq, H, P, N, 1, 64, 1e-6, 1e6, 1)))
    s2 = np.zeros((1, H, P, N), np.float32)
    Yr = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s2, 1, Lq, H, P, N, 1, 64, O.F16)
    assert_close(act_host(Y, O.F16), Yr, O.F16, 2e-2)
    rc = lib.lssm_ssd_chunked_f16(ctx.h, *args, Y.data_ptr(), sd.data_ptr(),
                                  L.SSDDims(Lq, H, P, N, 1, 128, 1e-6, 1e6, 1))
    assert rc == 1 and b"chunk_size" in lib.lssm_last_error()


# --------------------------------------------------------------------------- fused in_proj, embed, argmax
def test_inproj_fused_vs_oracle(ctx, rng):
    L = _lib()
    Lq, d_model, d_inner, N, G, H, K = 12, 768, 1536, 128, 1, 24, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    normed = O.to_act(rng.standard_normal((Lq, d_model)), O.F16)
    W = O.to_act(rng.standard_normal((proj, d_model)) * 0.02, O.F16)
    Wc = O.to_act(rng.standard_normal((xbc, K)) * 0.5, O.F16)
    cb = O.to_act(rng.standard_normal(xbc) * 0.1, O.F16)
    outs = [empty(s, O.F16) for s in ((Lq, d_inner), (Lq, d_inner), (Lq, G * N), (Lq, G * N), (Lq, H), (Lq, xbc))]
    L.check(L.lib.lssm_inproj_fused_f16(ctx.h, dev(normed).data_ptr(), dev(W).data_ptr(),
                                        dev(Wc).data_ptr(), dev(cb).data_ptr(),
                                        *[o.data_ptr() for o in outs],
                                        L.FusedInProjDims(Lq, d_model, d_inner, N, G, H, K, proj)))
    refs = O.inproj_fused(normed, W, Wc, cb, Lq, d_model, d_inner, N, G, H, K)
    for o, r in zip(outs, refs):
        assert_close(act_host(o, O.F16), r, O.F16, 2e-3, "inproj_fused")


INPROJ_CASES = [
    # batch 1..4: VALU GEMV (gemv1 / gemv_lds)
    (O.BF16, O.W_Q4_G64, 1, 2560), (O.F16, O.W_Q8_G32, 3, 2560), (O.F16, O.W_Q4_B32, 4, 2560),
    (O.F32, O.W_DENSE, 2, 2560),
    # 2..64: MFMA GEMV (2.7B in_proj: 3 tiles per block); 17 and 33 end
    # mid-tile, 64 fills four MFMA row tiles in four passes of 16 rows
    (O.BF16, O.W_Q4_G64, 2, 2560), (O.BF16, O.W_Q4_G64, 16, 2560), (O.BF16, O.W_Q4_G64, 17, 2560),
    (O.BF16, O.W_Q4_G64, 64, 2560), (O.F16, O.W_Q4_G64, 8, 2560), (O.BF16, O.W_Q4_B32, 5, 2560),
    (O.F16, O.W_Q4_B32, 33, 2560), (O.F16, O.W_Q8_G32, 16, 2560), (O.F16, O.W_DENSE, 7, 2560),
    # K = 5120: 16 rows take two passes of 8 (staging does not fit 16)
    (O.BF16, O.W_Q4_G64, 16, 5120), (O.F16, O.W_Q8_G32, 12, 5120),
    # 8B in_proj shape at batch 32 (4 tiles per block, 2 passes)
    (O.BF16, O.W_Q4_G64, 32, 4096),
]


@pytest.mark.parametrize("act,wfmt,batch,d_model", INPROJ_CASES,
                         ids=[f"{['f16', 'bf16', 'f32'][a]}-w{w}-b{b}-k{k}" for a, w, b, k in INPROJ_CASES])
def test_inproj_decode_vs_unfused_chain(ctx, rng, act, wfmt, batch, d_model):
    """The engine's fused decode in_proj == rmsnorm -> gemv -> conv update -> split
    SiLU, with the GEMV rule (exact dequantization) at every batch."""
    L = _lib()
    d_inner, N, G, H, K = {2560: (5120, 128, 1, 80, 4), 5120: (1024, 64, 2, 16, 4),
                           4096: (8192, 128, 8, 128, 4)}[d_model]
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    hid = O.to_act(rng.standard_normal((batch, d_model)) * 0.5, act)
    nw = O.to_act(1 + 0.1 * rng.standard_normal(d_model), act)
    w, s = _weights(rng, proj, d_model, wfmt, act)
    cw = O.to_act(rng.standard_normal((xbc, K)) * 0.3, act)
    cb = O.to_act(rng.standard_normal(xbc) * 0.1, act)
    cs = O.to_act(rng.standard_normal((batch, xbc, K)), act)
    csd = dev(cs)
    z, xa, dt = empty((batch, d_inner), act), empty((batch, xbc), act), empty((batch, H), act)
    L.check(L.lib.lssm_inproj_decode(ctx.h, dev(hid).data_ptr(), dev(nw).data_ptr(), dev(w).data_ptr(),
                                     None if s is None else dev(s).data_ptr(), csd.data_ptr(),
                                     dev(cw).data_ptr(), dev(cb).data_ptr(), z.data_ptr(), xa.data_ptr(),
                                     dt.data_ptr(), batch, d_model, d_inner, N, G, H, K, 1e-5, wfmt, act))
    normed = O.rmsnorm(hid, nw, 1e-5, act)
    pr = O.linear(normed, w, s, batch, proj, d_model, wfmt, act)
    bound = {O.F16: 2e-3, O.BF16: 1.6e-2, O.F32: 1e-5}[act]
    assert_close(act_host(z, act), np.ascontiguousarray(pr[:, :d_inner]), act, bound, "z")
    assert_close(act_host(dt, act), np.ascontiguousarray(pr[:, d_inner + xbc:]), act, bound, "dt")
    cs2 = cs.copy()
    conv = O.conv1d_update(np.ascontiguousarray(pr[:, d_inner:d_inner + xbc]), cs2, cw, cb, batch, xbc, K, act)
    ref = O.silu(conv, act)
    assert_close(act_host(xa, act), ref, act, bound * 4, "xbc_act")
    assert_close(act_host(csd, act), cs2, act, bound, "conv_state")


INPROJ_SSD_CASES = [
    # d_model, d_inner, N, G, H, act, wfmt: 2.7B (int4-g64 bf16), 130M (int8-g32 fp16),
    # a 2-group int4 fp16 shape
    (2560, 5120, 128, 1, 80, O.BF16, O.W_Q4_G64), (768, 1536, 128, 1, 24, O.F16, O.W_Q8_G32),
    (2048, 2048, 128, 2, 32, O.F16, O.W_Q4_G64),
]


@pytest.mark.parametrize("d_model,d_inner,N,G,H,act,wfmt", INPROJ_SSD_CASES,
                         ids=[f"dm{c[0]}-h{c[4]}-g{c[3]}" for c in INPROJ_SSD_CASES])
def test_inproj_ssd_decode_vs_unfused_chain(ctx, rng, d_model, d_inner, N, G, H, act, wfmt):
    """Batch-1 in_proj + conv + SSD step + SiLU(z) gate in one launch (rows passed
    between workgroups as tagged words): conv and SSD state bit-identical to
    lssm_inproj_decode -> lssm_ssd_step, y within rounding of r(silu(z) r(y));
    two calls in a row on the same word buffer (tags 1, 2)."""
    import lite_ssm_amd as L
    P, K = d_inner // H, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    nw = dev(O.to_act(1 + 0.1 * rng.standard_normal(d_model), act))
    w, s = _weights(rng, proj, d_model, wfmt, act)
    w, s = dev(w), None if s is None else dev(s)
    cw = dev(O.to_act(rng.standard_normal((xbc, K)) * 0.3, act))
    cb = dev(O.to_act(rng.standard_normal(xbc) * 0.1, act))
    dtb = dev(O.to_act(rng.standard_normal(H) * 0.5, act))
    alog = dev(O.to_act(rng.uniform(0, np.log(16), H), act))
    Dh = dev(O.to_act(rng.standard_normal(H), act))
    cs0 = O.to_act(rng.standard_normal((1, xbc, K)), act)
    st0 = (rng.standard_normal((H, P, N)) * 0.1).astype(np.float32)
    cs_f, cs_u = dev(cs0), dev(cs0)
    st_f, st_u = dev(st0), dev(st0)
    xfer = torch.zeros(proj, dtype=torch.int64, device="cuda")
    z, xa, dt = empty((1, d_inner), act), empty((1, xbc), act), empty((1, H), act)
    y_f, y_u = empty((1, d_inner), act), empty((1, d_inner), act)
    dims = L.SSDStepDims(H, P, N, G, 1e-6, 1e6, 1)
    for tag in (1, 2):
        hid = dev(O.to_act(rng.standard_normal((1, d_model)) * 0.5, act))
        L.check(L.lib.lssm_inproj_ssd_decode(
            ctx.h, hid.data_ptr(), nw.data_ptr(), w.data_ptr(), None if s is None else s.data_ptr(),
            cs_f.data_ptr(), cw.data_ptr(), cb.data_ptr(), dtb.data_ptr(), alog.data_ptr(), Dh.data_ptr(),
            st_f.data_ptr(), y_f.data_ptr(), xfer.data_ptr(), tag, d_model, d_inner, N, G, H, P, K,
            1e-5, wfmt, act))
        L.check(L.lib.lssm_inproj_decode(
            ctx.h, hid.data_ptr(), nw.data_ptr(), w.data_ptr(), None if s is None else s.data_ptr(),
            cs_u.data_ptr(), cw.data_ptr(), cb.data_ptr(), z.data_ptr(), xa.data_ptr(), dt.data_ptr(),
            1, d_model, d_inner, N, G, H, K, 1e-5, wfmt, act))
        es = xa.element_size()
        L.check(L.lib.lssm_ssd_step(ctx.h, xa.data_ptr(), xa.data_ptr() + d_inner * es,
                                    xa.data_ptr() + (d_inner + G * N) * es, dt.data_ptr(), dtb.data_ptr(),
                                    alog.data_ptr(), Dh.data_ptr(), st_u.data_ptr(), y_u.data_ptr(), 1, dims, act))
        torch.cuda.synchronize()
        assert torch.equal(cs_f, cs_u), f"conv state, tag {tag}"
        assert torch.equal(st_f, st_u), f"ssd state, tag {tag}"
        zf = O.from_act(act_host(z, act), act).astype(np.float64)
        yu = O.from_act(act_host(y_u, act), act).astype(np.float64)
        ref = O.to_act(zf / (1 + np.exp(-zf)) * yu, act)
        assert_close(act_host(y_f, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2}[act], f"y, tag {tag}")


MIXER_CASES = [c for c in INPROJ_SSD_CASES if (c[0], c[1]) in ((2560, 5120), (768, 1536), (2048, 2048))]


@pytest.mark.parametrize("d_model,d_inner,N,G,H,act,wfmt", MIXER_CASES,
                         ids=[f"dm{c[0]}-h{c[4]}-g{c[3]}" for c in MIXER_CASES])
def test_mixer_decode_vs_two_launches(ctx, rng, d_model, d_inner, N, G, H, act, wfmt):
    """A layer's whole batch-1 mixer in one launch == lssm_inproj_ssd_decode ->
    lssm_norm_linear_decode(EPI_ADD), bit for bit (hidden, conv and SSD state),
    on three calls in a row (tags 1, 2, 3)."""
    import lite_ssm_amd as L
    P, K = d_inner // H, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    nw = dev(O.to_act(1 + 0.1 * rng.standard_normal(d_model), act))
    mnw = dev(O.to_act(1 + 0.1 * rng.standard_normal(d_inner), act))
    wi, si = _weights(rng, proj, d_model, wfmt, act)
    wo, so = _weights(rng, d_model, d_inner, wfmt, act)
    wi, si, wo, so = dev(wi), dev(si), dev(wo), dev(so)
    cw = dev(O.to_act(rng.standard_normal((xbc, K)) * 0.3, act))
    cb = dev(O.to_act(rng.standard_normal(xbc) * 0.1, act))
    dtb = dev(O.to_act(rng.standard_normal(H) * 0.5, act))
    alog = dev(O.to_act(rng.uniform(0, np.log(16), H), act))
    Dh = dev(O.to_act(rng.standard_normal(H), act))
    cs0 = O.to_act(rng.standard_normal((1, xbc, K)), act)
    st0 = (rng.standard_normal((H, P, N)) * 0.1).astype(np.float32)
    h0 = O.to_act(rng.standard_normal((1, d_model)) * 0.5, act)
    cs_f, cs_u, st_f, st_u, h_f, h_u = dev(cs0), dev(cs0), dev(st0), dev(st0), dev(h0), dev(h0)
    xf = torch.zeros(proj + d_inner, dtype=torch.int64, device="cuda")
    xu = torch.zeros(proj, dtype=torch.int64, device="cuda")
    yg = empty((1, d_inner), act)
    for tag in (1, 2, 3):
        L.check(L.lib.lssm_mixer_decode(
            ctx.h, h_f.data_ptr(), nw.data_ptr(), wi.data_ptr(), si.data_ptr(), cs_f.data_ptr(), cw.data_ptr(),
            cb.data_ptr(), dtb.data_ptr(), alog.data_ptr(), Dh.data_ptr(), st_f.data_ptr(), mnw.data_ptr(),
            wo.data_ptr(), so.data_ptr(), xf.data_ptr(), tag, d_model, d_inner, N, G, H, P, K, 1e-5, wfmt, act))
        L.check(L.lib.lssm_inproj_ssd_decode(
            ctx.h, h_u.data_ptr(), nw.data_ptr(), wi.data_ptr(), si.data_ptr(), cs_u.data_ptr(), cw.data_ptr(),
            cb.data_ptr(), dtb.data_ptr(), alog.data_ptr(), Dh.data_ptr(), st_u.data_ptr(), yg.data_ptr(),
            xu.data_ptr(), tag, d_model, d_inner, N, G, H, P, K, 1e-5, wfmt, act))
        L.check(L.lib.lssm_norm_linear_decode(ctx.h, yg.data_ptr(), mnw.data_ptr(), 1e-5, wo.data_ptr(),
                                              so.data_ptr(), h_u.data_ptr(), h_u.data_ptr(), 1, d_model,
                                              d_inner, wfmt, act, O.EPI_ADD))
        torch.cuda.synchronize()
        assert torch.equal(cs_f, cs_u), f"conv state, tag {tag}"
        assert torch.equal(st_f, st_u), f"ssd state, tag {tag}"
        assert torch.equal(h_f, h_u), f"hidden, tag {tag}: max |d| " \
            f"{(O.from_act(act_host(h_f, act), act) - O.from_act(act_host(h_u, act), act)).max()}"


def test_inproj_ssd_decode_rejects_unsupported(ctx):
    """Shapes the fused launch does not take are refused with nothing run."""
    import lite_ssm_amd as L
    dummy = torch.zeros(1 << 16, dtype=torch.int64, device="cuda")
    p = dummy.data_ptr()
    # d_state 64 (the fused tail is built for 128)
    rc = L.lib.lssm_inproj_ssd_decode(ctx.h, p, p, p, p, p, p, p, p, p, p, p, p, p, 1,
                                      2560, 5120, 64, 1, 80, 64, 4, 1e-5, O.W_Q4_G64, O.BF16)
    assert rc == 1 and b"not supported" in L.lib.lssm_last_error()


NORM_LINEAR_CASES = [
    # rows, N, K, act, wfmt, epi: 2.7B out_proj (K 5120: 16 rows in two passes),
    # 8B out_proj (K 8192), odd N, the VALU GEMV rows (1, 3) and the fallback
    # formats (bf16 dense / int8 take gemv1 launches of <= 4 rows)
    (16, 2560, 5120, O.BF16, O.W_Q4_G64, O.EPI_ADD), (4, 2560, 5120, O.BF16, O.W_Q4_G64, O.EPI_ADD),
    (40, 2560, 5120, O.BF16, O.W_Q4_G64, O.EPI_ADD), (64, 1000, 2560, O.F16, O.W_Q4_B32, O.EPI_NONE),
    (9, 4096, 8192, O.BF16, O.W_Q4_G64, O.EPI_ADD), (32, 4096, 8192, O.BF16, O.W_Q4_G64, O.EPI_ADD),
    (2, 300, 1024, O.F16, O.W_Q8_G32, O.EPI_SILU),
    (24, 520, 1536, O.F16, O.W_DENSE, O.EPI_ADD), (1, 2560, 5120, O.BF16, O.W_Q4_G64, O.EPI_ADD),
    (3, 777, 2560, O.BF16, O.W_Q4_B32, O.EPI_NONE), (6, 512, 1024, O.BF16, O.W_DENSE, O.EPI_NONE),
]


@pytest.mark.parametrize("rows,N,K,act,wfmt,epi", NORM_LINEAR_CASES,
                         ids=[f"m{m}-n{n}-k{k}-{['f16', 'bf16', 'f32'][a]}-w{w}-e{e}" for m, n, k, a, w, e in NORM_LINEAR_CASES])
def test_norm_linear_decode_vs_oracle(ctx, rng, rows, N, K, act, wfmt, epi):
    """RMSNorm + linear (+ residual) for decode rows: the GEMV rule (exact
    dequantization) at every row count, against the oracle's chain."""
    L = _lib()
    x = O.to_act(rng.standard_normal((rows, K)) * 0.7, act)
    nw = O.to_act(1 + 0.1 * rng.standard_normal(K), act)
    w, s = _weights(rng, N, K, wfmt, act)
    res = O.to_act(rng.standard_normal((rows, N)), act)
    y = dev(res) if epi == O.EPI_ADD else empty((rows, N), act)
    L.check(L.lib.lssm_norm_linear_decode(ctx.h, dev(x).data_ptr(), dev(nw).data_ptr(), 1e-5,
                                          dev(w).data_ptr(), None if s is None else dev(s).data_ptr(),
                                          y.data_ptr(), y.data_ptr() if epi == O.EPI_ADD else None,
                                          rows, N, K, wfmt, act, epi))
    normed = O.rmsnorm(x, nw, 1e-5, act)
    ref = O.linear(normed, w, s, rows, N, K, wfmt, act, epi=epi, residual=res if epi == O.EPI_ADD else None)
    assert_close(act_host(y, act), ref, act, {O.F16: 2e-3, O.BF16: 1.6e-2}[act], "norm_linear_decode")


def test_norm_linear_decode_graph_replays_match_eager(ctx, rng):
    """The MFMA decode GEMV (16 rows, 2.7B out_proj) replayed from a HIP graph
    gives the eager bits on every replay (no memset nodes, deterministic sums)."""
    L = _lib()
    rows, N, K = 16, 2560, 5120
    x = dev(O.to_act(rng.standard_normal((rows, K)) * 0.7, O.BF16))
    nw = dev(O.to_act(1 + 0.1 * rng.standard_normal(K), O.BF16))
    w, s = _weights(rng, N, K, O.W_Q4_G64, O.BF16)
    wd, sd = dev(w), dev(s)
    y = empty((rows, N), O.BF16)
    run = lambda: L.check(L.lib.lssm_norm_linear_decode(ctx.h, x.data_ptr(), nw.data_ptr(), 1e-5, wd.data_ptr(),
                                                        sd.data_ptr(), y.data_ptr(), None, rows, N, K,
                                                        O.W_Q4_G64, O.BF16, O.EPI_NONE))
    run()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    c2 = L.Ctx(st.cuda_stream)
    y.zero_()
    torch.cuda.synchronize()
    c2.begin_batch()                      # enqueue only: no stream sync inside the capture
    with torch.cuda.stream(st):
        g.capture_begin()
        L.check(L.lib.lssm_norm_linear_decode(c2.h, x.data_ptr(), nw.data_ptr(), 1e-5, wd.data_ptr(),
                                              sd.data_ptr(), y.data_ptr(), None, rows, N, K,
                                              O.W_Q4_G64, O.BF16, O.EPI_NONE))
        g.capture_end()
    c2.commit_and_wait()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        run()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


@pytest.mark.parametrize("act", [O.F16, O.BF16])
def test_embed_and_argmax(ctx, rng, act):
    L = _lib()
    vocab, d = 50280, 256
    table = O.to_act(rng.standard_normal((vocab, d)), act)
    ids = np.array([0, 5, 50279, 1234], np.int32)
    out = empty((4, d), act)
    L.check(L.lib.lssm_embed(ctx.h, dev(table).data_ptr(), dev(ids).data_ptr(), out.data_ptr(), 4, d,
                             vocab, act))
    assert np.array_equal(act_host(out, act), table[ids])
    lg = O.to_act(rng.standard_normal((3, vocab)), act)
    top = O.to_act(np.array([99.0]), act)[0]
    lg[1, 777] = lg[1, 40000] = top                                    # tie -> first index
    lg[2, 8 * 3000 + 5] = lg[2, 8 * 3000 + 2] = lg[2, 8 * 4100 + 1] = top  # within one 8-value piece, and across threads
    got = torch.zeros(3, dtype=torch.int32, device="cuda")
    L.check(L.lib.lssm_argmax(ctx.h, dev(lg).data_ptr(), got.data_ptr(), 3, vocab, act))
    assert list(host(got, np.int32)) == list(O.argmax(lg, act))
    assert host(got, np.int32)[1] == 777 and host(got, np.int32)[2] == 8 * 3000 + 2
    # an odd vocabulary (the two-stage path) and a longer one (more than one pass of a block)
    for v, rows in ((50277, 2), (256000, 1), (65536, 4)):
        lg2 = O.to_act(rng.standard_normal((rows, v)), act)
        lg2[rows - 1, v - 1] = top
        got2 = torch.zeros(rows, dtype=torch.int32, device="cuda")
        L.check(L.lib.lssm_argmax(ctx.h, dev(lg2).data_ptr(), got2.data_ptr(), rows, v, act))
        assert list(host(got2, np.int32)) == list(O.argmax(lg2, act)), f"vocab {v}"
        assert host(got2, np.int32)[rows - 1] == v - 1


def test_batch_lifecycle_errors(ctx):
    L = _lib()
    ctx.begin_batch()
    assert ctx.batch_active()
    with pytest.raises(L.LssmError, match="already active"):
        ctx.begin_batch()
    ctx.commit_and_wait()
    with pytest.raises(L.LssmError, match="without an active batch"):
        ctx.commit_and_wait()
    assert L.lib.lssm_library_loaded() == 1

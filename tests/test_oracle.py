"""Pins of the CPU oracle (oracle/lssm_oracle.c) — no GPU.

The reference has no CPU implementation and commits no golden vectors
(.gitignore:27-28 excludes *.ssm / *.bin), so each oracle function is pinned
here against what the mathematics fixes: IEEE conversions checked against
numpy / torch, fp64 brute force, closed forms (the chunked SSD equals the
sequential recurrence; a vanishing decay reduces it to a cumulative sum),
composition identities (conv update over a sequence == causal conv), and the
model-level identity prefill(L) + step == prefill(L + 1).  Each check is
chosen so that a dropped term, a wrong sign or index, or a transposed operand
fails it.
"""
import numpy as np
import pytest
import torch

import oracle as O

ACTS = [O.F16, O.BF16, O.F32]


def f16_ulp(v):
    v = np.abs(np.asarray(v, np.float32))
    e = np.floor(np.log2(np.maximum(v, 6.1e-5)))
    return 2.0 ** (e - 10)


# --------------------------------------------------------------------------- conversions
def test_f16_conversion_matches_numpy_rne(rng):
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8,
                  6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    bits = O.to_act(x, O.F16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(bits, ref)
    back = O.from_act(bits, O.F16)
    assert np.array_equal(back, ref.view(np.float16).astype(np.float32))


def test_bf16_conversion_matches_torch_rne(rng):
    x = (rng.standard_normal(200000) * 10.0 ** rng.integers(-30, 30, 200000)).astype(np.float32)
    ties = np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0xBF808000], np.uint32).view(np.float32)
    x = np.concatenate([x, ties, np.array([0.0, -0.0, 3e38, -3e38], np.float32)])
    bits = O.to_act(x, O.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, ref)
    # ties go to even: 1 + 2^-8 -> 1.0 ; 1 + 3*2^-8 -> 1 + 2^-6
    assert list(bits[-8:-4]) == [0x3F80, 0x3F82, 0x3F81, 0xBF80]


# --------------------------------------------------------------------------- quantizer
def _np_unpack(packed, scales, wfmt):
    """Independent numpy dequantization of the [packed][scales] layout."""
    G = O.group_size(wfmt)
    if wfmt == O.W_Q8_G32:
        q = packed.view(np.int8).astype(np.int32)
    else:
        lo = (packed & 0x0F).astype(np.int32)
        hi = (packed >> 4).astype(np.int32)
        q = np.stack([lo, hi], -1).reshape(packed.shape[0], -1)
        q = np.where(q >= 8, q - 16, q)
    s = scales.view(np.float16).astype(np.float32)
    return q, q.astype(np.float32) * np.repeat(s, G, axis=1)


@pytest.mark.parametrize("wfmt", [O.W_Q4_B32, O.W_Q4_G64, O.W_Q8_G32])
def test_quantizer_properties(rng, wfmt):
    N, K = 48, 256
    G = O.group_size(wfmt)
    qmax = 127 if wfmt == O.W_Q8_G32 else 7
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16).astype(np.float32)
    w[3, :G] = 0.0                                   # all-zero group (clamp at 1e-12)
    packed, scales = O.quantize(w, wfmt)
    q, deq = _np_unpack(packed, scales, wfmt)
    blocks = w.reshape(N, K // G, G)
    amax = np.maximum(np.abs(blocks).max(-1), np.float32(1e-12))
    scale32 = (amax / np.float32(qmax)).astype(np.float32)
    assert np.array_equal(scales, scale32.astype(np.float16).view(np.uint16))
    assert q.min() >= -qmax - 1 and q.max() <= qmax
    # the absmax element of each group quantizes to +-qmax
    idx = np.abs(blocks).argmax(-1)
    qa = np.take_along_axis(q.reshape(N, K // G, G), idx[..., None], -1)[..., 0]
    nz = amax > 1e-12
    assert np.all(np.abs(qa[nz]) == qmax)
    # q = round_half_even(w / scale_f32): residual bounded by half a step
    r = blocks / scale32[..., None] - q.reshape(N, K // G, G)
    assert np.all(np.abs(r) <= 0.5 + 1e-6)
    assert np.all(q.reshape(N, K // G, G)[3, 0] == 0)
    # dequant of the oracle matches the independent unpack bit for bit
    assert np.array_equal(O.dequant(packed, scales, N, K, wfmt), deq)


def test_quantizer_ties_to_even_and_nibble_order():
    # group of 32: absmax 7 -> scale 1.0, values at exact .5 ties
    w = np.zeros((1, 32), np.float32)
    w[0, :8] = [7.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5]
    packed, scales = O.quantize(w, O.W_Q4_B32)
    q, _ = _np_unpack(packed, scales, O.W_Q4_B32)
    assert list(q[0, :8]) == [7, 2, 4, -2, -4, 0, 2, 0]
    # low nibble is the even k (linear.metal:47-61): byte0 = (q1 & 0xF) << 4 | (q0 & 0xF)
    assert packed[0, 0] == ((2 & 0xF) << 4) | 7
    assert packed[0, 1] == ((-2 & 0xF) << 4) | 4


@pytest.mark.parametrize("wfmt", [O.W_Q4_B32, O.W_Q4_G64, O.W_Q8_G32])
def test_oracle_quantizer_matches_device_quantizer_on_cpu(rng, wfmt):
    from lite_ssm_amd.model import quantize as tq
    w = (rng.standard_normal((32, 512)) * 0.02).astype(np.float16).astype(np.float32)
    p1, s1 = O.quantize(w, wfmt)
    p2, s2 = tq(torch.from_numpy(w), wfmt)
    assert np.array_equal(p1, p2.numpy())
    assert np.array_equal(s1, s2.view(torch.int16).numpy().view(np.uint16))


# --------------------------------------------------------------------------- linear
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("wfmt", [O.W_DENSE, O.W_Q4_B32, O.W_Q4_G64, O.W_Q8_G32])
def test_linear_vs_fp64(rng, act, wfmt):
    M, N, K = 3, 40, 256
    x = O.to_act(rng.standard_normal((M, K)), act)
    xf = O.from_act(x, act).astype(np.float64)
    wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if wfmt == O.W_DENSE:
        w, s = O.to_act(wf, act), None
        W = O.from_act(w, act).astype(np.float64)
    else:
        w, s = O.quantize(wf, wfmt)
        W = _np_unpack(w, s, wfmt)[1].astype(np.float64)
    for rd in (0, 1):
        Wr = W if (rd == 0 or wfmt == O.W_DENSE) else O.round_act(W.astype(np.float32), act).astype(np.float64)
        ref = (xf @ Wr.T).astype(np.float32)
        y = O.from_act(O.linear(x, w, s, M, N, K, wfmt, act, round_dequant=rd), act)
        exp_ = O.round_act(ref, act)
        # exact up to the double rounding fp64 -> fp32 -> act: at most one ulp of act
        tol = np.abs(exp_) * {O.F16: 2 ** -10, O.BF16: 2 ** -7, O.F32: 2 ** -22}[act] + 1e-30
        assert np.all(np.abs(y - exp_) <= tol)
        assert np.mean(y == exp_) > 0.99
    # epilogues
    acc = (xf @ W.T).astype(np.float32)
    ys = O.from_act(O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_SILU), act)
    sil = O.round_act(acc / (1 + np.exp(-acc)), act)
    assert np.allclose(ys, sil, rtol=2 ** -7, atol=1e-6)
    res = O.to_act(rng.standard_normal((M, N)), act)
    ya = O.from_act(O.linear(x, w, s, M, N, K, wfmt, act, epi=O.EPI_ADD, residual=res), act)
    ref_add = O.round_act(O.from_act(res, act) + O.round_act(acc, act), act)
    assert np.allclose(ya, ref_add, rtol=2 ** -7, atol=1e-6)


def test_linear_float32_sums_mode(rng):
    """O.accum_f32(): the linears sum in float32 (sixteen partial sums) instead
    of double.  Pinned against fp64: within the float32 summation bound
    (K + 16) * 2^-24 * sum |w x| of the exact product, not bit-equal to the
    double mode somewhere at K = 5120 (a different order really runs), bf16
    outputs equal to the double mode's wherever the exact value is not within
    that bound of a bf16 rounding boundary, and the default restored on exit."""
    M, N, K = 4, 256, 5120
    x = (rng.standard_normal((M, K))).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = (K + 16) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    y64 = O.linear(x, w, None, M, N, K, O.W_DENSE, O.F32)
    with O.accum_f32():
        y32 = O.linear(x, w, None, M, N, K, O.W_DENSE, O.F32)
    assert np.all(np.abs(y64 - exact) <= np.abs(exact) * 2.0 ** -24 + 1e-30)
    assert np.all(np.abs(y32 - exact) <= bound)
    assert not np.array_equal(y32, y64)
    # back to double sums after the block
    assert np.array_equal(O.linear(x, w, None, M, N, K, O.W_DENSE, O.F32), y64)
    # bf16 outputs: the two modes round to the same value unless the exact sum
    # lies within the float32 bound of a rounding boundary
    xb, wb = O.to_act(x, O.BF16), O.to_act(w, O.BF16)
    exb = O.from_act(xb, O.BF16).astype(np.float64) @ O.from_act(wb, O.BF16).astype(np.float64).T
    b64 = O.from_act(O.linear(xb, wb, None, M, N, K, O.W_DENSE, O.BF16), O.BF16)
    with O.accum_f32():
        b32 = O.from_act(O.linear(xb, wb, None, M, N, K, O.W_DENSE, O.BF16), O.BF16)
    lo = O.round_act((exb - bound).astype(np.float32), O.BF16)
    hi = O.round_act((exb + bound).astype(np.float32), O.BF16)
    clear = lo == hi
    assert np.array_equal(b32[clear], b64[clear])


# --------------------------------------------------------------------------- norms / activations
@pytest.mark.parametrize("act", ACTS)
def test_rmsnorm_vs_fp64(rng, act):
    x = O.to_act(rng.standard_normal((5, 768)) * 3, act)
    w = O.to_act(1 + 0.1 * rng.standard_normal(768), act)
    y = O.from_act(O.rmsnorm(x, w, 1e-5, act), act)
    xf, wf = O.from_act(x, act).astype(np.float64), O.from_act(w, act).astype(np.float64)
    ref = xf * wf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5)
    tol = {O.F16: 2 ** -10, O.BF16: 2 ** -7, O.F32: 1e-6}[act]
    assert np.allclose(y, ref, rtol=tol, atol=1e-6)


def _round_np(v, act):
    """fp64 -> activation dtype (RNE) through numpy / torch, not the oracle."""
    v = np.asarray(v, np.float64)
    if act == O.F16:
        return v.astype(np.float16).astype(np.float64)
    if act == O.BF16:
        return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()
    return v.astype(np.float32).astype(np.float64)


def _ulps(a, b, act):
    """|a - b| in units of the activation dtype's spacing at |b|."""
    mant = {O.F16: 10, O.BF16: 7, O.F32: 23}[act]
    e = np.floor(np.log2(np.maximum(np.abs(b), 2.0 ** -14)))
    return np.abs(a - b) / 2.0 ** (e - mant)


@pytest.mark.parametrize("act", ACTS)
def test_silu_gated_vs_fp64(rng, act):
    """activations.metal:76-87: y = r(silu(x) * gate), one rounding.  x and gate
    have different distributions, so silu(gate) * x (swapped operands) or a
    missing SiLU fails by far more than an ulp."""
    x = O.to_act(rng.standard_normal(20000) * 3 + 0.5, act)
    gate = O.to_act(rng.uniform(-2, 2, 20000), act)
    got = O.from_act(O.silu_gated(x, gate, act), act).astype(np.float64)
    xf = O.from_act(x, act).astype(np.float64)
    gf = O.from_act(gate, act).astype(np.float64)
    ref = _round_np(xf / (1 + np.exp(-xf)) * gf, act)
    u = _ulps(got, ref, act)
    # the reference computes silu(x) * gate in fp32 (exp, divide, multiply)
    # before r(): one ulp at most in fp16 / bf16, a few fp32 ulps in fp32
    assert u.max() <= (4.0 if act == O.F32 else 1.0), f"max {u.max()} ulp"
    assert (u == 0).mean() > (0.5 if act == O.F32 else 0.99)
    swapped = _round_np(gf / (1 + np.exp(-gf)) * xf, act)
    assert _ulps(got, swapped, act).max() > 100


@pytest.mark.parametrize("act", ACTS)
def test_add_inplace_vs_fp64(rng, act):
    """activations.metal:24-32: y = r(y + x), in place.  Operands of mixed
    magnitude; the sum of two same-dtype values of nearby exponent is exact in
    fp32, so the fp64 sum rounded once must match bit for bit."""
    y0 = O.to_act(rng.standard_normal(20000) * 2, act)
    x = O.to_act(rng.standard_normal(20000) * 0.5 + 0.25, act)
    y = y0.copy()
    O.add_inplace(y, x, act)
    got = O.from_act(y, act).astype(np.float64)
    ref = _round_np(O.from_act(y0, act).astype(np.float64) + O.from_act(x, act).astype(np.float64), act)
    assert np.array_equal(got, ref)
    # the addend is x, not y again, and nothing is subtracted
    assert not np.array_equal(got, _round_np(2 * O.from_act(y0, act).astype(np.float64), act))


@pytest.mark.parametrize("act", [O.F16, O.BF16])
def test_gated_rmsnorm_vs_fp64(rng, act):
    """Gate-then-norm over the full d_inner row (activations.metal:83-86, then
    norm.metal:52-79): g = r(silu(z) * y), out = r(g * w / sqrt(mean g^2 + eps)),
    computed here in fp64 with the one intermediate rounding of g."""
    z = O.to_act(rng.standard_normal((4, 512)), act)
    y = O.to_act(rng.standard_normal((4, 512)) * 2, act)
    w = O.to_act(1 + 0.1 * rng.standard_normal(512), act)
    got = O.from_act(O.gated_rmsnorm(z, y, w, 1e-5, act), act).astype(np.float64)
    zf, yf, wf = (O.from_act(a, act).astype(np.float64) for a in (z, y, w))
    g = _round_np(zf / (1 + np.exp(-zf)) * yf, act)
    ref = _round_np(g * wf / np.sqrt((g ** 2).mean(-1, keepdims=True) + 1e-5), act)
    assert _ulps(got, ref, act).max() <= 1.0
    # the gate is silu(z), not silu(y): swapping the roles fails
    g2 = _round_np(yf / (1 + np.exp(-yf)) * zf, act)
    ref2 = _round_np(g2 * wf / np.sqrt((g2 ** 2).mean(-1, keepdims=True) + 1e-5), act)
    assert _ulps(got, ref2, act).max() > 100


@pytest.mark.parametrize("act", [O.F16, O.BF16])
def test_gated_rmsnorm_is_gate_then_norm(rng, act):
    z = O.to_act(rng.standard_normal((4, 512)), act)
    y = O.to_act(rng.standard_normal((4, 512)), act)
    w = O.to_act(1 + 0.1 * rng.standard_normal(512), act)
    fused = O.gated_rmsnorm(z, y, w, 1e-5, act)
    two = O.rmsnorm(O.silu_gated(z, y, act), w, 1e-5, act)
    assert np.array_equal(fused, two)


def test_split_silu_and_silu(rng):
    act = O.F16
    d_inner, N, G, rows = 64, 16, 2, 3
    xbc = O.to_act(rng.standard_normal((rows, d_inner + 2 * G * N)) * 4, act)
    x, B, Cc = O.split_silu_xbc(xbc, rows, d_inner, N, G, act)
    v = O.from_act(xbc, act).astype(np.float64)
    s = O.round_act((v / (1 + np.exp(-v))).astype(np.float32), act)
    assert np.allclose(O.from_act(x, act), s[:, :d_inner], rtol=2 ** -10, atol=1e-7)
    assert np.allclose(O.from_act(B, act), s[:, d_inner:d_inner + G * N], rtol=2 ** -10, atol=1e-7)
    assert np.allclose(O.from_act(Cc, act), s[:, d_inner + G * N:], rtol=2 ** -10, atol=1e-7)
    assert np.array_equal(O.silu(xbc, act)[:, :d_inner], x)


def test_argmax_first_max_and_embed(rng):
    lg = O.to_act(rng.standard_normal((3, 100)), O.F16)
    lg[1, 10] = lg[1, 70] = O.to_act(np.array([50.0]), O.F16)[0]
    ids = O.argmax(lg, O.F16)
    assert ids[1] == 10
    assert ids[0] == int(np.argmax(O.from_act(lg[0], O.F16)))
    table = O.to_act(rng.standard_normal((10, 8)), O.BF16)
    out = O.embed(table, [3, 0, 9], 8, O.BF16)
    assert np.array_equal(out, table[[3, 0, 9]])


# --------------------------------------------------------------------------- conv
@pytest.mark.parametrize("act", ACTS)
def test_conv1d_vs_numpy_convolve(rng, act):
    B, L, D, K = 2, 19, 12, 4
    x = O.to_act(rng.standard_normal((B, L, D)), act)
    w = O.to_act(rng.standard_normal((D, K)) * 0.5, act)
    b = O.to_act(rng.standard_normal(D) * 0.1, act)
    y = O.from_act(O.conv1d(x, w, b, B, L, D, K, act), act)
    xf, wf, bf = (O.from_act(a, act).astype(np.float64) for a in (x, w, b))
    ref = np.zeros((B, L, D))
    for bb in range(B):
        for d in range(D):
            # y[t] = b + sum_tap w[tap] x[t - (K-1-tap)]  ==  full convolution with w reversed
            ref[bb, :, d] = np.convolve(xf[bb, :, d], wf[d, ::-1])[:L] + bf[d]
    tol = {O.F16: 2 ** -10, O.BF16: 2 ** -7, O.F32: 1e-6}[act]
    assert np.allclose(y, ref, rtol=tol, atol=1e-5)


@pytest.mark.parametrize("act", ACTS)
def test_conv_update_sequence_equals_causal_conv_and_seed(rng, act):
    B, L, D, K = 2, 11, 9, 4
    x = O.to_act(rng.standard_normal((B, L, D)), act)
    w = O.to_act(rng.standard_normal((D, K)) * 0.5, act)
    b = O.to_act(rng.standard_normal(D) * 0.1, act)
    full = O.conv1d(x, w, b, B, L, D, K, act)
    state = np.zeros((B, D, K), dtype=O.act_np_dtype(act))
    for t in range(L):
        y = O.conv1d_update(np.ascontiguousarray(x[:, t]), state, w, b, B, D, K, act)
        assert np.array_equal(y, full[:, t])
    assert np.array_equal(state, O.conv1d_seed(x, B, L, D, K, act))
    short = O.conv1d_seed(np.ascontiguousarray(x[:, :2]), B, 2, D, K, act)
    assert np.all(O.from_act(short[:, :, :2], act) == 0)
    assert np.array_equal(short[:, :, 2:], np.ascontiguousarray(x[:, :2].transpose(0, 2, 1)))


# --------------------------------------------------------------------------- SSD
def _ssd_inputs(rng, batch, L, H, P, N, G, act, dt_mean=-2.0):
    X = O.to_act(rng.standard_normal((batch, L, H, P)), act)
    B = O.to_act(rng.standard_normal((batch, L, G, N)) / np.sqrt(N), act)
    Cc = O.to_act(rng.standard_normal((batch, L, G, N)) / np.sqrt(N), act)
    dt = O.to_act(rng.normal(dt_mean, 0.5, (batch, L, H)), act)
    dtb = O.to_act(np.zeros(H), act)
    A_log = O.to_act(rng.uniform(0, np.log(16), H), act)
    D = O.to_act(rng.standard_normal(H), act)
    return X, B, Cc, dt, dtb, A_log, D


def _ssd_recurrence_fp64(X, B, Cc, dt, dtb, A_log, D, state, act):
    """Sequential Mamba-2 recurrence in fp64 (ssd_step.metal:55-76 applied per token)."""
    f = lambda a: O.from_act(a, act).astype(np.float64)
    X, B, Cc, dt, dtb, A_log, D = map(f, (X, B, Cc, dt, dtb, A_log, D))
    batch, L, H, P = X.shape
    G = B.shape[2]
    S = state.astype(np.float64).copy()
    Y = np.zeros_like(X)
    A = -np.exp(A_log)
    for t in range(L):
        v = dt[:, t] + dtb
        d = np.where(v > 20, v, np.log1p(np.exp(v)))
        d = np.clip(d, 1e-6, 1e6)                                   # [batch, H]
        for h in range(H):
            g = h // (H // G)
            S[:, h] = np.exp(A[h] * d[:, h])[:, None, None] * S[:, h] + \
                (d[:, h][:, None, None] * X[:, t, h][:, :, None] * B[:, t, g][:, None, :])
            Y[:, t, h] = (S[:, h] * Cc[:, t, g][:, None, :]).sum(-1) + D[h] * X[:, t, h]
    return Y, S


@pytest.mark.parametrize("G,H", [(1, 4), (2, 4)])
def test_ssd_step_vs_fp64(rng, G, H):
    act = O.F32
    batch, P, N = 2, 8, 16
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, 1, H, P, N, G, act)
    st = (rng.standard_normal((batch, H, P, N)) * 0.3).astype(np.float32)
    Yr, Sr = _ssd_recurrence_fp64(X, B, Cc, dt, dtb, A_log, D, st, act)
    s2 = st.copy()
    y = O.ssd_step(np.ascontiguousarray(X[:, 0]), np.ascontiguousarray(B[:, 0]),
                   np.ascontiguousarray(Cc[:, 0]), np.ascontiguousarray(dt[:, 0]), dtb, A_log, D,
                   s2, batch, H, P, N, G, act)
    assert np.allclose(y, Yr[:, 0], rtol=1e-5, atol=1e-5)
    assert np.allclose(s2, Sr, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("chunk", [64, 16, 7])
def test_ssd_chunked_fp32_equals_sequential_recurrence(rng, chunk):
    act = O.F32
    batch, L, H, P, N, G = 2, 150, 4, 16, 32, 2
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, L, H, P, N, G, act)
    st = (rng.standard_normal((batch, H, P, N)) * 0.3).astype(np.float32)
    Yr, Sr = _ssd_recurrence_fp64(X, B, Cc, dt, dtb, A_log, D, st, act)
    s2 = st.copy()
    Y = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s2, batch, L, H, P, N, G, chunk, act)
    scale = np.abs(Yr).max()
    assert np.abs(Y - Yr).max() <= 1e-4 * scale
    assert np.abs(s2 - Sr).max() <= 1e-4 * np.abs(Sr).max()


def test_ssd_chunked_vanishing_decay_is_cumulative_sum(rng):
    """A -> 0 (A_log = -30): S_t = S_0 + sum_{j<=t} dt_j x_j B_j^T exactly."""
    act = O.F32
    batch, L, H, P, N, G = 1, 70, 2, 4, 8, 1
    X, B, Cc, dt, dtb, _, D = _ssd_inputs(rng, batch, L, H, P, N, G, act)
    A_log = O.to_act(np.full(H, -30.0), act)
    st = np.zeros((batch, H, P, N), np.float32)
    Y = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, st, batch, L, H, P, N, G, 64, act)
    v = O.from_act(dt, act).astype(np.float64)
    d = np.log1p(np.exp(v))
    Xf, Bf, Cf = (O.from_act(a, act).astype(np.float64) for a in (X, B, Cc))
    contrib = d[..., None, None] * Xf[..., :, None] * Bf[:, :, :1, None, :]   # [b, L, H, P, N]
    S = np.cumsum(contrib, axis=1)
    Yref = (S * Cf[:, :, :1, None, :]).sum(-1) + O.from_act(D, act)[None, None, :, None] * Xf
    assert np.allclose(Y, Yref, rtol=1e-4, atol=1e-5)
    assert np.allclose(st, S[:, -1], rtol=1e-4, atol=1e-6)


def test_ssd_chunked_l1_equals_step(rng):
    act = O.F32
    batch, H, P, N, G = 1, 3, 8, 16, 1
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, 1, H, P, N, G, act)
    st = (rng.standard_normal((batch, H, P, N)) * 0.3).astype(np.float32)
    s1, s2 = st.copy(), st.copy()
    Y = O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, s1, batch, 1, H, P, N, G, 1, act)
    y = O.ssd_step(np.ascontiguousarray(X[:, 0]), np.ascontiguousarray(B[:, 0]),
                   np.ascontiguousarray(Cc[:, 0]), np.ascontiguousarray(dt[:, 0]), dtb, A_log, D,
                   s2, batch, H, P, N, G, act)
    assert np.allclose(Y[:, 0], y, rtol=1e-5, atol=1e-6)
    assert np.allclose(s1, s2, rtol=1e-5, atol=1e-7)


def test_ssd_chunked_f16_rounding_points_close_to_exact(rng):
    """fp16 storage of M and S (the reference's rounding points) stays within
    the 2e-2 bound of the exact recurrence."""
    act = O.F16
    batch, L, H, P, N, G = 1, 200, 3, 16, 64, 1
    X, B, Cc, dt, dtb, A_log, D = _ssd_inputs(rng, batch, L, H, P, N, G, act)
    st = np.zeros((batch, H, P, N), np.float32)
    Yr, _ = _ssd_recurrence_fp64(X, B, Cc, dt, dtb, A_log, D, st, act)
    Y = O.from_act(O.ssd_chunked(X, B, Cc, dt, dtb, A_log, D, st, batch, L, H, P, N, G, 64, act), act)
    assert np.abs(Y - Yr).max() <= 2e-2 * np.abs(Yr).max()


# --------------------------------------------------------------------------- fused in_proj
def test_inproj_fused_vs_unfused_chain(rng):
    act = O.F16
    L, d_model, d_inner, N, G, H, K = 9, 64, 128, 16, 1, 2, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    normed = O.to_act(rng.standard_normal((L, d_model)), act)
    W = O.to_act(rng.standard_normal((proj, d_model)) * 0.1, act)
    Wc = O.to_act(rng.standard_normal((xbc, K)) * 0.5, act)
    cb = O.to_act(rng.standard_normal(xbc) * 0.1, act)
    z, x, B, Cc, dtv, pxbc = O.inproj_fused(normed, W, Wc, cb, L, d_model, d_inner, N, G, H, K)
    full = O.linear(normed, W, None, L, proj, d_model, O.W_DENSE, act)
    assert np.array_equal(z, full[:, :d_inner])
    assert np.array_equal(pxbc, full[:, d_inner:d_inner + xbc])
    assert np.array_equal(dtv, full[:, d_inner + xbc:])
    conv = O.conv1d(np.ascontiguousarray(full[None, :, d_inner:d_inner + xbc]), Wc, cb, 1, L, xbc, K, act)
    x2, B2, C2 = O.split_silu_xbc(conv[0], L, d_inner, N, G, act)
    for a, b in ((x, x2), (B, B2), (Cc, C2)):
        fa, fb = O.from_act(a, act), O.from_act(b, act)
        assert np.allclose(fa, fb, rtol=4e-3, atol=4e-3)   # conv on unrounded fp32 (fused.metal:140-149)


# --------------------------------------------------------------------------- model
def test_mamba2_130m_shape_constants():
    """tests/test_mmap_loader.cpp:64-92: in_proj 3352 x 768, conv dim 1792."""
    from lite_ssm_amd.model import shape
    s = shape("mamba2-130m")
    assert (s.proj, s.d_model, s.xbc, s.n_heads * s.d_head) == (3352, 768, 1792, 1536)
    s27 = shape("mamba2-2.7b")
    assert (s27.proj, s27.xbc) == (10576, 5376)
    s8 = shape("mamba2-8b")
    assert (s8.proj, s8.xbc) == (18560, 10240)


def _tiny_host_model(rng, act, wfmt, n_layer=2, d_model=64, vocab=97, G=1):
    d_inner, N, K, H = 2 * d_model, 16, 4, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H

    def lin(Nr, Kc):
        w = (rng.standard_normal((Nr, Kc)) * 0.05).astype(np.float32)
        if wfmt == O.W_DENSE:
            return O.to_act(w, act), None
        return O.quantize(w, wfmt)

    layers = []
    for _ in range(n_layer):
        ip, ips = lin(proj, d_model)
        op, ops_ = lin(d_model, d_inner)
        layers.append(dict(
            norm_w=O.to_act(1 + 0.1 * rng.standard_normal(d_model), act), in_proj_w=ip, in_proj_s=ips,
            conv1d_w=O.to_act(rng.standard_normal((xbc, K)) * 0.3, act),
            conv1d_b=O.to_act(rng.standard_normal(xbc) * 0.1, act),
            dt_bias=O.to_act(rng.normal(-2, 0.5, H), act), A_log=O.to_act(rng.uniform(0, 2.7, H), act),
            D=O.to_act(1 + 0.1 * rng.standard_normal(H), act),
            mixer_norm_w=O.to_act(1 + 0.1 * rng.standard_normal(d_inner), act),
            out_proj_w=op, out_proj_s=ops_))
    emb = O.to_act(rng.standard_normal((vocab, d_model)) * 0.5, act)
    host = dict(embed=emb, norm_f=O.to_act(1 + 0.1 * rng.standard_normal(d_model), act),
                lm_head=emb, layers=layers)
    cfg = dict(d_model=d_model, n_layer=n_layer, d_state=N, d_conv=K, expand=2, vocab_size=vocab,
               n_heads=H, d_head=d_inner // H, chunk_size=256, n_groups=G)
    return O.Model(host, cfg, act, wfmt)


def test_model_prefill_plus_step_equals_longer_prefill(rng):
    """fp32 activations + dense weights have no storage rounding, so the chunked
    prefill of L+1 tokens must equal prefill(L) followed by one decode step:
    this pins the conv-state seed, the SSD state hand-off and the op order."""
    m = _tiny_host_model(rng, O.F32, O.W_DENSE, G=2)
    ids = rng.integers(0, 97, (2, 71)).astype(np.int32)
    c1, s1 = m.new_state(2)
    m.prefill(c1, s1, ids[:, :70])
    lg_step = m.decode(c1, s1, np.ascontiguousarray(ids[:, 70]))
    c2, s2 = m.new_state(2)
    lg_full = m.prefill(c2, s2, ids)
    assert np.allclose(lg_step, lg_full, rtol=1e-4, atol=1e-4)
    assert np.allclose(s1, s2, rtol=1e-4, atol=1e-5)
    assert np.allclose(c1, c2, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("L", [2, 12, 16, 17])
def test_model_short_fp16_prefill_vs_token_steps(rng, L):
    """fp16 dense weights: a prefill of 1 < L <= 16 tokens takes the reference's
    fused in_proj + conv branch (mamba2_block.cpp:97-98,130-148; the conv reads
    the unrounded projection), longer ones the chunked path.  Either way it
    must agree, within fp16 rounding, with L single-token steps from a zero
    state (the decode recurrence), in logits, SSD state and conv state.  (The
    fused op itself equals the unfused chain up to that rounding:
    test_inproj_fused_vs_unfused_chain.)"""
    m = _tiny_host_model(rng, O.F16, O.W_DENSE, G=2)
    ids = rng.integers(0, 97, (2, L)).astype(np.int32)
    c1, s1 = m.new_state(2)
    lg = O.from_act(m.prefill(c1, s1, ids), O.F16)
    c2, s2 = m.new_state(2)
    for t in range(L):
        lg_s = O.from_act(m.decode(c2, s2, np.ascontiguousarray(ids[:, t])), O.F16)
    assert np.abs(lg - lg_s).max() <= 2e-2 * np.abs(lg_s).max()
    assert np.abs(s1 - s2).max() <= 2e-2 * np.abs(s2).max()
    # the conv window holds the last K pre-conv projections: rounded once on
    # both routes, from projections that differ only by rounding
    cf, cs = O.from_act(c1, O.F16), O.from_act(c2, O.F16)
    assert np.abs(cf - cs).max() <= 2e-2 * np.abs(cs).max()


@pytest.mark.parametrize("act,wfmt", [(O.F16, O.W_Q4_B32), (O.BF16, O.W_Q4_G64), (O.F16, O.W_Q8_G32)])
def test_model_batch_rows_are_independent(rng, act, wfmt):
    m = _tiny_host_model(rng, act, wfmt)
    ids = rng.integers(0, 97, (2, 20)).astype(np.int32)
    c, s = m.new_state(2)
    lg = m.prefill(c, s, ids)
    c1, s1 = m.new_state(1)
    lg1 = m.prefill(c1, s1, ids[1:2])
    assert np.array_equal(lg[1:2], lg1)
    nxt = m.decode(c, s, np.array([5, 7], np.int32))
    nxt1 = m.decode(c1, s1, np.array([7], np.int32))
    assert np.array_equal(nxt[1:2], nxt1)

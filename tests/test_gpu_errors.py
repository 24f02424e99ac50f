"""Device-side failure reporting: conditions a kernel detects (a token id out of
range, a bounded cross-workgroup wait that gives up) reach the host as errors
at the next synchronisation point instead of silently corrupting results.

The reference throws std::out_of_range for an id >= vocab
(src/model/mamba2_model.cpp:128-131) before anything runs; here ids live in
device memory, so the embedding kernel flags them and the host raises.  The
wait timeout is forced from the host (LSSM_DEBUG_STALE_WAIT: the SSD items wait
for a tag that no workgroup publishes), so every kernel still exits normally.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import act_host, assert_close, dev, empty

pytestmark = pytest.mark.gpu


def _lib():
    import lite_ssm_amd as L
    return L


@pytest.mark.parametrize("bad", [-1, 50280])
def test_embed_out_of_range_id_raises(ctx, rng, bad):
    L = _lib()
    vocab, d = 50280, 256
    table = O.to_act(rng.standard_normal((vocab, d)), O.BF16)
    tdev = dev(table)
    ids = np.array([3, bad, 7], np.int32)
    out = empty((3, d), O.BF16)
    rc = L.lib.lssm_embed(ctx.h, tdev.data_ptr(), dev(ids).data_ptr(), out.data_ptr(), 3, d, vocab, O.BF16)
    assert rc == 1, "LSSM_EINVAL expected"
    assert "token_id out of range" in L.lib.lssm_last_error().decode()
    got = act_host(out, O.BF16)
    assert np.array_equal(got[0], table[3]) and np.array_equal(got[2], table[7])
    assert not got[1].any(), "an out-of-range id gives a zero row"
    # the status word was cleared: a good call afterwards succeeds
    good = np.array([0, vocab - 1, 1], np.int32)
    L.check(L.lib.lssm_embed(ctx.h, tdev.data_ptr(), dev(good).data_ptr(), out.data_ptr(), 3, d, vocab, O.BF16))
    assert np.array_equal(act_host(out, O.BF16), table[good])


def test_engine_out_of_range_id_raises(ctx):
    L = _lib()
    from lite_ssm_amd.model import DeviceModel, Engine, shape
    sh = shape("mamba2-130m", n_layer=2, vocab_size=1000)
    m = DeviceModel(sh, act=O.F16, wfmt=O.W_Q8_G32, seed=3)
    eng = Engine(ctx, m, max_batch=2, max_seq=32)
    nxt = torch.zeros(2, dtype=torch.int32, device="cuda")
    ids = torch.randint(0, 1000, (2, 32), dtype=torch.int32)
    ids[1, 5] = 1000
    with pytest.raises(L.LssmError, match="token_id out of range"):
        eng.prefill(ids.cuda(), nxt)
    eng.reset()
    ids[1, 5] = 4
    eng.prefill(ids.cuda(), nxt)                               # clean again
    for bad in (-1, 1000):
        tok = torch.tensor([1, bad], dtype=torch.int32, device="cuda")
        with pytest.raises(L.LssmError, match="token_id out of range"):
            eng.decode(tok, nxt)
    # batch-1 graph replay reports it too
    tok = torch.tensor([2000], dtype=torch.int32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(L.LssmError, match="token_id out of range"):
        eng.decode_graph(tok, out, 2)
    tok.fill_(5)
    eng.decode_graph(tok, out, 1)                              # and recovers
    eng.close()


def test_fused_decode_wait_timeout_is_reported(ctx, rng):
    """The fused batch-1 in_proj + SSD launch with waits that cannot succeed:
    LSSM_EDEVICE, the SSD state untouched, the outputs NaN, the conv window
    shifted by the step's token (as the message says); afterwards the same
    call without the switch succeeds."""
    L = _lib()
    act, wfmt = O.F16, O.W_Q8_G32
    d_model, d_inner, N, G, H, K = 768, 1536, 128, 1, 24, 4
    P = d_inner // H
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    nw = dev(O.to_act(1 + 0.1 * rng.standard_normal(d_model), act))
    wq, sq = O.quantize((rng.standard_normal((proj, d_model)) * 0.02).astype(np.float32), wfmt)
    w, s = dev(wq), dev(sq)
    cw = dev(O.to_act(rng.standard_normal((xbc, K)) * 0.3, act))
    cb = dev(O.to_act(rng.standard_normal(xbc) * 0.1, act))
    dtb = dev(O.to_act(rng.standard_normal(H) * 0.5, act))
    alog = dev(O.to_act(rng.uniform(0, np.log(16), H), act))
    Dh = dev(O.to_act(rng.standard_normal(H), act))
    st0 = (rng.standard_normal((H, P, N)) * 0.1).astype(np.float32)
    st = dev(st0)
    cs = dev(O.to_act(rng.standard_normal((1, xbc, K)), act))
    hid = dev(O.to_act(rng.standard_normal((1, d_model)) * 0.5, act))
    y = empty((1, d_inner), act)
    xfer = torch.zeros(proj, dtype=torch.int64, device="cuda")

    def call(tag):
        return L.lib.lssm_inproj_ssd_decode(
            ctx.h, hid.data_ptr(), nw.data_ptr(), w.data_ptr(), s.data_ptr(), cs.data_ptr(), cw.data_ptr(),
            cb.data_ptr(), dtb.data_ptr(), alog.data_ptr(), Dh.data_ptr(), st.data_ptr(), y.data_ptr(),
            xfer.data_ptr(), tag, d_model, d_inner, N, G, H, P, K, 1e-5, wfmt, act)

    cs0 = act_host(cs, act).copy()
    ctx.set_debug(L.DEBUG_STALE_WAIT)
    try:
        rc = call(1)
        msg = L.lib.lssm_last_error().decode()
    finally:
        ctx.set_debug(0)
    assert rc == 2, "LSSM_EDEVICE expected"
    assert "timed out" in msg and "conv state did advance" in msg, msg
    assert np.array_equal(st.cpu().numpy(), st0), "SSD state must be left as it was"
    assert np.isnan(O.from_act(act_host(y, act), act)).all(), "timed-out outputs are NaN"
    # the conv window shifted: taps 1..3 moved down, the projection's xBC row in tap 3
    cs1 = act_host(cs, act)
    assert np.array_equal(cs1[..., :K - 1], cs0[..., 1:]), "conv window not shifted"
    normed = O.rmsnorm(act_host(hid, act), act_host(nw, act), 1e-5, act)
    prow = O.linear(normed, wq, sq, 1, proj, d_model, wfmt, act)
    assert_close(cs1[0, :, K - 1], prow[0, d_inner:d_inner + xbc], act, 2e-3, "conv tap 3")
    # without the switch: succeeds, state advanced, finite outputs
    L.check(call(2))
    assert not np.array_equal(st.cpu().numpy(), st0)
    assert np.isfinite(O.from_act(act_host(y, act), act)).all()

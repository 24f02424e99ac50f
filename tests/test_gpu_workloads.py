"""Parity on the code paths the BASELINE workloads take, at their shapes.

 * The dense lm_head GEMV with its norm_f prologue at the real vocabularies
   (50280 x 2560, 256000 x 4096, 50280 / 50288 x 768): many row-group passes
   per launch (mamba2_model.cpp:144-175, linear.metal:82-109).
 * Config 3 end to end (Mamba-2-130M shape: 24 layers, vocab 50280, int8-g32,
   fp16): a 2048-token prefill, then 256 greedy steps.  Teacher-forced logits
   at every step against the oracle, and the free-running greedy ids of the
   engine's graph-replayed decode against the oracle's own free-running ids
   (runtime/inference.cpp:55-67, first-max ties sampler.cpp:13-21).
 * Configs 4 and 5 (2.7B: 64 layers, vocab 50280; 8B: 56 layers, G = 8, vocab
   256000; int4-g64, bf16) at full depth and vocabulary, layer by layer: the
   engine records the hidden rows entering every layer (lssm_engine_set_trace)
   and the oracle runs run_block (mamba2_block.cpp:51-290) for each layer on
   exactly those rows, so an error cannot hide behind 64 layers of
   compounding; decode at batch 1 / 4 / 16 (2.7B) and 1 / 32 (8B).
 * The full-size prefills (4 x 4096 at 2.7B, 8192 at 8B): the first and last
   layers checked against the oracle on a whole 4096 / 8192-token sequence
   (the 64- and 128-chunk scans), finite logits, and a decode graph that is
   bit-identical to eager decode from the prefilled state.

Bounds: max-rel (max |gpu - ref| / max |ref|) 2e-2 for fp16 / bf16 tensors
(BASELINE north_star); greedy ids must agree wherever the oracle's top-2
margin exceeds twice the observed logit error.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import MAXREL, dev, max_rel

pytestmark = pytest.mark.gpu


def _bits(t):
    """device activation tensor -> numpy bit pattern (uint16) / float32."""
    a = t.detach().cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        return a.view(torch.int16).numpy().view(np.uint16)
    return a.numpy()


def _top2_margin(row):
    top2 = np.sort(row)[-2:]
    return float(top2[1] - top2[0])


def _check_ids(gpu_lg, ref_lg, what):
    """max-rel bound on logits; greedy ids equal where the margin is clear."""
    assert np.all(np.isfinite(gpu_lg)), f"{what}: non-finite logits"
    e = max_rel(gpu_lg, ref_lg)
    assert e <= 2e-2, f"{what}: logits max-rel {e:.3e}"
    err = np.abs(gpu_lg - ref_lg).max(axis=-1)
    for r in range(ref_lg.shape[0]):
        if _top2_margin(ref_lg[r]) > 2 * err[r]:
            assert int(np.argmax(gpu_lg[r])) == int(np.argmax(ref_lg[r])), f"{what}: greedy id row {r}"
    return e


# --------------------------------------------------------------------------- lm_head
LMHEAD = [(50280, 2560, O.BF16), (256000, 4096, O.BF16), (50280, 768, O.F16), (50288, 768, O.F16)]


@pytest.mark.parametrize("rows", [1, 3])
@pytest.mark.parametrize("N,K,act", LMHEAD, ids=[f"v{c[0]}-k{c[1]}" for c in LMHEAD])
def test_lm_head_gemv_real_vocab(ctx, N, K, act, rows):
    import lite_ssm_amd as L
    print(f"case: lm_head N={N} K={K} act={act} rows={rows}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(N + K + rows)
    tdt = torch.bfloat16 if act == O.BF16 else torch.float16
    w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(tdt)
    nw = (1 + 0.1 * torch.randn(K, generator=g, device="cuda")).to(tdt)
    x = (torch.randn(rows, K, generator=g, device="cuda") * 2).to(tdt)
    y = torch.zeros(rows, N, dtype=tdt, device="cuda")
    L.check(L.lib.lssm_norm_linear_decode(ctx.h, x.data_ptr(), nw.data_ptr(), 1e-5, w.data_ptr(), None,
                                          y.data_ptr(), None, rows, N, K, O.W_DENSE, act, O.EPI_NONE))
    normed = O.rmsnorm(_bits(x), _bits(nw), 1e-5, act)
    ref = O.from_act(O.linear(normed, _bits(w), None, rows, N, K, O.W_DENSE, act), act)
    got = O.from_act(_bits(y), act)
    bound = {O.F16: 2e-3, O.BF16: 1.6e-2}[act]
    e = max_rel(got, ref)
    assert np.all(np.isfinite(got)) and e <= bound, f"max-rel {e:.3e}"
    # every row of the weight was produced: compare the last rows exactly-ish too
    assert max_rel(got[:, -64:], ref[:, -64:]) <= bound
    _check_ids(got, ref, "lm_head")


# --------------------------------------------------------------------------- config 3
def test_config3_130m_prefill2048_greedy256(ctx, parity_record):
    from lite_ssm_amd.model import DeviceModel, Engine, shape
    print("case: config 3 (130M int8-g32 fp16, prefill 2048, 256 greedy steps)", flush=True)
    act, wfmt = O.F16, O.W_Q8_G32
    sh = shape("mamba2-130m")
    # embeddings ~ N(0, 1): logits spread over tens of units, so the top-2
    # margin is rarely below the fp16 resolution of the logits (with N(0, 0.02)
    # they sit within a few fp16 ulps of each other and ties are common).  The
    # head is a permutation of the embedding rows: with a tied head the
    # residual stream's copy of the input embedding makes the input token the
    # greedy choice again, and 256 free-running steps repeat one id.
    m = DeviceModel(sh, act=act, wfmt=wfmt, seed=3, embed_std=1.0, head="permuted")
    om = O.Model(m.to_host(), vars(sh), act, wfmt)
    Lp, steps = 2048, 256
    ids = torch.randint(0, sh.vocab_size, (1, Lp), generator=torch.Generator().manual_seed(33),
                        dtype=torch.int32)
    # oracle, free-running
    conv, ssd = om.new_state(1)
    ref = [O.from_act(om.prefill(conv, ssd, ids.numpy()), act)[0]]
    ref_ids = []
    for t in range(steps):
        ref_ids.append(int(O.argmax(O.to_act(ref[-1][None], act), act)[0]))
        if t + 1 < steps:
            ref.append(O.from_act(om.decode(conv, ssd, np.array([ref_ids[-1]], np.int32)), act)[0])
    print(f"oracle done: ids[:8] {ref_ids[:8]}", flush=True)
    eng = Engine(ctx, m, 1, Lp)
    try:
        # teacher-forced by the oracle's ids: logits at every step
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), nxt)
        errs, margins, errabs = [], [], []
        for t in range(steps):
            g = eng.logits(1).float().cpu().numpy()[0]
            errs.append(max_rel(g, ref[t]))
            errabs.append(float(np.abs(g - ref[t]).max()))
            margins.append(_top2_margin(ref[t]))
            assert np.all(np.isfinite(g)), f"step {t}: non-finite"
            assert errs[-1] <= MAXREL[act], f"step {t}: logits max-rel {errs[-1]:.3e}"
            if margins[-1] > 2 * errabs[-1]:
                assert int(np.argmax(g)) == ref_ids[t], f"step {t}: greedy id"
            if t + 1 < steps:
                eng.decode(torch.tensor([ref_ids[t]], dtype=torch.int32, device="cuda"), nxt)
        # free-running: the engine's own ids through the captured decode graphs
        # (four steps per graph launch, as the bench replays them), recorded
        # on the device by the id log
        eng.reset()
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), tok)
        id0 = int(tok.item())
        log = torch.full((steps - 1, 1), -1, dtype=torch.int32, device="cuda")
        eng.set_id_log(log)
        eng.decode_graph(tok, tok, steps - 1)
        eng.set_id_log(None)
        gpu_ids = [id0] + [int(v) for v in log[:, 0].cpu()]
    finally:
        eng.close()
    same = next((t for t in range(steps) if gpu_ids[t] != ref_ids[t]), steps)
    near = sum(1 for mg, ea in zip(margins, errabs) if mg <= 2 * ea)
    distinct = len(set(gpu_ids))
    print(f"config 3: identical greedy prefix {same}/{steps}; teacher-forced logits max-rel "
          f"max {max(errs):.2e}; smallest top-2 margin {min(margins):.3e}; "
          f"steps with a margin within twice the error: {near}; distinct ids {distinct}", flush=True)
    parity_record("config 3 130M free-running 256 (4-step graphs)", identical_prefix=f"{same}/{steps}",
                  distinct_ids=distinct, logits_maxrel_worst=round(max(errs), 6),
                  smallest_top2_margin=round(min(margins), 4), near_tie_steps=near)
    if same < steps:
        # the first divergence must be a near-tie the observed error can flip
        assert margins[same] <= 2 * errabs[same], \
            f"free-running ids diverge at step {same} with a clear margin {margins[same]:.3e}"
    assert same >= 200, f"identical greedy prefix only {same}/{steps}"
    assert distinct >= 32, f"the free-running ids repeat: {distinct} distinct in {steps}"


# --------------------------------------------------------------------------- configs 4 / 5, layer by layer
def _layer_check(om, trace, conv, ssd, B, L, decode, what, layers=None):
    """Run the oracle's run_block for every layer on the GPU's own input rows;
    compare each layer's output rows with the GPU's.  Returns the worst error."""
    n_layer = trace.shape[0] - 1
    worst = 0.0
    for li in (range(n_layer) if layers is None else layers):
        h = np.ascontiguousarray(trace[li])
        om.block(li, h, conv, ssd, B, L, decode)
        e = max_rel(O.from_act(h, om.act), O.from_act(trace[li + 1], om.act))
        worst = max(worst, e)
        assert e <= MAXREL[om.act], f"{what}: layer {li} output max-rel {e:.3e}"
    return worst


@pytest.fixture(scope="module")
def m2p7b(torch_cuda):
    from lite_ssm_amd.model import DeviceModel, shape
    print("building 2.7B-shaped model", flush=True)
    sh = shape("mamba2-2.7b")
    m = DeviceModel(sh, act=O.BF16, wfmt=O.W_Q4_G64, seed=5)
    om = O.Model(m.to_host(), vars(sh), O.BF16, O.W_Q4_G64)
    yield sh, m, om
    del m


@pytest.fixture(scope="module")
def m8b(torch_cuda):
    from lite_ssm_amd.model import DeviceModel, shape
    print("building 8B-shaped model", flush=True)
    sh = shape("mamba2-8b")
    m = DeviceModel(sh, act=O.BF16, wfmt=O.W_Q4_G64, seed=6)
    om = O.Model(m.to_host(), vars(sh), O.BF16, O.W_Q4_G64)
    yield sh, m, om
    del m


def _trace_buf(sh, rows):
    return torch.zeros((sh.n_layer + 1, rows, sh.d_model), dtype=torch.bfloat16, device="cuda")


def _prefill_layers(ctx, sh, m, om, B, Lq, seed, what):
    from lite_ssm_amd.model import Engine
    eng = Engine(ctx, m, B, Lq)
    try:
        tr = _trace_buf(sh, B * Lq)
        eng.set_trace(tr)
        ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=torch.Generator().manual_seed(seed),
                            dtype=torch.int32)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), nxt)
        trace = _bits(tr)
        lg = eng.logits(B).float().cpu().numpy()
        gconv, gssd = eng.state()
        conv, ssd = om.new_state(B)
        worst = _layer_check(om, trace, conv, ssd, B, Lq, False, what)
        # final state per layer, and logits of the GPU's last rows
        e_ssd = max_rel(gssd[:, :B].cpu().numpy(), ssd)
        assert e_ssd <= MAXREL[O.BF16], f"{what}: SSD state max-rel {e_ssd:.3e}"
        last = np.ascontiguousarray(trace[-1].reshape(B, Lq, -1)[:, -1])
        _check_ids(lg, O.from_act(om.logits(last), O.BF16), what + " logits")
        print(f"{what}: worst layer max-rel {worst:.2e}, state {e_ssd:.2e}", flush=True)
    finally:
        eng.close()


def _decode_layers(ctx, sh, m, om, batches, steps, what):
    """From a zero state, `steps` decode steps at each batch size, every layer
    of every step checked on the GPU's own input rows (the second step on runs
    with a nonzero state)."""
    from lite_ssm_amd.model import Engine
    eng = Engine(ctx, m, max(batches), 8)
    try:
        for B in batches:
            eng.reset()
            tr = _trace_buf(sh, B)
            eng.set_trace(tr)
            conv, ssd = om.new_state(B)
            rng = np.random.default_rng(B)
            nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
            worst = 0.0
            for step in range(steps):
                tok = rng.integers(0, sh.vocab_size, B).astype(np.int32)
                eng.decode(torch.from_numpy(tok).cuda(), nxt)
                trace = _bits(tr)
                worst = max(worst, _layer_check(om, trace, conv, ssd, B, 1, True, f"{what} b{B} s{step}"))
                lg = eng.logits(B).float().cpu().numpy()
                _check_ids(lg, O.from_act(om.logits(np.ascontiguousarray(trace[-1])), O.BF16),
                           f"{what} b{B} s{step} logits")
            gconv, gssd = eng.state()
            e_ssd = max_rel(gssd[:, :B].cpu().numpy(), ssd)
            assert e_ssd <= MAXREL[O.BF16], f"{what} b{B}: SSD state max-rel {e_ssd:.3e}"
            print(f"{what} decode b{B}: worst layer max-rel {worst:.2e}, state {e_ssd:.2e}", flush=True)
            eng.set_trace(None)
    finally:
        eng.close()


def test_config4_2p7b_prefill_layer_by_layer(ctx, m2p7b):
    sh, m, om = m2p7b
    print("case: config 4 prefill 2 x 80 tokens, 64 layers, vocab 50280", flush=True)
    _prefill_layers(ctx, sh, m, om, 2, 80, 41, "2.7B prefill")


def test_config4_2p7b_decode_layer_by_layer(ctx, m2p7b):
    sh, m, om = m2p7b
    print("case: config 4 decode at batch 1 / 4 / 16, 64 layers", flush=True)
    _decode_layers(ctx, sh, m, om, (1, 4, 16), 3, "2.7B")


def test_config5_8b_prefill_layer_by_layer(ctx, m8b):
    sh, m, om = m8b
    print("case: config 5 prefill 1 x 80 tokens, 56 layers, G 8, vocab 256000", flush=True)
    _prefill_layers(ctx, sh, m, om, 1, 80, 51, "8B prefill")


def test_config5_8b_decode_layer_by_layer(ctx, m8b):
    sh, m, om = m8b
    print("case: config 5 decode at batch 1 / 32, 56 layers", flush=True)
    _decode_layers(ctx, sh, m, om, (1, 32), 2, "8B")


# --------------------------------------------------------------------------- full-size prefills
def _full_prefill(ctx, sh, m, om, B, Lq, check_layers, what):
    from lite_ssm_amd.model import Engine
    eng = Engine(ctx, m, B, Lq)
    try:
        tr = _trace_buf(sh, B * Lq)
        eng.set_trace(tr)
        ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=torch.Generator().manual_seed(7),
                            dtype=torch.int32)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), nxt)
        lg = eng.logits(B).float().cpu().numpy()
        assert np.all(np.isfinite(lg)), f"{what}: non-finite logits"
        assert list(nxt.cpu().numpy()) == [int(np.argmax(r)) for r in lg]
        gconv, gssd = eng.state()
        # sequence 0 of the checked layers, on the whole sequence
        for li in check_layers:
            rows = _bits(tr[li].view(B, Lq, -1)[0])
            conv, ssd = om.new_state(1)
            h = np.ascontiguousarray(rows)
            om.block(li, h, conv, ssd, 1, Lq, False)
            e = max_rel(O.from_act(h, O.BF16), O.from_act(_bits(tr[li + 1].view(B, Lq, -1)[0]), O.BF16))
            es = max_rel(gssd[li, 0].cpu().numpy(), ssd[li, 0])
            print(f"{what}: layer {li} on {Lq} tokens: output max-rel {e:.2e}, SSD state {es:.2e}",
                  flush=True)
            assert e <= MAXREL[O.BF16], f"{what}: layer {li} output max-rel {e:.3e}"
            assert es <= MAXREL[O.BF16], f"{what}: layer {li} SSD state max-rel {es:.3e}"
        del tr
        eng.set_trace(None)
        # decode from the prefilled state: graph replay == eager, bit for bit
        conv0, ssd0 = eng.state()
        t_e = nxt.clone()
        for _ in range(3):
            eng.decode(t_e, t_e)
        ce, se = eng.state()
        lg_e = eng.logits(B)
        # restore the prefilled state, then the same steps through the graph
        import lite_ssm_amd as L
        import ctypes as C
        cp, sp = C.c_void_p(), C.c_void_p()
        L.check(L.lib.lssm_engine_state(eng.h, C.byref(cp), C.byref(sp)))
        L.check(L.lib.lssm_memcpy_d2d(ctx.h, cp.value, conv0.data_ptr(), conv0.numel() * conv0.element_size()))
        L.check(L.lib.lssm_memcpy_d2d(ctx.h, sp.value, ssd0.data_ptr(), ssd0.numel() * 4))
        t_g = nxt.clone()
        eng.decode_graph(t_g, t_g, 3)
        cg, sg = eng.state()
        assert torch.equal(t_g, t_e) and torch.equal(sg, se) and torch.equal(cg, ce)
        assert torch.equal(eng.logits(B), lg_e)
    finally:
        eng.close()


def test_config4_full_prefill_4x4096(ctx, m2p7b):
    sh, m, om = m2p7b
    print("case: config 4 full prefill 4 x 4096", flush=True)
    _full_prefill(ctx, sh, m, om, 4, 4096, (0, sh.n_layer - 1), "2.7B 4x4096")


def test_config5_full_prefill_8192(ctx, m8b):
    sh, m, om = m8b
    print("case: config 5 full prefill 1 x 8192", flush=True)
    _full_prefill(ctx, sh, m, om, 1, 8192, (sh.n_layer - 1,), "8B 8192")


def test_config5_prefill_split_in_time_full_depth(ctx, m8b, monkeypatch):
    """Config 5's prefill as the bench runs it: one 8192-token sequence in two
    halves in time on two streams (no trace buffer, which keeps one stream),
    against the same prefill on one stream, whose layers the test above checks
    against the oracle.  Over 56 layers of random weights any rounding-level
    difference grows (measured: the split, and the gated norm unfused -- the
    same arithmetic with other rounding points -- move the last layer's SSD
    state by 0.10 and 0.27 of its largest entry, the logits by 5e-2 and 8e-2,
    and both change the greedy id), so the split is held to the first two
    layers' states, where only the fp32 state carried between the halves
    rounds differently, and at every depth to at most twice what unfusing the
    gated norm moves."""
    from lite_ssm_amd.model import Engine
    sh, m, om = m8b
    ids = torch.randint(0, sh.vocab_size, (1, 8192), generator=torch.Generator().manual_seed(23),
                        dtype=torch.int32).cuda()
    out = {}
    for name, env in (("split", {"LSSM_SPLIT_PREFILL": "1"}), ("one", {"LSSM_SPLIT_PREFILL": "0"}),
                      ("gn", {"LSSM_SPLIT_PREFILL": "0", "LSSM_FUSED_GATED_NORM": "0"})):
        monkeypatch.delenv("LSSM_FUSED_GATED_NORM", raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        eng = Engine(ctx, m, 1, 8192)
        try:
            nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
            eng.prefill(ids, nxt)
            conv, ssd = eng.state()
            out[name] = (eng.logits(1).float().cpu().numpy(), int(nxt.item()), conv.float().cpu().numpy(),
                         ssd.cpu().numpy())
        finally:
            eng.close()
        print(f"case: 8B 1 x 8192 prefill ({name}) done", flush=True)
    lg0, id0, c0, s0 = out["one"]
    dev = {}
    for name in ("split", "gn"):
        lg, i, c, sd = out[name]
        assert np.all(np.isfinite(lg)) and i == int(np.argmax(lg[0])), name
        dev[name] = (max_rel(lg, lg0), [max_rel(c[l], c0[l]) for l in range(sh.n_layer)],
                     [max_rel(sd[l], s0[l]) for l in range(sh.n_layer)])
        print(f"case: 8B 1 x 8192 {name} against one stream: logits {dev[name][0]:.2e}, conv state max "
              f"{max(dev[name][1]):.2e}, SSD state max {max(dev[name][2]):.2e}, id {i} / {id0}", flush=True)
    (e_lg, e_c, e_s), (g_lg, g_c, g_s) = dev["split"], dev["gn"]
    assert max(e_c[:2]) <= 1e-3 and max(e_s[:2]) <= 1e-3, (e_c[:2], e_s[:2])
    assert max(e_c) <= 2 * max(g_c) and max(e_s) <= 2 * max(g_s)
    assert e_lg <= max(2 * g_lg, MAXREL[O.BF16])

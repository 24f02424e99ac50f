"""Decode parity over the BASELINE step counts, on the paths the bench times.

The reference's generation loop (runtime/inference.cpp:55-67) feeds each
greedy id (sampler.cpp:13-21, first maximum on ties) back as the next input.
These tests run that loop for hundreds of steps, where rounding differences
could accumulate in the fp32 SSM state, and compare with the CPU oracle:

 * 2.7B (config 4) at batch 1, 512 free-running steps after a 16-token
   prefill.  The engine runs them through lssm_engine_decode_graph with the
   four-step graphs and the fused in_proj + SSD launch (the bench's path), its
   ids recorded by lssm_engine_set_id_log.  The same 512 steps run eagerly
   must give the same ids, state and logits bit for bit, and their logits are
   kept at every step.  The oracle is then fed the engine's ids: its logits
   must agree at every step, and every step where its greedy id differs from
   the engine's must be a near-tie (the engine's id within twice the step's
   observed logit error of the oracle's maximum).  Since the oracle follows
   the engine's ids, the first such step is where an oracle run on its own
   ids would part from the engine's: the identical free-running prefix.
   The final conv and SSD states of all 64 layers are compared.
 * 2.7B at batch 16, 128 teacher-forced steps after an 8-token prefill:
   logits of all 16 sequences compared at every step (the normalise-on-load
   MFMA decode path), the final states, and graph replay equal to eager.
 * 8B (config 5) at batch 32, 32 teacher-forced steps after a 4-token
   prefill: likewise.

The 2.7B model's head is a permutation of its embedding rows
(DeviceModel(head="permuted")): a tied head with embeddings large enough for
clear top-2 margins predicts the input token again, so greedy decoding would
repeat one id; the permuted head makes it walk a long cycle instead.

Two kinds of comparison, with their own bounds:

 * per layer, from the engine's own state (LAYER_BOUND = 2e-2, the BASELINE
   north_star bar for bf16 outputs): at steps 128, 256 and 512 the engine's
   hidden rows entering every layer (lssm_engine_set_trace) and its conv /
   SSD state before the step go through the oracle's run_block
   (mamba2_block.cpp:51-290) one layer at a time; each layer's output rows and
   updated states must agree.  This is the parity bar of the step itself, at
   any depth into the run.
 * whole model: the oracle runs its own 64 (56) layers on the same ids from
   the start, so the two computations part by the compounding of bf16
   rounding differences over every layer and step.  The yardstick for that
   drift is a second oracle run whose linears sum in float32 instead of
   double (O.accum_f32; the reference's kernels sum in fp32 in their own
   order, so both runs restate it faithfully): the engine's whole-model drift
   in the logits (worst step) and in the final states must stay within
   DRIFT_FACTOR times the drift between the two oracle runs, or within the
   2e-2 bar where that is larger.

The figures go to the parity records (tests/conftest.py) printed at the end
of the run.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import MAXREL, max_rel

pytestmark = pytest.mark.gpu

LAYER_BOUND = MAXREL[O.BF16]
DRIFT_FACTOR = 3.0


def _drift_ok(engine, yard):
    return engine <= max(DRIFT_FACTOR * yard, LAYER_BOUND)


class _Oracles:
    """The oracle run twice in lockstep: double sums (the reference point)
    and float32 sums (the yardstick of whole-model drift)."""

    def __init__(self, om, B):
        self.om = om
        self.st = [om.new_state(B), om.new_state(B)]
        self.yard = []          # per step: max-rel of the float32 run against the double run

    def _both(self, fn):
        a = O.from_act(fn(*self.st[0]), self.om.act)
        with O.accum_f32():
            b = O.from_act(fn(*self.st[1]), self.om.act)
        self.yard.append(max_rel(b, a))
        return a

    def prefill(self, ids):
        return self._both(lambda c, s: self.om.prefill(c, s, ids))

    def decode(self, ids):
        return self._both(lambda c, s: self.om.decode(c, s, ids))

    def state_yard(self):
        """worst per-layer drift of the float32 run's final states."""
        (c0, s0), (c1, s1) = self.st
        act = self.om.act
        e_ssd = max(max_rel(s1[li], s0[li]) for li in range(self.om.n_layer))
        e_conv = max(max_rel(O.from_act(c1[li], act), O.from_act(c0[li], act)) for li in range(self.om.n_layer))
        return e_ssd, e_conv


def _bits(t):
    a = t.detach().cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        return a.view(torch.int16).numpy().view(np.uint16)
    return a.numpy()


def _top2(row):
    s = np.sort(row)[-2:]
    return float(s[1] - s[0])


def _state_errs(om, gconv, gssd, conv, ssd, B):
    """worst per-layer max-rel of the SSD and conv states."""
    act = om.act
    e_ssd = max(max_rel(gssd[li, :B].cpu().numpy(), ssd[li]) for li in range(om.n_layer))
    gc = _bits(gconv)
    e_conv = max(max_rel(O.from_act(gc[li, :B], act), O.from_act(conv[li], act))
                 for li in range(om.n_layer))
    return e_ssd, e_conv


def _layers_from_engine_state(om, trace, conv0, ssd0, conv1, ssd1, B, what):
    """One decode step, layer by layer, from the engine's own state: trace =
    hidden rows entering each layer and after the last ([n_layer + 1, B,
    d_model] bits); conv0 / ssd0 = the engine's state before the step, conv1 /
    ssd1 after it (host arrays [n_layer, B, ...]).  Returns the worst errors
    of (layer outputs, SSD states, conv states)."""
    act = om.act
    conv, ssd = conv0.copy(), ssd0.copy()
    wo = ws = wc = 0.0
    for li in range(om.n_layer):
        h = np.ascontiguousarray(trace[li])
        om.block(li, h, conv, ssd, B, 1, True)
        e = max_rel(O.from_act(h, act), O.from_act(trace[li + 1], act))
        es = max_rel(ssd1[li], ssd[li])
        ec = max_rel(O.from_act(conv1[li], act), O.from_act(conv[li], act))
        assert e <= LAYER_BOUND, f"{what}: layer {li} output max-rel {e:.3e}"
        assert es <= LAYER_BOUND, f"{what}: layer {li} SSD state max-rel {es:.3e}"
        assert ec <= LAYER_BOUND, f"{what}: layer {li} conv state max-rel {ec:.3e}"
        wo, ws, wc = max(wo, e), max(ws, es), max(wc, ec)
    return wo, ws, wc


def _host_state(eng, B):
    gconv, gssd = eng.state()
    return np.ascontiguousarray(_bits(gconv)[:, :B]), np.ascontiguousarray(gssd[:, :B].cpu().numpy())


@pytest.fixture(scope="module")
def m2p7b_walk(torch_cuda, progress):
    say = progress
    from lite_ssm_amd.model import DeviceModel, shape
    say("building 2.7B-shaped model (permuted head)")
    sh = shape("mamba2-2.7b")
    m = DeviceModel(sh, act=O.BF16, wfmt=O.W_Q4_G64, seed=21, embed_std=1.5, head="permuted")
    om = O.Model(m.to_host(), vars(sh), O.BF16, O.W_Q4_G64)
    yield sh, m, om
    del m


@pytest.mark.timeout(1200)
def test_decode_2p7b_bs1_512_free_running(ctx, m2p7b_walk, parity_record, progress):
    say = progress
    from lite_ssm_amd.model import Engine
    sh, m, om = m2p7b_walk
    Lp, steps, chunk = 16, 512, 128
    say(f"case: 2.7B batch 1, prefill {Lp}, {steps} free-running steps (4-step graphs)")
    prompt = torch.randint(0, sh.vocab_size, (1, Lp), generator=torch.Generator().manual_seed(77),
                           dtype=torch.int32)
    eng = Engine(ctx, m, 1, Lp)
    try:
        # the bench's path: graph replay, fused in_proj + SSD launch
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        eng.prefill(prompt.cuda(), tok)
        id0 = int(tok.item())
        log = torch.full((steps, 1), -1, dtype=torch.int32, device="cuda")
        eng.set_id_log(log)
        graph_lg = {}
        for c in range(chunk, steps + 1, chunk):
            eng.decode_graph(tok, tok, chunk)
            graph_lg[c] = eng.logits(1).float().cpu().numpy()[0]
        fused, _ = eng.fused_layers()
        g_ids = [id0] + [int(v) for v in log[:, 0].cpu()]
        gconv, gssd = eng.state()
        eng.set_id_log(None)
        say(f"graph run done: fused layers {fused}, ids[:8] {g_ids[:8]}")
        assert fused == sh.n_layer, "the fused in_proj + SSD launch did not run"
        assert min(g_ids) >= 0

        # the same steps eagerly: logits at every step, identical to the
        # graph's; at the checkpoints the hidden rows entering every layer and
        # the state before and after the step are kept
        eng.reset()
        eng.prefill(prompt.cuda(), tok)
        e_ids = [int(tok.item())]
        lg = [eng.logits(1).float().cpu().numpy()[0]]
        tr = torch.zeros((sh.n_layer + 1, 1, sh.d_model), dtype=torch.bfloat16, device="cuda")
        kept = {}
        for s in range(1, steps + 1):
            if s in graph_lg:
                before = _host_state(eng, 1)
                eng.set_trace(tr)
            eng.decode(tok, tok)
            if s in graph_lg:
                eng.set_trace(None)
                kept[s] = (_bits(tr).copy(), before, _host_state(eng, 1))
            e_ids.append(int(tok.item()))
            lg.append(eng.logits(1).float().cpu().numpy()[0])
        econv, essd = eng.state()
    finally:
        eng.close()
    assert e_ids == g_ids, "eager and graph-replayed decode chose different ids"
    assert torch.equal(essd, gssd) and torch.equal(econv, gconv), "eager and graph states differ"
    for c, g in graph_lg.items():
        assert np.array_equal(g, lg[c]), f"step {c}: graph and eager logits differ"

    # every layer of the checkpoint steps, from the engine's own state
    layer_errs = {}
    for c, (trace, (c0, s0), (c1, s1)) in kept.items():
        layer_errs[c] = [round(v, 5) for v in
                         _layers_from_engine_state(om, trace, c0, s0, c1, s1, 1, f"step {c}")]
        say(f"step {c}: worst layer output / SSD / conv max-rel {layer_errs[c]}")
    del kept

    # the whole model: the oracle's own 64 layers (twice), fed the engine's ids
    orc = _Oracles(om, 1)
    ref = orc.prefill(prompt.numpy())[0]
    errs, first, flips, margins = [], None, 0, []
    at = {}
    for s in range(steps + 1):
        if s > 0:
            ref = orc.decode(np.array([g_ids[s - 1]], np.int32))[0]
        g = lg[s]
        assert np.all(np.isfinite(g)), f"step {s}: non-finite logits"
        e = max_rel(g, ref)
        errs.append(e)
        if s in graph_lg or s % 32 == 0:
            at[s] = round(e, 5)
        margins.append(_top2(ref) / max(np.abs(ref).max(), 1e-30))
        r_id = int(np.argmax(ref))
        if r_id != g_ids[s]:
            gap = float(ref[r_id] - ref[g_ids[s]])
            err_abs = float(np.abs(g - ref).max())
            assert gap <= 2 * err_abs, \
                f"step {s}: engine id {g_ids[s]} is {gap:.3f} below the oracle's maximum (error {err_abs:.3f})"
            flips += 1
            if first is None:
                first = (s, gap, err_abs)
        if s % 32 == 0:
            say(f"oracle at step {s}: logits max-rel so far {max(errs):.2e} (oracle f32 against f64 "
                  f"{max(orc.yard):.2e}), flips {flips}")
    conv, ssd = orc.st[0]
    e_ssd, e_conv = _state_errs(om, gconv, gssd, conv, ssd, 1)
    y_ssd, y_conv = orc.state_yard()
    prefix = first[0] if first else steps + 1
    parity_record("2.7B bs1 free-running 512 (4-step graphs, fused launch)",
                  identical_prefix=f"{prefix}/{steps + 1}",
                  first_divergence=None if first is None else
                  dict(step=first[0], oracle_gap=round(first[1], 4), logit_err=round(first[2], 4)),
                  near_tie_flips=flips, distinct_ids=len(set(g_ids)),
                  layer_check_at=layer_errs,
                  model_logits_maxrel_worst=round(max(errs), 5), model_logits_maxrel_at=at,
                  model_ssd_state_maxrel=round(e_ssd, 5), model_conv_state_maxrel=round(e_conv, 5),
                  yardstick_logits_maxrel_worst=round(max(orc.yard), 5),
                  yardstick_ssd_state_maxrel=round(y_ssd, 5), yardstick_conv_state_maxrel=round(y_conv, 5),
                  smallest_top2_margin_rel=round(float(min(margins)), 5))
    assert _drift_ok(max(errs), max(orc.yard)), \
        f"whole-model logits drift {max(errs):.3e} against the oracles' {max(orc.yard):.3e}"
    assert _drift_ok(e_ssd, y_ssd), f"whole-model SSD state drift {e_ssd:.3e} against {y_ssd:.3e}"
    assert _drift_ok(e_conv, y_conv), f"whole-model conv state drift {e_conv:.3e} against {y_conv:.3e}"
    assert len(set(g_ids)) >= 64, f"only {len(set(g_ids))} distinct ids in {steps + 1} steps"


def _teacher_forced(ctx, sh, m, om, B, Lp, steps, seed, what, parity_record, say):
    """Prefill Lp tokens per sequence, then `steps` eager decode steps with
    given ids: whole-model logits of every sequence at every step; every layer
    at the middle and last steps from the engine's own state; then graph
    replay of free-running steps against eager, bit for bit."""
    from lite_ssm_amd.model import Engine
    gen = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, sh.vocab_size, (B, Lp), generator=gen, dtype=torch.int32)
    tf = torch.randint(0, sh.vocab_size, (steps, B), generator=gen, dtype=torch.int32)
    checks = (steps // 2, steps)
    eng = Engine(ctx, m, B, Lp)
    try:
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(prompt.cuda(), nxt)
        orc = _Oracles(om, B)
        ref = orc.prefill(prompt.numpy())
        g = eng.logits(B).float().cpu().numpy()
        errs = [max_rel(g, ref)]
        id_checked = id_same = 0
        tr = torch.zeros((sh.n_layer + 1, B, sh.d_model), dtype=torch.bfloat16, device="cuda")
        layer_errs = {}
        for s in range(1, steps + 1):
            if s in checks:
                before = _host_state(eng, B)
                eng.set_trace(tr)
            eng.decode(tf[s - 1].cuda(), nxt)
            if s in checks:
                eng.set_trace(None)
                c0, s0 = before
                c1, s1 = _host_state(eng, B)
                layer_errs[s] = [round(v, 5) for v in _layers_from_engine_state(
                    om, _bits(tr).copy(), c0, s0, c1, s1, B, f"{what} step {s}")]
                say(f"{what} step {s}: worst layer output / SSD / conv max-rel {layer_errs[s]}")
            g = eng.logits(B).float().cpu().numpy()
            ref = orc.decode(tf[s - 1].numpy())
            assert np.all(np.isfinite(g)), f"{what} step {s}: non-finite logits"
            e = max_rel(g, ref)
            errs.append(e)
            err = np.abs(g - ref).max(axis=-1)
            gid = nxt.cpu().numpy()
            for r in range(B):
                if _top2(ref[r]) > 2 * err[r]:
                    id_checked += 1
                    assert gid[r] == int(np.argmax(ref[r])), f"{what} step {s}: greedy id of row {r}"
                    id_same += 1
            if s % 4 == 0:
                say(f"{what}: step {s}, whole-model logits max-rel so far {max(errs):.2e} (oracle f32 "
                      f"against f64 {max(orc.yard):.2e})")
        gconv, gssd = eng.state()
        conv, ssd = orc.st[0]
        e_ssd, e_conv = _state_errs(om, gconv, gssd, conv, ssd, B)
        y_ssd, y_conv = orc.state_yard()

        # free-running from the same prefill: graph replay == eager, bit for bit
        free = min(steps, 32)
        eng.reset()
        eng.prefill(prompt.cuda(), nxt)
        e_ids = []
        for _ in range(free):
            eng.decode(nxt, nxt)
            e_ids.append(nxt.cpu().numpy().copy())
        ec, es_ = eng.state()
        elg = eng.logits(B)
        eng.reset()
        tok = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(prompt.cuda(), tok)
        log = torch.full((free, B), -1, dtype=torch.int32, device="cuda")
        eng.set_id_log(log)
        eng.decode_graph(tok, tok, free)
        eng.set_id_log(None)
        gc, gs = eng.state()
        assert np.array_equal(log.cpu().numpy(), np.stack(e_ids)), f"{what}: graph ids differ from eager"
        assert torch.equal(gs, es_) and torch.equal(gc, ec), f"{what}: graph state differs from eager"
        assert torch.equal(eng.logits(B), elg), f"{what}: graph logits differ from eager"
    finally:
        eng.close()
    parity_record(f"{what} teacher-forced {steps} steps", batch=B, prefill=Lp,
                  layer_check_at=layer_errs,
                  model_logits_maxrel_worst=round(max(errs), 5),
                  model_logits_maxrel_by_32=[round(max(errs[i:i + 32]), 5) for i in range(0, len(errs), 32)],
                  model_ssd_state_maxrel=round(e_ssd, 5), model_conv_state_maxrel=round(e_conv, 5),
                  yardstick_logits_maxrel_worst=round(max(orc.yard), 5),
                  yardstick_ssd_state_maxrel=round(y_ssd, 5), yardstick_conv_state_maxrel=round(y_conv, 5),
                  greedy_ids_checked=id_checked, greedy_ids_equal=id_same,
                  graph_eq_eager_steps=free)
    assert _drift_ok(max(errs), max(orc.yard)), \
        f"{what}: whole-model logits drift {max(errs):.3e} against the oracles' {max(orc.yard):.3e}"
    assert _drift_ok(e_ssd, y_ssd), f"{what}: whole-model SSD state drift {e_ssd:.3e} against {y_ssd:.3e}"
    assert _drift_ok(e_conv, y_conv), f"{what}: whole-model conv state drift {e_conv:.3e} against {y_conv:.3e}"


@pytest.mark.timeout(1200)
def test_decode_2p7b_bs16_128_teacher_forced(ctx, m2p7b_walk, parity_record, progress):
    say = progress
    sh, m, om = m2p7b_walk
    say("case: 2.7B batch 16, prefill 8, 128 teacher-forced steps")
    _teacher_forced(ctx, sh, m, om, 16, 8, 128, 81, "2.7B bs16", parity_record, say)


@pytest.fixture(scope="module")
def m8b_long(torch_cuda, progress):
    say = progress
    from lite_ssm_amd.model import DeviceModel, shape
    say("building 8B-shaped model")
    sh = shape("mamba2-8b")
    m = DeviceModel(sh, act=O.BF16, wfmt=O.W_Q4_G64, seed=31)
    om = O.Model(m.to_host(), vars(sh), O.BF16, O.W_Q4_G64)
    say("8B-shaped model built on the device and in the oracle")
    yield sh, m, om
    del m


@pytest.mark.timeout(1200)
def test_decode_8b_bs32_32_teacher_forced(ctx, m8b_long, parity_record, progress):
    say = progress
    sh, m, om = m8b_long
    say("case: 8B batch 32, prefill 4, 32 teacher-forced steps")
    _teacher_forced(ctx, sh, m, om, 32, 4, 32, 91, "8B bs32", parity_record, say)

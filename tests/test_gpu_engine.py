"""Whole-model parity: the engine (fused decode kernels, MFMA prefill, HIP
graph replay) against the oracle's restatement of Mamba2Model::run_block
(mamba2_block.cpp:51-327) on the same random-init weights and token ids.

Decode is teacher-forced: both sides are fed the oracle's greedy token, so a
near-tie flip cannot make the sequences diverge; every step's logits are
compared (max-rel 2e-2 for fp16 / bf16, 1e-3 for fp32), and the greedy ids
must agree wherever the oracle's top-2 margin exceeds the comparison bound.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import MAXREL, max_rel

pytestmark = pytest.mark.gpu


def _setup(ctx, name, act, wfmt, seed=11, **over):
    import lite_ssm_amd as L
    from lite_ssm_amd.model import DeviceModel, shape
    sh = shape(name, **over)
    m = DeviceModel(sh, act=act, wfmt=wfmt, seed=seed)
    om = O.Model(m.to_host(), vars(sh), act, wfmt)
    return L, sh, m, om


def _check_logits(gpu, ref_bits, act, what):
    ref = O.from_act(ref_bits, act)
    e = max_rel(gpu, ref)
    assert np.all(np.isfinite(gpu)), what
    assert e <= MAXREL[act], f"{what}: logits max-rel {e:.3e}"
    # greedy ids agree wherever the top-2 margin is clear of the error bound
    for r in range(ref.shape[0]):
        top2 = np.sort(ref[r])[-2:]
        if top2[1] - top2[0] > 4 * e * np.abs(ref).max():
            assert int(np.argmax(gpu[r])) == int(np.argmax(ref[r])), f"{what}: greedy id row {r}"
    return e


CASES = [
    ("f16-q8g32", O.F16, O.W_Q8_G32),     # config 3 formats
    ("bf16-q4g64", O.BF16, O.W_Q4_G64),   # configs 4/5 formats
    ("f16-q4b32", O.F16, O.W_Q4_B32),     # the reference's INT4_B32
    ("f16-dense", O.F16, O.W_DENSE),      # the reference's fp16 checkpoints
    ("f32-dense", O.F32, O.W_DENSE),
]


@pytest.mark.parametrize("tag,act,wfmt", CASES, ids=[c[0] for c in CASES])
def test_engine_prefill_then_decode_vs_oracle(ctx, tag, act, wfmt):
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-130m", act, wfmt, n_layer=2, vocab_size=2048)
    B, Lq = 2, 100
    eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=g, dtype=torch.int32)
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(ids.cuda(), nxt)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids.numpy())
    _check_logits(eng.logits(B).float().cpu().numpy(), ref, act, f"{tag} prefill")
    # the engine's greedy ids are the argmax of its own logits
    assert list(nxt.cpu().numpy()) == list(np.argmax(eng.logits(B).float().cpu().numpy(), -1))
    gconv, gssd = eng.state()
    assert max_rel(gssd.cpu().numpy(), ssd) < MAXREL[act]
    tok = O.argmax(ref, act)
    for step in range(3):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, act, f"{tag} decode {step}")
        tok = O.argmax(ref, act)
    eng.close()


def test_engine_graph_replay_matches_eager(ctx):
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-130m", O.BF16, O.W_Q4_G64, n_layer=3, vocab_size=1024)
    eng = Engine(ctx, m, max_batch=1, max_seq=64)
    ids = torch.randint(0, sh.vocab_size, (1, 64), dtype=torch.int32).cuda()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    eng.prefill(ids, tok)
    conv0, ssd0 = eng.state()
    # eager: 11 steps feeding back the engine's own greedy ids
    t_e = tok.clone()
    eager = []
    for _ in range(11):
        eng.decode(t_e, t_e)
        eager.append(int(t_e.item()))
    conv_e, ssd_e = eng.state()
    lg_e = eng.logits(1)
    # graph: restore the post-prefill state, replay 5 steps one call at a
    # time, then 6 in one call (launches of the unrolled graph of 4 steps by
    # default and of the one-step graph); then, from the start again, 11 + 11
    # steps against 11 more eager steps
    eng.reset()
    eng.prefill(ids, tok)
    t_g = tok.clone()
    graph = []
    for _ in range(5):
        eng.decode_graph(t_g, t_g, 1)
        graph.append(int(t_g.item()))
    eng.decode_graph(t_g, t_g, 6)
    graph.append(int(t_g.item()))
    eager = eager[:5] + [eager[-1]]
    conv_g, ssd_g = eng.state()
    assert graph == eager
    assert torch.equal(ssd_g, ssd_e) and torch.equal(conv_g, conv_e)
    assert torch.equal(eng.logits(1), lg_e)
    for _ in range(11):
        eng.decode(t_e, t_e)
    conv_e, ssd_e = eng.state()
    lg_e = eng.logits(1)
    eng.reset()
    eng.prefill(ids, tok)
    t_g = tok.clone()
    eng.decode_graph(t_g, t_g, 11)
    eng.decode_graph(t_g, t_g, 11)
    conv_g, ssd_g = eng.state()
    assert torch.equal(t_g, t_e)
    assert torch.equal(ssd_g, ssd_e) and torch.equal(conv_g, conv_e)
    assert torch.equal(eng.logits(1), lg_e)
    eng.close()


def test_engine_batched_graph_and_stale_rows(ctx):
    """Batched decode on the normalise-on-load path (int4-g64 bf16, 3 layers):
    graph replay is bit-identical to eager steps, and a batch of 5 decoded after
    a batch of 8 (whose rows 5..15 of the packed-x and partial-sum buffers then
    hold stale values the GEMVs read and drop) gives the bits a fresh engine
    gives."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=3, vocab_size=1024, seed=31)
    g = torch.Generator().manual_seed(9)
    ids8 = torch.randint(0, sh.vocab_size, (8, 24), generator=g, dtype=torch.int32).cuda()
    ids5 = torch.randint(0, sh.vocab_size, (5, 24), generator=g, dtype=torch.int32).cuda()

    def run5(eng):
        tok = torch.zeros(5, dtype=torch.int32, device="cuda")
        eng.prefill(ids5, tok)
        for _ in range(3):
            eng.decode(tok, tok)
        return eng.logits(5), tok.clone()

    fresh = Engine(ctx, m, max_batch=8, max_seq=24)
    try:
        lg_fresh, tok_fresh = run5(fresh)
    finally:
        fresh.close()
    eng = Engine(ctx, m, max_batch=8, max_seq=24)
    try:
        tok = torch.zeros(8, dtype=torch.int32, device="cuda")
        eng.prefill(ids8, tok)
        t_e = tok.clone()
        for _ in range(4):
            eng.decode(t_e, t_e)
        conv_e, ssd_e = eng.state()
        conv_e, ssd_e = conv_e.clone(), ssd_e.clone()
        lg_e = eng.logits(8)
        eng.reset()
        eng.prefill(ids8, tok)
        t_g = tok.clone()
        eng.decode_graph(t_g, t_g, 4)
        conv_g, ssd_g = eng.state()
        assert torch.equal(t_g, t_e)
        assert torch.equal(ssd_g, ssd_e) and torch.equal(conv_g, conv_e)
        assert torch.equal(eng.logits(8), lg_e)
        eng.reset()
        lg5, tok5 = run5(eng)
        assert torch.equal(tok5, tok_fresh)
        assert torch.equal(lg5, lg_fresh), "batch-5 logits depend on the earlier batch-8 rows"
    finally:
        eng.close()


def test_engine_batch8_decode(ctx):
    """Batch 8: prefill on the MFMA GEMMs, decode on the MFMA GEMV (exact
    dequantization, as the oracle's and the reference's decode)."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-130m", O.BF16, O.W_Q4_G64, n_layer=2, vocab_size=1024)
    B = 8
    eng = Engine(ctx, m, max_batch=B, max_seq=70)
    ids = np.random.default_rng(2).integers(0, sh.vocab_size, (B, 70)).astype(np.int32)
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(torch.from_numpy(ids).cuda(), nxt)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids)
    _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, "b8 prefill")
    tok = O.argmax(ref, O.BF16)
    for step in range(2):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, f"b8 decode {step}")
        tok = O.argmax(ref, O.BF16)
    eng.close()


PACK_CASES = [("f16-q8g32", O.F16, O.W_Q8_G32), ("f16-q4b32", O.F16, O.W_Q4_B32),
              ("bf16-q4g64", O.BF16, O.W_Q4_G64), ("f16-dense", O.F16, O.W_DENSE)]


@pytest.mark.parametrize("B", [8, 24, 32])
@pytest.mark.parametrize("tag,act,wfmt", PACK_CASES, ids=[c[0] for c in PACK_CASES])
def test_engine_batch8_packed_staging(ctx, tag, act, wfmt, B):
    """Decode batches from 8 rows take the packing pass (x normalised and
    packed once per linear) and the single-pass MFMA GEMV, which reads the
    packed rows straight from memory: 8 and 24/32 rows (one and two tiles of
    16 batch rows), for every format the MFMA GEMV takes; against the
    oracle's per-sequence decode."""
    from lite_ssm_amd.model import Engine
    print(f"case: packed decode {tag} batch {B}", flush=True)
    L, sh, m, om = _setup(ctx, "mamba2-130m", act, wfmt, n_layer=2, vocab_size=1024, seed=17)
    eng = Engine(ctx, m, max_batch=B, max_seq=40)
    try:
        ids = np.random.default_rng(3).integers(0, sh.vocab_size, (B, 40)).astype(np.int32)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(torch.from_numpy(ids).cuda(), nxt)
        conv, ssd = om.new_state(B)
        ref = om.prefill(conv, ssd, ids)
        tok = O.argmax(ref, act)
        for step in range(3):
            eng.decode(torch.from_numpy(tok).cuda(), nxt)
            ref = om.decode(conv, ssd, tok)
            _check_logits(eng.logits(B).float().cpu().numpy(), ref, act, f"{tag} b{B} decode {step}")
            tok = O.argmax(ref, act)
    finally:
        eng.close()


@pytest.mark.parametrize("B", [8, 24])
def test_engine_8b_widths_packed_decode(ctx, B):
    """8B layer widths (d_model 4096, in_proj 18560 rows, G 8) at decode batches
    8 and 24: the packing pass and the single-pass MFMA GEMV with five 16-row
    tiles per block (in_proj) at one and two tiles of batch rows, and the
    K 8192 out_proj; against the oracle's per-sequence decode."""
    from lite_ssm_amd.model import Engine
    print(f"case: 8B widths, packed decode batch {B}", flush=True)
    L, sh, m, om = _setup(ctx, "mamba2-8b", O.BF16, O.W_Q4_G64, n_layer=1, vocab_size=512, seed=23)
    Lq = 8
    eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
    try:
        ids = np.random.default_rng(5).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(torch.from_numpy(ids).cuda(), nxt)
        conv, ssd = om.new_state(B)
        ref = om.prefill(conv, ssd, ids)
        tok = O.argmax(ref, O.BF16)
        for step in range(2):
            eng.decode(torch.from_numpy(tok).cuda(), nxt)
            ref = om.decode(conv, ssd, tok)
            _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, f"8B widths b{B} decode {step}")
            tok = O.argmax(ref, O.BF16)
    finally:
        eng.close()


@pytest.mark.parametrize("name,B", [("mamba2-2.7b", 3), ("mamba2-2.7b", 4), ("mamba2-2.7b", 8),
                                    ("mamba2-2.7b", 17), ("mamba2-2.7b", 24), ("mamba2-2.7b", 32),
                                    ("mamba2-8b", 16)])
def test_engine_normalise_on_load_decode(ctx, monkeypatch, name, B):
    """Packed decode batches without the pack launches between layers: out_proj
    writes r(h w) (w: the next layer's norm weight) in the single-pass GEMV's
    fragment order with its rows' partial sums of squares of h, the SSD step
    r(y w') likewise, and the next linear scales its fp32 sums by the rows'
    1 / rms.  Three engines on the same weights and ids: LSSM_NOPACK=0 (a pack
    launch of r(x w / rms) before each linear), =2 (a pack launch of r(x w)
    with one partial a row: the GEMV's scaling alone) and the default (the
    producers).  Every mode against the oracle's per-sequence decode; and the
    hidden rows after each layer of the first decode step, where modes 1 and 2
    feed the GEMVs the same r(x w) values and differ only in the order the
    sums of squares are added (fp32 rounding of 1 / rms), must be bit-identical
    in nearly every element: a lost, doubled or misplaced partial scales whole
    rows and changes most of them."""
    from lite_ssm_amd.model import Engine
    print(f"case: normalise on load, {name} batch {B}", flush=True)
    L, sh, m, om = _setup(ctx, name, O.BF16, O.W_Q4_G64, n_layer=3, vocab_size=512, seed=29)
    Lq = 8
    ids = np.random.default_rng(7).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
    conv, ssd = om.new_state(B)
    refs = [om.prefill(conv, ssd, ids)]
    toks = [O.argmax(refs[0], O.BF16)]
    for step in range(3):
        refs.append(om.decode(conv, ssd, toks[-1]))
        toks.append(O.argmax(refs[-1], O.BF16))
    logits, traces = {}, {}
    for mode in ("0", "2", "1"):
        monkeypatch.setenv("LSSM_NOPACK", mode)
        eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
        try:
            nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
            eng.prefill(torch.from_numpy(ids).cuda(), nxt)
            tr = torch.zeros((sh.n_layer + 1) * B * sh.d_model, dtype=torch.bfloat16, device="cuda")
            out = []
            for step in range(3):
                eng.set_trace(tr if step == 0 else None)
                eng.decode(torch.from_numpy(toks[step]).cuda(), nxt)
                out.append(eng.logits(B).float().cpu().numpy())
            logits[mode] = out
            traces[mode] = tr.view(torch.int16).cpu().numpy().reshape(sh.n_layer + 1, B, sh.d_model)
        finally:
            eng.close()
    for mode in ("0", "2", "1"):
        for step in range(3):
            _check_logits(logits[mode][step], refs[step + 1], O.BF16, f"{name} b{B} mode {mode} decode {step}")
    # (measured: 1.0000 after the first layer, >= 0.993 after the second,
    # >= 0.93 after the third, where single-ulp flips have spread)
    for li in range(1, sh.n_layer + 1):
        same = float(np.mean(traces["1"][li] == traces["2"][li]))
        print(f"hidden rows after layer {li - 1}: {same:.4f} of elements equal (modes 1, 2)", flush=True)
        bound = 0.99 if li <= 2 else 0.9
        assert same >= bound, f"layer {li - 1}: only {same:.4f} of the hidden elements match the raw-pack path"


def test_engine_prefill_folded_norms(ctx, monkeypatch):
    """Both RMSNorms of a prefill layer folded into their neighbours: out_proj's
    epilogue writes the next layer's r(h w) with sums of h^2 per 128 columns
    and the next in_proj scales its fp32 sums by 1 / rms; the chunked scan's Y
    stores hold the gated norm's r(g w) with sums of g^2 and out_proj scales
    by that 1 / rms.  Full-width 2.7B layers at 1600 rows (7 row tiles: the
    out_proj GEMM runs unsplit, so the fold is taken): every layer against the
    oracle's run_block on the engine's own input rows, and against an engine
    with both folds off (LSSM_FOLD_PRE_NORM=0, LSSM_FUSED_GATED_NORM=0), which
    must differ (the folds ran) but stay within the bound."""
    from lite_ssm_amd.model import Engine
    print("case: folded prefill norms, 2.7B widths, 3 layers, 1 x 1600", flush=True)
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=3, vocab_size=512, seed=37)
    B, Lq = 1, 1600
    ids = np.random.default_rng(9).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
    traces = {}
    for mode in ("off", "on"):
        v = "0" if mode == "off" else "1"
        monkeypatch.setenv("LSSM_FOLD_PRE_NORM", v)
        monkeypatch.setenv("LSSM_FUSED_GATED_NORM", v)
        eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
        try:
            tr = torch.zeros((sh.n_layer + 1, B * Lq, sh.d_model), dtype=torch.bfloat16, device="cuda")
            eng.set_trace(tr)
            nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
            eng.prefill(torch.from_numpy(ids).cuda(), nxt)
            eng.set_trace(None)
            traces[mode] = tr.view(torch.int16).cpu().numpy()
        finally:
            eng.close()
    on, off = traces["on"], traces["off"]
    assert np.array_equal(on[0], off[0]), "the embedding rows differ"
    conv, ssd = om.new_state(B)
    for li in range(sh.n_layer):
        h = np.ascontiguousarray(on[li])
        om.block(li, h, conv, ssd, B, Lq, False)
        e = max_rel(O.from_act(h, O.BF16), O.from_act(on[li + 1], O.BF16))
        d = max_rel(O.from_act(on[li + 1], O.BF16), O.from_act(off[li + 1], O.BF16))
        same = float(np.mean(on[li + 1] == off[li + 1]))
        print(f"layer {li}: folded against the oracle {e:.2e}, against unfolded {d:.2e} "
              f"({same:.3f} of elements equal)", flush=True)
        assert e <= MAXREL[O.BF16], f"layer {li}: output max-rel {e:.3e} against the oracle"
        assert d <= MAXREL[O.BF16], f"layer {li}: folded and unfolded differ by {d:.3e}"
    assert not np.array_equal(on[2], off[2]), "the second layer's rows are bit-identical: no fold ran"


@pytest.mark.parametrize("name,act,wfmt,vocab", [
    ("mamba2-130m", O.BF16, O.W_Q4_G64, 50280),
    ("mamba2-130m", O.F16, O.W_Q8_G32, 50280),
    ("mamba2-8b", O.BF16, O.W_Q4_G64, 256000),      # config 5's lm_head: K 4096, 256000 rows
], ids=["130m-bf16", "130m-f16", "8b-bf16"])
def test_engine_lm_head_argmax_fused(ctx, monkeypatch, name, act, wfmt, vocab):
    """Batch 1: the lm_head launch that also reduces each block's rows to
    (max, first index) plus one final reduction, against the two-pass argmax
    over the stored logits (LSSM_FUSED_ARGMAX=0), at the real vocabulary (one
    partial per block of a grid of about one block per CU).  The lm_head
    repeats every row four times (rows 2k, 2k + 1, V/2 + 2k, V/2 + 2k + 1), so
    the maximum is always a tie inside one block and across blocks, and the
    first-index rule (sampler.cpp:13-21) must pick the even row below V/2."""
    from lite_ssm_amd.model import DeviceModel, Engine, shape
    sh = shape(name, n_layer=1 if name == "mamba2-8b" else 2, vocab_size=vocab)
    m = DeviceModel(sh, act=act, wfmt=wfmt, seed=11)
    V, half = sh.vocab_size, sh.vocab_size // 2
    m.lm_head = m.lm_head.clone()
    m.lm_head[half:2 * half] = m.lm_head[:half]
    m.lm_head[1:half:2] = m.lm_head[0:half - 1:2]
    m.lm_head[half + 1:2 * half:2] = m.lm_head[half:2 * half - 1:2]
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, V, (1, 40), generator=g, dtype=torch.int32).cuda()

    def run(fused):
        monkeypatch.setenv("LSSM_FUSED_ARGMAX", "1" if fused else "0")
        eng = Engine(ctx, m, max_batch=1, max_seq=64)
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        out, lgs = [], []
        eng.prefill(ids, tok)
        out.append(int(tok.item()))
        lgs.append(eng.logits(1))
        for _ in range(6):                       # eager, feeding back its own ids
            eng.decode(tok, tok)
            out.append(int(tok.item()))
            lgs.append(eng.logits(1))
        for _ in range(2):                       # graph replay: 1 + 4 + 1 steps, then 5
            eng.decode_graph(tok, tok, 6)
            out.append(int(tok.item()))
            lgs.append(eng.logits(1))
        eng.close()
        return out, lgs

    ids_f, lg_f = run(True)
    ids_p, lg_p = run(False)
    assert ids_f == ids_p
    for a, b in zip(lg_f, lg_p):
        assert torch.equal(a, b)
    print(f"case: {name} vocab {V}: ids {ids_f}", flush=True)
    for i, lg in zip(ids_f, lg_f):
        h = lg.float().cpu().numpy()[0]
        assert i == int(np.argmax(h))            # first index of the maximum
        assert i < half and i % 2 == 0, i
        assert h[i] == h[i + 1] == h[half + i] == h[half + i + 1]


def test_engine_prefill_split_two_streams(ctx, monkeypatch):
    """A prefill of 4 x 2048 tokens (8192 rows) runs as two halves of two
    sequences, the second on the engine's own stream: logits, greedy ids and
    the final conv / SSD state against the oracle, as with one stream
    (LSSM_SPLIT_PREFILL=0); then two teacher-forced decode steps from the
    split prefill's state."""
    from lite_ssm_amd.model import Engine
    act, wfmt = O.BF16, O.W_Q4_G64
    L, sh, m, om = _setup(ctx, "mamba2-130m", act, wfmt, n_layer=2, vocab_size=1024)
    B, Lq = 4, 2048
    g = torch.Generator().manual_seed(13)
    ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=g, dtype=torch.int32)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids.numpy())
    engines = {}
    for split in ("1", "0"):
        monkeypatch.setenv("LSSM_SPLIT_PREFILL", split)
        eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), nxt)
        lg = eng.logits(B).float().cpu().numpy()
        _check_logits(lg, ref, act, f"prefill split={split}")
        assert list(nxt.cpu().numpy()) == list(np.argmax(lg, -1))
        gconv, gssd = eng.state()
        es, ec = max_rel(gssd.cpu().numpy(), ssd), max_rel(gconv.float().cpu().numpy(), O.from_act(conv, act))
        print(f"case: split={split}: SSD state max-rel {es:.4f}, conv state {ec:.4f}", flush=True)
        # the second layer's state after 2048 tokens: its input carries the
        # first layer's rounding, and the segmented scan (fewer walks than CUs
        # in both forms) carries its state across segment boundaries in fp32
        # where the reference rounds it after every chunk
        assert es < 3e-2, f"split={split}: SSD state"
        assert ec < MAXREL[act], f"split={split}: conv state"
        engines[split] = eng
    engines["0"].close()
    eng = engines["1"]
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    tok = O.argmax(ref, act)
    for step in range(2):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, act, f"decode {step} after the split prefill")
        tok = O.argmax(ref, act)
    eng.close()


def test_engine_prefill_split_in_time(ctx, monkeypatch):
    """One sequence of 8192 tokens runs as two halves in time: tokens 4096 ..
    on the engine's own stream, each layer continuing from the SSD state and
    conv window the first half left (the conv reads its first rows' history
    from the conv state).  Logits, greedy id and final conv / SSD state
    against the oracle, as with one stream (LSSM_SPLIT_PREFILL=0); then two
    teacher-forced decode steps from the split prefill's state."""
    from lite_ssm_amd.model import Engine
    act, wfmt = O.BF16, O.W_Q4_G64
    L, sh, m, om = _setup(ctx, "mamba2-130m", act, wfmt, n_layer=2, vocab_size=1024)
    B, Lq = 1, 8192
    g = torch.Generator().manual_seed(17)
    ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=g, dtype=torch.int32)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids.numpy())
    engines = {}
    for split in ("1", "0"):
        monkeypatch.setenv("LSSM_SPLIT_PREFILL", split)
        eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
        nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
        eng.prefill(ids.cuda(), nxt)
        lg = eng.logits(B).float().cpu().numpy()
        _check_logits(lg, ref, act, f"prefill split={split}")
        assert list(nxt.cpu().numpy()) == list(np.argmax(lg, -1))
        gconv, gssd = eng.state()
        es, ec = max_rel(gssd.cpu().numpy(), ssd), max_rel(gconv.float().cpu().numpy(), O.from_act(conv, act))
        print(f"case: split={split}: SSD state max-rel {es:.4f}, conv state {ec:.4f}", flush=True)
        # as in the batch split test: the second layer's state after many
        # tokens, through the segmented scan's fp32 segment boundaries
        assert es < 3e-2, f"split={split}: SSD state"
        assert ec < MAXREL[act], f"split={split}: conv state"
        engines[split] = eng
    engines["0"].close()
    eng = engines["1"]
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    tok = O.argmax(ref, act)
    for step in range(2):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, act, f"decode {step} after the split prefill")
        tok = O.argmax(ref, act)
    eng.close()


def test_engine_one_token_prefill(ctx):
    """L == 1 prefill takes the reference's GEMV / conv-update / SSD-step path
    and seeds the conv state (mamba2_block.cpp:111-116, 155-162, 183-195, 285-289)."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-130m", O.F16, O.W_Q4_B32, n_layer=2, vocab_size=1024)
    eng = Engine(ctx, m, max_batch=1, max_seq=8)
    nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
    eng.prefill(torch.tensor([[17]], dtype=torch.int32).cuda(), nxt)
    conv, ssd = om.new_state(1)
    ref = om.prefill(conv, ssd, np.array([[17]], np.int32))
    _check_logits(eng.logits(1).float().cpu().numpy(), ref, O.F16, "L1 prefill")
    gconv, _ = eng.state()
    g = gconv.cpu().view(torch.int16).numpy().view(np.uint16)
    # the seeded window after one token: older taps exactly zero, the newest
    # tap the token's xBC value (a rounded fp32 sum: the f16 bound, not bits)
    assert np.array_equal(g[..., :-1], conv[..., :-1])
    e = max_rel(O.from_act(np.ascontiguousarray(g[..., -1]), O.F16),
                O.from_act(np.ascontiguousarray(conv[..., -1]), O.F16))
    assert e <= 2e-3, f"seeded conv state max-rel {e:.3e}"
    eng.close()


def test_engine_2p7b_layer_shapes(ctx):
    """Full-width Mamba-2-2.7B layers (d_model 2560, 80 heads, int4 group-64,
    bf16): 2 layers, reduced vocab, prefill 130 tokens at batch 2 + 2 decode steps."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=2, vocab_size=512)
    B, Lq = 2, 130
    eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
    ids = np.random.default_rng(3).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(torch.from_numpy(ids).cuda(), nxt)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids)
    _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, "2.7b prefill")
    tok = O.argmax(ref, O.BF16)
    for step in range(2):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, f"2.7b decode {step}")
        tok = O.argmax(ref, O.BF16)
    eng.close()


@pytest.mark.parametrize("B", [16, 5, 40])
def test_engine_2p7b_batched_decode(ctx, B):
    """Full-width 2.7B layers decoding B sequences at once on the MFMA GEMV
    (in_proj: 3 tiles per block; out_proj: K 5120; 40 rows: past the
    single-pass kernel's 32, the staged kernel with a pack launch before each
    linear), against the oracle's per-sequence GEMV-rule decode."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=1, vocab_size=512, seed=13)
    Lq = 8
    eng = Engine(ctx, m, max_batch=B, max_seq=Lq + 3)
    ids = np.random.default_rng(6).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(torch.from_numpy(ids).cuda(), nxt)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids)
    tok = O.argmax(ref, O.BF16)
    for step in range(3):
        eng.decode(torch.from_numpy(tok).cuda(), nxt)
        ref = om.decode(conv, ssd, tok)
        _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, f"2.7b b{B} decode {step}")
        tok = O.argmax(ref, O.BF16)
    eng.close()


def test_engine_8b_groups(ctx):
    """Mamba-2-8B layer shapes (d_model 4096, 128 heads, 8 groups), 1 layer."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-8b", O.BF16, O.W_Q4_G64, n_layer=1, vocab_size=512)
    B, Lq = 1, 80
    eng = Engine(ctx, m, max_batch=B, max_seq=Lq)
    ids = np.random.default_rng(4).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(torch.from_numpy(ids).cuda(), nxt)
    conv, ssd = om.new_state(B)
    ref = om.prefill(conv, ssd, ids)
    _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, "8b prefill")
    tok = O.argmax(ref, O.BF16)
    eng.decode(torch.from_numpy(tok).cuda(), nxt)
    ref = om.decode(conv, ssd, tok)
    _check_logits(eng.logits(B).float().cpu().numpy(), ref, O.BF16, "8b decode")
    eng.close()


def test_engine_argument_errors(ctx):
    import lite_ssm_amd as L
    from lite_ssm_amd.model import Engine
    _, sh, m, _ = _setup(ctx, "mamba2-130m", O.F16, O.W_Q8_G32, n_layer=1, vocab_size=256)
    eng = Engine(ctx, m, max_batch=1, max_seq=8)
    nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(L.LssmError, match="exceeds workspace max_seq_len"):
        eng.prefill(torch.zeros(1, 9, dtype=torch.int32, device="cuda"), nxt)
    with pytest.raises(L.LssmError, match="batch out of range"):
        eng.decode(torch.zeros(2, dtype=torch.int32, device="cuda"), nxt)
    eng.close()


FUSED_CASES = [
    # tag, shape, act, wfmt, overrides, whole mixer in one launch
    ("2.7b-bf16-q4g64", "mamba2-2.7b", O.BF16, O.W_Q4_G64, dict(n_layer=2, vocab_size=512), True),
    ("130m-f16-q8g32", "mamba2-130m", O.F16, O.W_Q8_G32, dict(n_layer=2, vocab_size=1024), True),
    # a (d_model, d_inner) the one-launch mixer is not built for: SSD fused only
    ("1536-bf16-q4g64", "mamba2-130m", O.BF16, O.W_Q4_G64,
     dict(n_layer=2, vocab_size=1024, d_model=1536, n_heads=48), False),
]


@pytest.mark.parametrize("tag,name,act,wfmt,over,mixer", FUSED_CASES, ids=[c[0] for c in FUSED_CASES])
def test_engine_fused_ssd_decode_bs1(ctx, tag, name, act, wfmt, over, mixer):
    """Batch-1 decode with the SSD step (and, where built, out_proj) inside the
    in_proj launch (tagged words read across CUs): bit-identical to the
    three-launch decode (LSSM_FUSED_SSD=0) on every step, eager and
    graph-replayed (the step tag advances inside the graph), and within
    tolerance of the oracle."""
    import os
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, name, act, wfmt, **over)
    Lq = 40
    os.environ["LSSM_FUSED_MIXER"] = "1"
    os.environ["LSSM_FUSED_SSD"] = "1"
    try:
        fused = Engine(ctx, m, max_batch=1, max_seq=Lq)
    finally:
        del os.environ["LSSM_FUSED_MIXER"]
        del os.environ["LSSM_FUSED_SSD"]
    os.environ["LSSM_FUSED_SSD"] = "0"
    try:
        plain = Engine(ctx, m, max_batch=1, max_seq=Lq)
    finally:
        del os.environ["LSSM_FUSED_SSD"]
    try:
        _fused_vs_plain(tag, sh, om, act, fused, plain, Lq, (sh.n_layer, sh.n_layer if mixer else 0))
    finally:
        fused.close()
        plain.close()


def test_engine_fused_ssd_decode_batched(ctx, monkeypatch):
    """Decode batches of 3..16 (the normalise-on-load path) with the SSD step
    inside the single-pass MFMA in_proj launch (tagged words per row):
    bit-identical to the separate SSD step launch (LSSM_FUSED_SSD_B=0) in
    logits, conv and SSD state and the ids, on every step, eager and
    graph-replayed, with the batch changing between calls (stale words of
    larger batches must not be taken); within tolerance of the oracle.  Batch
    2 takes the VALU GEMV and is not fused."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=2, vocab_size=512, seed=41)
    Lq, BMAX = 6, 16
    monkeypatch.setenv("LSSM_FUSED_SSD_B", "1")
    fused = Engine(ctx, m, max_batch=BMAX, max_seq=Lq)
    monkeypatch.setenv("LSSM_FUSED_SSD_B", "0")
    plain = Engine(ctx, m, max_batch=BMAX, max_seq=Lq)
    try:
        for B in (16, 4, 3, 2, 8):
            print(f"case: batched fused SSD, batch {B}", flush=True)
            ids = np.random.default_rng(B).integers(0, sh.vocab_size, (B, Lq)).astype(np.int32)
            n_f = torch.zeros(B, dtype=torch.int32, device="cuda")
            n_p = torch.zeros_like(n_f)
            fused.reset()
            plain.reset()
            fused.prefill(torch.from_numpy(ids).cuda(), n_f)
            plain.prefill(torch.from_numpy(ids).cuda(), n_p)
            conv, ssd = om.new_state(B)
            ref = om.prefill(conv, ssd, ids)
            tok = O.argmax(ref, O.BF16)

            def same(step):
                assert torch.equal(fused.logits(B), plain.logits(B)), f"batch {B} logits, step {step}"
                cf, sf = fused.state()
                cp, sp = plain.state()
                assert torch.equal(sf[:, :B], sp[:, :B]) and torch.equal(cf[:, :B], cp[:, :B]), \
                    f"batch {B} state, step {step}"

            want = (sh.n_layer, 0) if B >= 3 else (0, 0)
            for step in range(3):
                t = torch.from_numpy(tok).cuda()
                fused.decode(t, n_f)
                plain.decode(t, n_p)
                assert fused.fused_layers() == want and plain.fused_layers() == (0, 0), f"batch {B}"
                same(step)
                ref = om.decode(conv, ssd, tok)
                _check_logits(fused.logits(B).float().cpu().numpy(), ref, O.BF16, f"batch {B} decode {step}")
                tok = O.argmax(ref, O.BF16)
            t_f = torch.from_numpy(tok).cuda()
            t_p = t_f.clone()
            fused.decode_graph(t_f, t_f, 5)
            for _ in range(5):
                plain.decode(t_p, t_p)
            assert torch.equal(t_f, t_p), f"batch {B} graph ids"
            same("graph")
    finally:
        fused.close()
        plain.close()


def test_engine_default_bs1_fuses_ssd_only(ctx):
    """The default batch-1 decode runs the SSD step inside the in_proj launch
    and out_proj as its own launch (LSSM_FUSED_MIXER unset), bit-identical to
    the three-launch decode."""
    import os
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-2.7b", O.BF16, O.W_Q4_G64, n_layer=2, vocab_size=512)
    Lq = 20
    fused = Engine(ctx, m, max_batch=1, max_seq=Lq)
    os.environ["LSSM_FUSED_SSD"] = "0"
    try:
        plain = Engine(ctx, m, max_batch=1, max_seq=Lq)
    finally:
        del os.environ["LSSM_FUSED_SSD"]
    try:
        _fused_vs_plain("2.7b default", sh, om, O.BF16, fused, plain, Lq, (sh.n_layer, 0))
    finally:
        fused.close()
        plain.close()


def test_engine_default_bs1_small_model_three_launches(ctx):
    """A model whose SSD step has work items for fewer than half the CUs (the
    130M shape: 24 heads x 64 rows = 48 items of 32 rows) decodes batch 1 in
    three launches per layer by default, within tolerance of the oracle."""
    from lite_ssm_amd.model import Engine
    L, sh, m, om = _setup(ctx, "mamba2-130m", O.F16, O.W_Q8_G32, n_layer=2, vocab_size=1024)
    eng = Engine(ctx, m, max_batch=1, max_seq=16)
    try:
        ids = np.random.default_rng(3).integers(0, sh.vocab_size, (1, 16)).astype(np.int32)
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        eng.prefill(torch.from_numpy(ids).cuda(), nxt)
        conv, ssd = om.new_state(1)
        ref = om.prefill(conv, ssd, ids)
        tok = O.argmax(ref, O.F16)
        for step in range(2):
            eng.decode(torch.from_numpy(tok).cuda(), nxt)
            assert eng.fused_layers() == (0, 0)
            ref = om.decode(conv, ssd, tok)
            _check_logits(eng.logits(1).float().cpu().numpy(), ref, O.F16, f"130m default decode {step}")
            tok = O.argmax(ref, O.F16)
    finally:
        eng.close()


def _fused_vs_plain(tag, sh, om, act, fused, plain, Lq, counts):
    ids = np.random.default_rng(7).integers(0, sh.vocab_size, (1, Lq)).astype(np.int32)
    n_f = torch.zeros(1, dtype=torch.int32, device="cuda")
    n_p = torch.zeros_like(n_f)
    fused.prefill(torch.from_numpy(ids).cuda(), n_f)
    plain.prefill(torch.from_numpy(ids).cuda(), n_p)
    conv, ssd = om.new_state(1)
    ref = om.prefill(conv, ssd, ids)
    tok = O.argmax(ref, act)

    def same(step):
        assert torch.equal(fused.logits(1), plain.logits(1)), f"{tag} logits, step {step}"
        cf, sf = fused.state()
        cp, sp = plain.state()
        assert torch.equal(sf, sp) and torch.equal(cf, cp), f"{tag} state, step {step}"

    for step in range(4):
        t = torch.from_numpy(tok).cuda()
        fused.decode(t, n_f)
        plain.decode(t, n_p)
        assert fused.fused_layers() == counts and plain.fused_layers() == (0, 0)
        same(step)
        ref = om.decode(conv, ssd, tok)
        _check_logits(fused.logits(1).float().cpu().numpy(), ref, act, f"{tag} decode {step}")
        tok = O.argmax(ref, act)
    t_f = torch.from_numpy(tok).cuda()
    t_p = t_f.clone()
    fused.decode_graph(t_f, t_f, 6)
    for _ in range(6):
        plain.decode(t_p, t_p)
    assert fused.fused_layers() == counts
    assert torch.equal(t_f, t_p)
    same("graph")

"""The drop-in check: the reference's own host code (src/core/{allocator,
ssm_loader}.cpp, src/model/*.cpp, src/runtime/{inference,sampler}.cpp, compiled
unchanged into oracle/_ref/libref_host.so against include/lite_ssm/*.hpp) runs
greedy generation on this HIP backend (tests/cpp/_bin/ref_model_run).

The reference's model layer only knows fp16 activations with fp16 or INT4_B32
weights (mamba2_block.cpp:97-129), so those are the cases.  Its logits at every
generated step are compared with the C oracle teacher-forced by the reference's
own ids, and with this repository's engine on the same file and ids.  Prompts
of 40 tokens take the chunked scan; 12 tokens with fp16 weights take the
reference's fused short-prefill branch (mamba2_block.cpp:97-98,130-148).
"""
import json
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import max_rel

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_bin", "ref_model_run")
BOUND = 2e-2          # fp16 logits, max-rel

CASES = [("q4b32-L40", O.W_Q4_B32, 40), ("q4b32-L12", O.W_Q4_B32, 12),
         ("dense-L40", O.W_DENSE, 40), ("dense-L12", O.W_DENSE, 12)]


def _margin_ok(ref_row, err_abs):
    top2 = np.sort(ref_row)[-2:]
    return top2[1] - top2[0] > 2 * err_abs


@pytest.mark.parametrize("tag,wfmt,L", CASES, ids=[c[0] for c in CASES])
def test_reference_model_layer_on_this_backend(ctx, tmp_path, tag, wfmt, L):
    from lite_ssm_amd.model import shape
    _ref_case(ctx, tmp_path, tag, shape("mamba2-130m", n_layer=4, vocab_size=4096), wfmt, L)


# The larger BASELINE widths in the reference's quantized format: the headline
# model's (d_model 2560, 80 heads) at 4 layers with the chunked scan and at all
# 64 (a 167 MB SSM state in one DeviceBuffer, 1.4 GB of weights) with a short
# prompt; the 8B's (d_model 4096, 128 heads, 8 groups of B / C) at 4 layers.
CASES_WIDE = [("2p7b-4layers-L40", "mamba2-2.7b", 4, 40), ("2p7b-64layers-L12", "mamba2-2.7b", 64, 12),
              ("8b-4layers-L40", "mamba2-8b", 4, 40)]


@pytest.mark.parametrize("tag,name,n_layer,L", CASES_WIDE, ids=[c[0] for c in CASES_WIDE])
def test_reference_model_layer_wide(ctx, tmp_path, tag, name, n_layer, L):
    from lite_ssm_amd.model import shape
    _ref_case(ctx, tmp_path, tag, shape(name, n_layer=n_layer, vocab_size=4096), O.W_Q4_B32, L)


def _ref_case(ctx, tmp_path, tag, sh, wfmt, L):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import Engine
    if not os.path.exists(EXE):
        pytest.skip("tests/cpp/_bin/ref_model_run not built (needs the reference checkout at build time)")
    print(f"case: reference model layer {tag}", flush=True)
    p = tmp_path / "m.ssm"
    S.write_random(p, sh, O.F16, wfmt, seed=17)
    n_new = 8
    prompt = np.random.default_rng(5).integers(0, sh.vocab_size, L).astype(np.int32)
    lpath = tmp_path / "logits.bin"
    r = subprocess.run([EXE, str(p), str(n_new), str(lpath), ",".join(str(int(t)) for t in prompt)],
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stdout + r.stderr
    ids = json.loads(r.stdout.strip().splitlines()[-1])["ids"]
    assert len(ids) == n_new
    ref_lg = np.fromfile(lpath, np.float32).reshape(n_new, sh.vocab_size)
    assert np.all(np.isfinite(ref_lg))
    # the reference picks the first maximum of its own logits (sampler.cpp:13-21)
    assert ids == [int(np.argmax(row)) for row in ref_lg]

    with S.SSMFile(p) as f:
        fm = f.model(ctx)
        om = O.Model(fm.to_host(), vars(fm.shape), O.F16, wfmt)
        conv, ssd = om.new_state(1)
        eng = Engine(ctx, fm, 1, L)
        try:
            nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
            orc = O.from_act(om.prefill(conv, ssd, prompt[None, :]), O.F16)
            eng.prefill(torch.from_numpy(prompt[None, :]).cuda(), nxt)
            for step in range(n_new):
                gpu = eng.logits(1).float().cpu().numpy()
                e_orc = max_rel(ref_lg[step], orc[0])
                e_eng = max_rel(gpu[0], ref_lg[step])
                print(f"{tag} step {step}: ref-vs-oracle {e_orc:.2e}, engine-vs-ref {e_eng:.2e}, "
                      f"id {ids[step]}", flush=True)
                assert e_orc <= BOUND, f"{tag} step {step}: reference vs oracle {e_orc:.3e}"
                assert e_eng <= BOUND, f"{tag} step {step}: engine vs reference {e_eng:.3e}"
                err_abs = np.abs(ref_lg[step] - orc[0]).max()
                if _margin_ok(orc[0], err_abs):
                    assert ids[step] == int(np.argmax(orc[0])), f"{tag} step {step}: greedy id"
                tok = np.array([ids[step]], np.int32)                 # teacher-forced by the reference
                orc = O.from_act(om.decode(conv, ssd, tok), O.F16)
                eng.decode(torch.from_numpy(tok).cuda(), nxt)
        finally:
            eng.close()

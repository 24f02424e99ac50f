""".ssm files on the GPU: the HBM upload is a byte-exact copy of the file, an
engine built from an uploaded file computes bit-identically to one built from
the same tensors already in HBM, and a random-initialised file runs through the
engine within the parity bar of the oracle (which reads the file's tensors on
the host).  The reference's path: SSMFile (ssm_loader.cpp) -> UnifiedBuffer
(metal_buffer.mm:37-67) -> Mamba2Model (mamba2_model.cpp:62-116)."""
import time

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import MAXREL, max_rel

pytestmark = pytest.mark.gpu


def _engine_run(eng, ids, B, steps):
    """prefill + `steps` greedy decode steps; returns logits of every step and ids."""
    nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
    eng.prefill(ids.cuda(), nxt)
    outs, toks = [eng.logits(B).clone()], [nxt.clone()]
    for _ in range(steps):
        eng.decode(nxt.clone(), nxt)
        outs.append(eng.logits(B).clone())
        toks.append(nxt.clone())
    return outs, toks


def test_upload_is_an_exact_copy(ctx, tmp_path):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import shape
    print("case: upload copy 130m-shaped 2 layers", flush=True)
    p = tmp_path / "r.ssm"
    S.write_random(p, shape("mamba2-130m", n_layer=2, vocab_size=2048), O.BF16, O.W_Q4_G64, 3)
    with S.SSMFile(p) as f:
        base = f.upload(ctx)
        assert f.upload(ctx) == base                  # uploaded once
        size = f.header.file_size
        back = torch.empty(size, dtype=torch.uint8, device="cuda")
        import lite_ssm_amd as L
        L.check(L.lib.lssm_memcpy_d2d(ctx.h, back.data_ptr(), base, size))
        torch.cuda.synchronize()
        assert back.cpu().numpy().tobytes() == open(p, "rb").read()


CASES = [("bf16-q4g64", O.BF16, O.W_Q4_G64, False), ("f16-q8g32", O.F16, O.W_Q8_G32, False),
         ("f16-q4b32-lm_head", O.F16, O.W_Q4_B32, True), ("f16-dense", O.F16, O.W_DENSE, False)]


@pytest.mark.parametrize("tag,act,wfmt,lm_head", CASES, ids=[c[0] for c in CASES])
def test_engine_from_file_matches_device_model(ctx, tmp_path, tag, act, wfmt, lm_head):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import DeviceModel, Engine, shape
    print(f"case: engine from file vs device model {tag}", flush=True)
    sh = shape("mamba2-130m", n_layer=2, vocab_size=2048)
    m = DeviceModel(sh, act=act, wfmt=wfmt, seed=21)
    p = tmp_path / "m.ssm"
    S.write_device_model(p, m, lm_head=lm_head)
    B, Lq = 2, 64
    ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=torch.Generator().manual_seed(4),
                        dtype=torch.int32)
    with S.SSMFile(p) as f:
        fm = f.model(ctx)
        assert (fm.act, fm.wfmt) == (act, wfmt)
        assert (fm.lm_head != fm.embed) == lm_head
        ea, eb = Engine(ctx, m, B, Lq), Engine(ctx, fm, B, Lq)
        try:
            la, ta = _engine_run(ea, ids, B, 3)
            lb, tb = _engine_run(eb, ids, B, 3)
            for s, (x, y) in enumerate(zip(la, lb)):
                assert torch.equal(x, y), f"{tag}: logits differ at step {s}"
            for x, y in zip(ta, tb):
                assert torch.equal(x, y)
        finally:
            ea.close()
            eb.close()


def test_engine_from_random_file_vs_oracle(ctx, tmp_path):
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import Engine, shape
    print("case: random file through the engine vs oracle", flush=True)
    act, wfmt = O.BF16, O.W_Q4_G64
    sh = shape("mamba2-130m", n_layer=2, vocab_size=2048)
    p = tmp_path / "r.ssm"
    S.write_random(p, sh, act, wfmt, seed=9)
    with S.SSMFile(p) as f:
        fm = f.model(ctx)
        om = O.Model(fm.to_host(), vars(fm.shape), act, wfmt)
        B, Lq = 2, 80
        ids = torch.randint(0, sh.vocab_size, (B, Lq), generator=torch.Generator().manual_seed(6),
                            dtype=torch.int32)
        eng = Engine(ctx, fm, B, Lq)
        try:
            nxt = torch.zeros(B, dtype=torch.int32, device="cuda")
            eng.prefill(ids.cuda(), nxt)
            conv, ssd = om.new_state(B)
            ref = om.prefill(conv, ssd, ids.numpy())
            for step in range(4):
                g = eng.logits(B).float().cpu().numpy()
                r = O.from_act(ref, act)
                assert np.all(np.isfinite(g))
                e = max_rel(g, r)
                assert e <= MAXREL[act], f"step {step}: logits max-rel {e:.3e}"
                tok = O.argmax(ref, act)             # teacher-forced by the oracle's ids
                eng.decode(torch.from_numpy(tok).cuda(), nxt)
                ref = om.decode(conv, ssd, tok)
        finally:
            eng.close()


def test_upload_rate_2p7b_layers(ctx, tmp_path):
    """Upload of a 2.7B-shaped file (16 of 64 layers, ~0.6 GB): checks the copy's
    first and last bytes and prints the host-to-HBM rate."""
    from lite_ssm_amd import ssm as S
    from lite_ssm_amd.model import shape
    print("case: upload rate 2.7b-shaped 16 layers", flush=True)
    p = tmp_path / "big.ssm"
    S.write_random(p, shape("mamba2-2.7b", n_layer=16), O.BF16, O.W_Q4_G64, 1)
    with S.SSMFile(p) as f:
        size = f.header.file_size
        t0 = time.perf_counter()
        base = f.upload(ctx)
        dt = time.perf_counter() - t0
        print(f"upload {size / 1e9:.3f} GB in {dt * 1e3:.1f} ms = {size / dt / 1e9:.1f} GB/s", flush=True)
        import lite_ssm_amd as L
        n = 1 << 20
        for off in (0, size - n):
            back = torch.empty(n, dtype=torch.uint8, device="cuda")
            L.check(L.lib.lssm_memcpy_d2d(ctx.h, back.data_ptr(), base + off, n))
            torch.cuda.synchronize()
            with open(p, "rb") as fh:
                fh.seek(off)
                assert back.cpu().numpy().tobytes() == fh.read(n)

"""lssm_inproj_ssd_decode_noalloc: the fused batch-1 in_proj + conv + SSD step
launch with its tagged words in the library's static device array instead of a
caller workspace.  Checked bit for bit against lssm_inproj_ssd_decode (same
kernels, same arithmetic) on the same inputs: conv state, SSD state and the
gated output, over calls in a row of different sizes (the second smaller, the
third the first shape again, so words of an earlier call sit in the array with
an older tag)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev

pytestmark = pytest.mark.gpu

SHAPES = [  # d_model, d_inner, N, G, H, act, wfmt
    (2560, 5120, 128, 1, 80, O.BF16, O.W_Q4_G64),   # 2.7B
    (768, 1536, 128, 1, 24, O.F16, O.W_Q8_G32),     # 130M (smaller)
    (2560, 5120, 128, 1, 80, O.BF16, O.W_Q4_G64),
]


def _case(rng, d_model, d_inner, N, G, H, act, wfmt):
    P, K = d_inner // H, 4
    xbc = d_inner + 2 * G * N
    proj = d_inner + xbc + H
    w, s = O.quantize((rng.standard_normal((proj, d_model)) * 0.02).astype(np.float32), wfmt)
    c = dict(
        nw=O.to_act(1 + 0.1 * rng.standard_normal(d_model), act), w=w, s=s,
        cw=O.to_act(rng.standard_normal((xbc, K)) * 0.3, act),
        cb=O.to_act(rng.standard_normal(xbc) * 0.1, act),
        dtb=O.to_act(rng.standard_normal(H) * 0.5, act),
        alog=O.to_act(rng.uniform(0, np.log(16), H), act),
        D=O.to_act(rng.standard_normal(H), act),
        cs=O.to_act(rng.standard_normal((1, xbc, K)), act),
        st=(rng.standard_normal((H, P, N)) * 0.1).astype(np.float32),
        hid=O.to_act(rng.standard_normal((1, d_model)) * 0.5, act))
    return c, (P, K, proj)


def test_noalloc_matches_workspace_entry(ctx):
    import lite_ssm_amd as L
    rng = np.random.default_rng(77)
    xfer = torch.zeros(1 << 16, dtype=torch.int64, device="cuda")
    tag = 0
    for i, (d_model, d_inner, N, G, H, act, wfmt) in enumerate(SHAPES):
        print(f"case: noalloc call {i}: d_model {d_model} d_inner {d_inner} H {H}", flush=True)
        c, (P, K, proj) = _case(rng, d_model, d_inner, N, G, H, act, wfmt)
        t = {k: dev(v) for k, v in c.items()}
        cs_a, cs_b = t["cs"].clone(), t["cs"].clone()
        st_a, st_b = t["st"].clone(), t["st"].clone()
        y_a = torch.zeros(d_inner, dtype=torch.int16, device="cuda")
        y_b = torch.zeros(d_inner, dtype=torch.int16, device="cuda")
        common = (t["hid"].data_ptr(), t["nw"].data_ptr(), t["w"].data_ptr(), t["s"].data_ptr())
        tag += 1
        L.check(L.lib.lssm_inproj_ssd_decode(
            ctx.h, *common, cs_a.data_ptr(), t["cw"].data_ptr(), t["cb"].data_ptr(), t["dtb"].data_ptr(),
            t["alog"].data_ptr(), t["D"].data_ptr(), st_a.data_ptr(), y_a.data_ptr(), xfer.data_ptr(), tag,
            d_model, d_inner, N, G, H, P, K, 1e-5, wfmt, act))
        L.check(L.lib.lssm_inproj_ssd_decode_noalloc(
            ctx.h, *common, cs_b.data_ptr(), t["cw"].data_ptr(), t["cb"].data_ptr(), t["dtb"].data_ptr(),
            t["alog"].data_ptr(), t["D"].data_ptr(), st_b.data_ptr(), y_b.data_ptr(),
            d_model, d_inner, N, G, H, P, K, 1e-5, wfmt, act))
        torch.cuda.synchronize()
        assert torch.equal(cs_a, cs_b), f"call {i}: conv state"
        assert torch.equal(st_a, st_b), f"call {i}: SSD state"
        assert torch.equal(y_a, y_b), f"call {i}: gated output"
        assert not torch.equal(st_b, t["st"]), f"call {i}: the state advanced"


def test_noalloc_refuses_oversized_shapes(ctx):
    import lite_ssm_amd as L
    p = torch.zeros(16, dtype=torch.int64, device="cuda").data_ptr()
    # d_inner 65536: the projection rows exceed the static array; nothing runs
    rc = L.lib.lssm_inproj_ssd_decode_noalloc(ctx.h, p, p, p, p, p, p, p, p, p, p, p, p, 4096, 65536, 128, 1,
                                              1024, 64, 4, 1e-5, O.W_Q4_G64, O.BF16)
    assert rc == 1
    assert "static scratch" in L.lib.lssm_last_error().decode()

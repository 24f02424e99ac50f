"""Helpers shared by the GPU parity tests: numpy <-> device tensors (bit exact)
and the tolerance checks of the parity bar.

Tolerances: integer dequantization bit-exact; fp32
scan / GEMM outputs within max-rel 1e-3; fp16 / bf16 outputs within max-rel
2e-2.  "max-rel" = max |gpu - ref| / max |ref| over the tensor.  Tighter
per-op bounds are used where the arithmetic allows.
"""
import numpy as np
import torch

import oracle as O

MAXREL = {O.F16: 2e-2, O.BF16: 2e-2, O.F32: 1e-3}


# Device copies made by dev() stay referenced until the end of the test (the
# conftest fixture clears this list), so `dev(a).data_ptr()` can be passed
# straight to a C entry point without the allocator reusing the block.
KEEP = []


def dev(a: np.ndarray) -> torch.Tensor:
    """Device copy with identical bits (uint16 carried as int16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    t = torch.from_numpy(a.copy()).cuda()
    KEEP.append(t)
    return t


def host(t: torch.Tensor, dtype) -> np.ndarray:
    torch.cuda.synchronize()
    a = t.detach().cpu().numpy()
    return a.view(dtype) if a.dtype != dtype else a


def empty(shape, act_or_dtype):
    if act_or_dtype in (O.F16, O.BF16):
        return torch.zeros(shape, dtype=torch.int16, device="cuda")
    if act_or_dtype == O.F32:
        return torch.zeros(shape, dtype=torch.float32, device="cuda")
    return torch.zeros(shape, dtype=act_or_dtype, device="cuda")


def act_host(t, act):
    return host(t, O.act_np_dtype(act))


def max_rel(gpu, ref):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(gpu - ref).max() / den)


def assert_close(gpu_bits, ref_bits, act, bound=None, what=""):
    g = O.from_act(gpu_bits, act)
    r = O.from_act(ref_bits, act)
    assert np.all(np.isfinite(g)), f"{what}: non-finite GPU output"
    b = MAXREL[act] if bound is None else bound
    e = max_rel(g, r)
    assert e <= b, f"{what}: max-rel {e:.3e} > {b:.1e}"
    return e


def ulp_diff16(a_bits, b_bits):
    """Distance in units-in-the-last-place between fp16 (or bf16) bit patterns."""
    def ordered(x):
        x = np.asarray(x).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(ordered(a_bits) - ordered(b_bits))

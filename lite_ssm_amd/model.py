"""Model shapes, random-init weights in HBM, and the whole-model engine wrapper.

Weights follow the .ssm tensor set of a Mamba-2 checkpoint
(src/model/mamba2_model.cpp:62-116): per layer norm, in_proj (rows
[z | xBC | dt]), conv1d weight/bias, dt_bias, A_log, D, mixer norm, out_proj;
plus embeddings, norm_f and a tied lm_head.  Only in_proj / out_proj are
quantized, as the reference exporter does (tools/export_mamba2.py:55-65).

The quantizer here runs on the device with torch and follows
tools/export_mamba2.py:68-103: fp32 per-group absmax (clamped at 1e-12) / qmax,
q = round-half-even(w / scale_fp32) clamped to [qmin, qmax], scale stored fp16,
int4 nibbles packed low = even k.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import torch

from . import (BF16, F16, F32, W_DENSE, W_Q4_B32, W_Q4_G64, W_Q8_G32, LayerWeights, ModelConfig,
               check, lib)

SHAPES = {
    # BASELINE configs 3-5; vocab 50280 as the configs state (the real 130M
    # export is padded to 50288, tests/test_mmap_loader.cpp:69)
    "mamba2-130m": dict(d_model=768, n_layer=24, d_state=128, d_conv=4, expand=2,
                        vocab_size=50280, n_heads=24, d_head=64, chunk_size=256, n_groups=1),
    "mamba2-2.7b": dict(d_model=2560, n_layer=64, d_state=128, d_conv=4, expand=2,
                        vocab_size=50280, n_heads=80, d_head=64, chunk_size=256, n_groups=1),
    "mamba2-8b": dict(d_model=4096, n_layer=56, d_state=128, d_conv=4, expand=2,
                      vocab_size=256000, n_heads=128, d_head=64, chunk_size=256, n_groups=8),
}

TORCH_DTYPE = {F16: torch.float16, BF16: torch.bfloat16, F32: torch.float32}
GROUP = {W_Q4_B32: 32, W_Q4_G64: 64, W_Q8_G32: 32}


@dataclass
class Shape:
    d_model: int
    n_layer: int
    d_state: int
    d_conv: int
    expand: int
    vocab_size: int
    n_heads: int
    d_head: int
    chunk_size: int
    n_groups: int

    @property
    def d_inner(self):
        return self.expand * self.d_model

    @property
    def xbc(self):
        return self.d_inner + 2 * self.n_groups * self.d_state

    @property
    def proj(self):
        return self.d_inner + self.xbc + self.n_heads

    def linear_params(self):
        """in_proj + out_proj parameters per layer."""
        return self.proj * self.d_model + self.d_model * self.d_inner


def shape(name: str, **over) -> Shape:
    d = dict(SHAPES[name])
    d.update(over)
    return Shape(**d)


def quantize(w: torch.Tensor, wfmt: int):
    """w [N, K] float -> (packed uint8 [N, K/2 | K], fp16 scales [N, K/G])."""
    N, K = w.shape
    G = GROUP[wfmt]
    is8 = wfmt == W_Q8_G32
    qmax, qmin = (127.0, -128.0) if is8 else (7.0, -8.0)
    blocks = w.float().reshape(N, K // G, G)
    amax = blocks.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
    scale = amax / qmax
    q = torch.round(blocks / scale).clamp(qmin, qmax).to(torch.int8).reshape(N, K)
    scales = scale.reshape(N, K // G).to(torch.float16)
    if is8:
        packed = q.view(torch.uint8)
    else:
        pairs = q.reshape(N, K // 2, 2)
        lo = (pairs[..., 0] & 0x0F).to(torch.uint8)
        hi = (pairs[..., 1] & 0x0F).to(torch.uint8)
        packed = (hi << 4) | lo
    return packed.contiguous(), scales.contiguous()


def dequantize(packed: torch.Tensor, scales: torch.Tensor, wfmt: int) -> torch.Tensor:
    """Exact fp32 dequantization (float(q) * float(scale))."""
    N = packed.shape[0]
    G = GROUP[wfmt]
    if wfmt == W_Q8_G32:
        q = packed.view(torch.int8).float()
    else:
        b = packed.to(torch.int16)
        lo = b & 0x0F
        hi = (b >> 4) & 0x0F
        q = torch.stack([lo, hi], dim=-1).reshape(N, -1)
        q = torch.where(q >= 8, q - 16, q).float()
    K = q.shape[1]
    return (q.reshape(N, K // G, G) * scales.float().reshape(N, K // G, 1)).reshape(N, K)


class DeviceModel:
    """Random-init Mamba-2 weights resident in HBM (one GPU)."""

    def __init__(self, sh: Shape, act: int = BF16, wfmt: int = W_Q4_G64, seed: int = 0,
                 device: str = "cuda", std: float = 0.02, embed_std: float | None = None,
                 head: str = "tied"):
        """Random init: linears ~ N(0, std), embeddings ~ N(0, embed_std or std).

        head = "tied": lm_head is the embedding (mamba2_model.cpp:75-83).
        head = "permuted": lm_head row pi(j) is embedding row j, for a random
        permutation pi.  With a large embed_std the residual stream keeps the
        input token's embedding, so a tied head mostly predicts the input token
        again (greedy decoding repeats one id); the permuted head predicts
        pi(input) instead, and greedy decoding walks a long cycle of pi, with
        top-2 margins that the layers' outputs move but rarely close."""
        self.shape, self.act, self.wfmt, self.device = sh, act, wfmt, device
        dt = TORCH_DTYPE[act]
        g = torch.Generator(device=device)
        g.manual_seed(seed)

        def randn(*s, scale=1.0, mean=0.0):
            return torch.randn(*s, generator=g, device=device, dtype=torch.float32) * scale + mean

        def act_t(x):
            return x.to(dt).contiguous()

        def lin(N, K):
            # the exporter's input is the fp16 checkpoint tensor
            w = randn(N, K, scale=std).to(torch.float16).float()
            if wfmt == W_DENSE:
                return act_t(w), None
            return quantize(w, wfmt)

        H = sh.n_heads
        self.embed = act_t(randn(sh.vocab_size, sh.d_model, scale=std if embed_std is None else embed_std))
        self.norm_f = act_t(randn(sh.d_model, scale=0.1, mean=1.0))
        self.layers = []
        for _ in range(sh.n_layer):
            Lw = {}
            Lw["norm_w"] = act_t(randn(sh.d_model, scale=0.1, mean=1.0))
            Lw["in_proj_w"], Lw["in_proj_s"] = lin(sh.proj, sh.d_model)
            Lw["conv1d_w"] = act_t(randn(sh.xbc, sh.d_conv, scale=0.3))
            Lw["conv1d_b"] = act_t(randn(sh.xbc, scale=0.1))
            # Mamba-2 init: dt log-uniform in [1e-3, 1e-1], dt_bias = softplus^-1(dt)
            u = torch.rand(H, generator=g, device=device)
            dtv = torch.exp(u * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
            Lw["dt_bias"] = act_t(dtv + torch.log(-torch.expm1(-dtv)))
            Lw["A_log"] = act_t(torch.log(1.0 + 15.0 * torch.rand(H, generator=g, device=device)))
            Lw["D"] = act_t(randn(H, scale=0.1, mean=1.0))
            Lw["mixer_norm_w"] = act_t(randn(sh.d_inner, scale=0.1, mean=1.0))
            Lw["out_proj_w"], Lw["out_proj_s"] = lin(sh.d_model, sh.d_inner)
            self.layers.append(Lw)
        if head == "tied":
            self.lm_head = self.embed   # tied (mamba2_model.cpp:75-83)
        elif head == "permuted":
            perm = torch.randperm(sh.vocab_size, generator=g, device=device)
            self.lm_head = torch.empty_like(self.embed)
            self.lm_head[perm] = self.embed
        else:
            raise ValueError(f"head must be 'tied' or 'permuted', not {head!r}")

    # -- C-ABI views ------------------------------------------------------
    def config(self) -> ModelConfig:
        s = self.shape
        return ModelConfig(s.d_model, s.n_layer, s.d_state, s.d_conv, s.expand, s.vocab_size,
                           s.n_heads, s.d_head, s.chunk_size, s.n_groups, self.act, self.wfmt)

    def layer_structs(self):
        arr = (LayerWeights * self.shape.n_layer)()
        for i, Lw in enumerate(self.layers):
            for k in LayerWeights._fields_:
                name = k[0]
                t = Lw.get(name)
                setattr(arr[i], name, t.data_ptr() if t is not None else None)
        return arr

    def weight_bytes(self):
        """Bytes of all weights read once per decode step (per sequence-independent)."""
        n = 0
        for Lw in self.layers:
            for t in Lw.values():
                if t is not None:
                    n += t.numel() * t.element_size()
        return n + self.norm_f.numel() * self.norm_f.element_size() + \
            self.lm_head.numel() * self.lm_head.element_size()

    def to_host(self):
        """numpy copies (bit patterns) of every tensor, for the CPU oracle."""
        import numpy as np

        def h(t):
            if t is None:
                return None
            t = t.detach().cpu().contiguous()
            if t.dtype in (torch.float16, torch.bfloat16):
                return t.view(torch.int16).numpy().view(np.uint16).copy()
            return t.numpy().copy()

        return {
            "embed": h(self.embed), "norm_f": h(self.norm_f), "lm_head": h(self.lm_head),
            "layers": [{k: h(v) for k, v in Lw.items()} for Lw in self.layers],
        }


class Engine:
    """lssm_engine wrapper: prefill / decode / graph-replayed decode."""

    def __init__(self, ctx, model, max_batch: int, max_seq: int):
        """`model`: a DeviceModel, or the FileModel of an uploaded .ssm file
        (lite_ssm_amd.ssm), whose tensors are device addresses (ints)."""
        self.ctx, self.model = ctx, model
        self._cfg = model.config()
        self._layers = model.layer_structs()
        ptr = lambda t: t if isinstance(t, int) else t.data_ptr()  # noqa: E731
        h = C.c_void_p()
        check(lib.lssm_engine_create(C.byref(h), ctx.h, C.byref(self._cfg), ptr(model.embed),
                                     ptr(model.norm_f), ptr(model.lm_head),
                                     self._layers, max_batch, max_seq))
        self.h = h
        self.max_batch, self.max_seq = max_batch, max_seq

    def close(self):
        if getattr(self, "h", None):
            lib.lssm_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        check(lib.lssm_engine_reset(self.h))

    def prefill(self, ids: torch.Tensor, next_ids: torch.Tensor):
        B, L = ids.shape
        check(lib.lssm_engine_prefill(self.h, ids.data_ptr(), B, L, next_ids.data_ptr()))

    def decode(self, ids: torch.Tensor, next_ids: torch.Tensor):
        check(lib.lssm_engine_decode(self.h, ids.data_ptr(), ids.shape[0], next_ids.data_ptr()))

    def decode_graph(self, ids: torch.Tensor, next_ids: torch.Tensor, steps: int):
        check(lib.lssm_engine_decode_graph(self.h, ids.data_ptr(), ids.shape[0],
                                           next_ids.data_ptr(), steps))

    def logits(self, rows: int) -> torch.Tensor:
        p = C.c_void_p()
        check(lib.lssm_engine_logits(self.h, C.byref(p)))
        out = torch.empty(rows, self.model.shape.vocab_size, dtype=TORCH_DTYPE[self.model.act],
                          device=self.model.device)
        check(lib.lssm_memcpy_d2d(self.ctx.h, out.data_ptr(), p.value, out.numel() * out.element_size()))
        return out

    def set_trace(self, buf):
        """Parity hook: every later prefill / decode writes the hidden rows
        entering each layer (and after the last) into `buf` (a device tensor of
        at least (n_layer + 1) * rows * d_model activation elements), or None."""
        if buf is None:
            check(lib.lssm_engine_set_trace(self.h, None, 0))
        else:
            check(lib.lssm_engine_set_trace(self.h, buf.data_ptr(), buf.numel() * buf.element_size()))
        self._trace = buf

    def set_id_log(self, buf):
        """Every later decode step (eager or graph-replayed) appends its greedy
        ids to `buf` (device int32 [steps, batch]) row by row; None turns it off."""
        if buf is None:
            check(lib.lssm_engine_set_id_log(self.h, None, 0))
        else:
            assert buf.dtype == torch.int32 and buf.is_contiguous()
            check(lib.lssm_engine_set_id_log(self.h, buf.data_ptr(), buf.shape[0]))
        self._id_log = buf

    def fused_layers(self):
        """(layers of the last decode step whose SSD step ran inside the in_proj
        launch, layers whose whole mixer ran as one launch)."""
        a, b = C.c_uint32(), C.c_uint32()
        check(lib.lssm_engine_fused_layers(self.h, C.byref(a), C.byref(b)))
        return a.value, b.value

    def state(self):
        """(conv [n_layer, max_batch, xbc, d_conv] act, ssd [n_layer, max_batch, H, P, N] f32) copies."""
        cp, sp = C.c_void_p(), C.c_void_p()
        check(lib.lssm_engine_state(self.h, C.byref(cp), C.byref(sp)))
        s = self.model.shape
        conv = torch.empty(s.n_layer, self.max_batch, s.xbc, s.d_conv,
                           dtype=TORCH_DTYPE[self.model.act], device=self.model.device)
        ssd = torch.empty(s.n_layer, self.max_batch, s.n_heads, s.d_head, s.d_state,
                          dtype=torch.float32, device=self.model.device)
        check(lib.lssm_memcpy_d2d(self.ctx.h, conv.data_ptr(), cp.value, conv.numel() * conv.element_size()))
        check(lib.lssm_memcpy_d2d(self.ctx.h, ssd.data_ptr(), sp.value, ssd.numel() * 4))
        return conv, ssd

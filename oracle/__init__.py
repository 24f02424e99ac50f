"""CPU oracle for the lite-ssm Mamba-2 hot path — TEST INFRASTRUCTURE ONLY.

ctypes binding of ``oracle/liblssm_oracle.so`` (built from ``lssm_oracle.c`` by
``oracle/Makefile``), a restatement of the reference's Metal kernels in C.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as a checker / baseline.

Arrays are numpy; activation tensors are carried as their bit patterns
(uint16 for fp16 / bf16, float32 for fp32).  Every function names the
reference file:line it restates in ``lssm_oracle.c``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblssm_oracle.so")

F16, BF16, F32 = 0, 1, 2
W_DENSE, W_Q4_B32, W_Q4_G64, W_Q8_G32 = 0, 6, 7, 8
EPI_NONE, EPI_SILU, EPI_ADD = 0, 1, 2


def _build_if_missing():
    if not os.path.exists(LIB_PATH):
        import subprocess
        subprocess.run(["make", "-s", "-C", _HERE], check=True)


_build_if_missing()
_L = C.CDLL(LIB_PATH)
_vp, _u32, _i, _f, _sz = C.c_void_p, C.c_uint32, C.c_int, C.c_float, C.c_size_t


class _SSDDims(C.Structure):
    _fields_ = [("L", _u32), ("H", _u32), ("P", _u32), ("N", _u32), ("n_groups", _u32),
                ("chunk_size", _u32), ("dt_min", _f), ("dt_max", _f), ("has_D", _u32)]


class _SSDStepDims(C.Structure):
    _fields_ = [("H", _u32), ("P", _u32), ("N", _u32), ("n_groups", _u32), ("dt_min", _f),
                ("dt_max", _f), ("has_D", _u32)]


class _FusedDims(C.Structure):
    _fields_ = [(n, _u32) for n in
                ("L", "d_model", "d_inner", "d_state", "n_groups", "n_heads", "d_conv", "proj_dim")]


class _Cfg(C.Structure):
    _fields_ = [(n, _u32) for n in
                ("d_model", "n_layer", "d_state", "d_conv", "expand", "vocab_size", "n_heads",
                 "d_head", "chunk_size", "n_groups", "act", "wfmt")]


class _Layer(C.Structure):
    _fields_ = [(n, _vp) for n in
                ("norm_w", "in_proj_w", "in_proj_s", "conv1d_w", "conv1d_b", "dt_bias", "A_log",
                 "D", "mixer_norm_w", "out_proj_w", "out_proj_s")]


class _Model(C.Structure):
    _fields_ = [("cfg", _Cfg), ("embed", _vp), ("norm_f", _vp), ("lm_head", _vp),
                ("layers", C.POINTER(_Layer))]


_SIGS = {
    "orc_f2h": ([_f], C.c_uint16), "orc_h2f": ([C.c_uint16], _f),
    "orc_f2b": ([_f], C.c_uint16), "orc_b2f": ([C.c_uint16], _f),
    "orc_f32_to_act": ([_vp, _vp, _sz, _i], None),
    "orc_act_to_f32": ([_vp, _vp, _sz, _i], None),
    "orc_wfmt_group": ([_i], _sz),
    "orc_packed_nbytes": ([_i, _sz, _sz, _i], _sz),
    "orc_dequant": ([_vp, _vp, _vp, _u32, _u32, _i, _i], None),
    "orc_quantize": ([_vp, _u32, _u32, _i, _vp, _vp], None),
    "orc_rmsnorm": ([_vp, _vp, _vp, _u32, _u32, _f, _i], None),
    "orc_linear": ([_vp, _u32, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _i, _i, _i, _i], None),
    "orc_silu": ([_vp, _vp, _u32, _i], None),
    "orc_add_inplace": ([_vp, _vp, _u32, _i], None),
    "orc_silu_gated": ([_vp, _vp, _vp, _u32, _i], None),
    "orc_split_silu_xbc": ([_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _i], None),
    "orc_conv1d": ([_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _i], None),
    "orc_conv1d_update": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _i], None),
    "orc_conv1d_seed": ([_vp, _vp, _u32, _u32, _u32, _u32, _i], None),
    "orc_gated_rmsnorm": ([_vp, _vp, _vp, _vp, _u32, _u32, _f, _i], None),
    "orc_inproj_fused": ([_vp] * 10 + [_FusedDims, _i], None),
    "orc_ssd_chunked": ([_vp] * 9 + [_u32, _SSDDims, _i], None),
    "orc_ssd_step": ([_vp] * 9 + [_u32, _SSDStepDims, _i], None),
    "orc_embed": ([_vp, _vp, _vp, _u32, _u32, _i], None),
    "orc_argmax": ([_vp, _vp, _u32, _u32, _i], None),
    "orc_model_prefill": ([C.POINTER(_Model), _vp, _vp, _vp, _u32, _u32, _vp], None),
    "orc_model_decode": ([C.POINTER(_Model), _vp, _vp, _vp, _u32, _vp], None),
    "orc_model_block": ([C.POINTER(_Model), _u32, _vp, _vp, _vp, _u32, _u32, _i], None),
    "orc_model_logits": ([C.POINTER(_Model), _vp, _u32, _vp], None),
    "orc_num_threads": ([], _i),
    "orc_set_num_threads": ([_i], None),
    "orc_set_accum": ([_i], None),
    "orc_accum": ([], _i),
}
for _n, (_a, _r) in _SIGS.items():
    _fn = getattr(_L, _n)
    _fn.argtypes = _a
    _fn.restype = _r


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def act_np_dtype(act):
    return np.float32 if act == F32 else np.uint16


# --- conversions -------------------------------------------------------------
def to_act(x, act):
    """float32 array -> activation bit pattern array (RNE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=act_np_dtype(act))
    _L.orc_f32_to_act(_ptr(x), _ptr(out), x.size, act)
    return out


def from_act(a, act):
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, dtype=np.float32)
    _L.orc_act_to_f32(_ptr(a), _ptr(out), a.size, act)
    return out


def round_act(x, act):
    return from_act(to_act(x, act), act)


# --- weights ------------------------------------------------------------------
def group_size(wfmt):
    return int(_L.orc_wfmt_group(wfmt))


def quantize(w, wfmt):
    """w float32 [N, K] -> (packed uint8, scales uint16 fp16 bits)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    G = group_size(wfmt)
    packed = np.zeros((N, K if wfmt == W_Q8_G32 else K // 2), dtype=np.uint8)
    scales = np.zeros((N, K // G), dtype=np.uint16)
    _L.orc_quantize(_ptr(w), N, K, wfmt, _ptr(packed), _ptr(scales))
    return packed, scales


def dequant(packed, scales, N, K, wfmt, act=F16):
    out = np.empty((N, K), dtype=np.float32)
    _L.orc_dequant(_ptr(packed), _ptr(scales), _ptr(out), N, K, wfmt, act)
    return out


# --- kernels --------------------------------------------------------------------
def rmsnorm(x, w, eps, act):
    rows, dim = x.shape
    y = np.empty_like(x)
    _L.orc_rmsnorm(_ptr(x), _ptr(w), _ptr(y), rows, dim, eps, act)
    return y


def linear(x, w, s, M, N, K, wfmt, act, epi=EPI_NONE, residual=None, round_dequant=0):
    y = np.empty((M, N), dtype=act_np_dtype(act))
    _L.orc_linear(_ptr(x), 0, _ptr(w), _ptr(s), _ptr(y), 0, _ptr(residual), M, N, K, wfmt, act,
                  epi, round_dequant)
    return y


def silu(x, act):
    y = np.empty_like(x)
    _L.orc_silu(_ptr(x), _ptr(y), x.size, act)
    return y


def add_inplace(y, x, act):
    _L.orc_add_inplace(_ptr(y), _ptr(x), y.size, act)
    return y


def silu_gated(x, g, act):
    y = np.empty_like(x)
    _L.orc_silu_gated(_ptr(x), _ptr(g), _ptr(y), x.size, act)
    return y


def split_silu_xbc(xbc, rows, d_inner, d_state, n_groups, act):
    GN = d_state * n_groups
    dt = act_np_dtype(act)
    x = np.empty((rows, d_inner), dt)
    B = np.empty((rows, GN), dt)
    Cc = np.empty((rows, GN), dt)
    _L.orc_split_silu_xbc(_ptr(xbc), _ptr(x), _ptr(B), _ptr(Cc), rows, d_inner, d_state, n_groups, act)
    return x, B, Cc


def conv1d(x, w, b, B, L, D, K, act):
    y = np.empty((B, L, D), dtype=act_np_dtype(act))
    _L.orc_conv1d(_ptr(x), _ptr(w), _ptr(b), _ptr(y), B, L, D, K, act)
    return y


def conv1d_update(x_new, state, w, b, B, D, K, act):
    """Updates `state` in place; returns y [B, D]."""
    y = np.empty((B, D), dtype=act_np_dtype(act))
    _L.orc_conv1d_update(_ptr(x_new), _ptr(state), _ptr(w), _ptr(b), _ptr(y), B, D, K, act)
    return y


def conv1d_seed(xbc, B, L, D, K, act):
    st = np.empty((B, D, K), dtype=act_np_dtype(act))
    _L.orc_conv1d_seed(_ptr(xbc), _ptr(st), B, L, D, K, act)
    return st


def gated_rmsnorm(z, y, w, eps, act):
    rows, dim = z.shape
    out = np.empty_like(z)
    _L.orc_gated_rmsnorm(_ptr(z), _ptr(y), _ptr(w), _ptr(out), rows, dim, eps, act)
    return out


def inproj_fused(normed, W_in, W_conv, conv_b, L, d_model, d_inner, d_state, n_groups, n_heads,
                 d_conv, act=F16):
    GN = n_groups * d_state
    xbc = d_inner + 2 * GN
    proj = d_inner + xbc + n_heads
    dt = act_np_dtype(act)
    z = np.empty((L, d_inner), dt)
    x = np.empty((L, d_inner), dt)
    B = np.empty((L, GN), dt)
    Cc = np.empty((L, GN), dt)
    dtv = np.empty((L, n_heads), dt)
    pxbc = np.empty((L, xbc), dt)
    d = _FusedDims(L, d_model, d_inner, d_state, n_groups, n_heads, d_conv, proj)
    _L.orc_inproj_fused(_ptr(normed), _ptr(W_in), _ptr(W_conv), _ptr(conv_b), _ptr(z), _ptr(x),
                        _ptr(B), _ptr(Cc), _ptr(dtv), _ptr(pxbc), d, act)
    return z, x, B, Cc, dtv, pxbc


def ssd_chunked(X, B, Cc, dt_raw, dt_bias, A_log, D, state, batch, L, H, P, N, G, chunk, act,
                dt_min=1e-6, dt_max=1e6, has_D=1):
    """Updates `state` (float32 [batch, H, P, N]) in place; returns Y [batch, L, H, P]."""
    Y = np.empty((batch, L, H, P), dtype=act_np_dtype(act))
    d = _SSDDims(L, H, P, N, G, chunk, dt_min, dt_max, has_D)
    _L.orc_ssd_chunked(_ptr(X), _ptr(B), _ptr(Cc), _ptr(dt_raw), _ptr(dt_bias), _ptr(A_log),
                       _ptr(D), _ptr(Y), _ptr(state), batch, d, act)
    return Y


def ssd_step(x, B, Cc, dt_raw, dt_bias, A_log, D, state, batch, H, P, N, G, act, dt_min=1e-6,
             dt_max=1e6, has_D=1):
    """Updates `state` in place; returns y [batch, H, P]."""
    y = np.empty((batch, H, P), dtype=act_np_dtype(act))
    d = _SSDStepDims(H, P, N, G, dt_min, dt_max, has_D)
    _L.orc_ssd_step(_ptr(x), _ptr(B), _ptr(Cc), _ptr(dt_raw), _ptr(dt_bias), _ptr(A_log), _ptr(D),
                    _ptr(state), _ptr(y), batch, d, act)
    return y


def embed(table, ids, d_model, act):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, d_model), dtype=act_np_dtype(act))
    _L.orc_embed(_ptr(table), _ptr(ids), _ptr(out), ids.size, d_model, act)
    return out


def argmax(logits, act):
    rows, vocab = logits.shape
    ids = np.empty(rows, dtype=np.int32)
    _L.orc_argmax(_ptr(logits), _ptr(ids), rows, vocab, act)
    return ids


# --- whole model -------------------------------------------------------------------
class Model:
    """Host copy of a model (DeviceModel.to_host() layout) bound for the oracle."""

    def __init__(self, host: dict, cfg: dict, act: int, wfmt: int):
        self.host, self.act, self.wfmt = host, act, wfmt
        self.cfg = dict(cfg)
        n_layer = len(host["layers"])
        self._layers = (_Layer * n_layer)()
        for i, Lw in enumerate(host["layers"]):
            for name, _ in _Layer._fields_:
                a = Lw.get(name)
                setattr(self._layers[i], name, _ptr(a) if a is not None else None)
        c = self.cfg
        self._m = _Model(_Cfg(c["d_model"], n_layer, c["d_state"], c["d_conv"], c["expand"],
                              c["vocab_size"], c["n_heads"], c["d_head"], c["chunk_size"],
                              c["n_groups"], act, wfmt),
                         _ptr(host["embed"]), _ptr(host["norm_f"]), _ptr(host["lm_head"]),
                         C.cast(self._layers, C.POINTER(_Layer)))
        self.n_layer = n_layer

    def new_state(self, batch):
        c = self.cfg
        d_inner = c["expand"] * c["d_model"]
        xbc = d_inner + 2 * c["n_groups"] * c["d_state"]
        conv = np.zeros((self.n_layer, batch, xbc, c["d_conv"]), dtype=act_np_dtype(self.act))
        ssd = np.zeros((self.n_layer, batch, c["n_heads"], c["d_head"], c["d_state"]), np.float32)
        return conv, ssd

    def prefill(self, conv, ssd, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        batch, L = ids.shape
        logits = np.empty((batch, self.cfg["vocab_size"]), dtype=act_np_dtype(self.act))
        _L.orc_model_prefill(C.byref(self._m), _ptr(conv), _ptr(ssd), _ptr(ids), batch, L, _ptr(logits))
        return logits

    def block(self, li, hidden, conv, ssd, batch, L, decode):
        """run_block of layer li on `hidden` ([batch * L, d_model] act bits,
        updated in place); conv / ssd are new_state(batch) arrays."""
        assert hidden.flags["C_CONTIGUOUS"] and hidden.shape == (batch * L, self.cfg["d_model"])
        _L.orc_model_block(C.byref(self._m), li, _ptr(hidden), _ptr(conv), _ptr(ssd), batch, L,
                           1 if decode else 0)
        return hidden

    def logits(self, hidden_rows):
        """norm_f + lm_head of hidden rows [rows, d_model] -> logits [rows, vocab]."""
        hidden_rows = np.ascontiguousarray(hidden_rows)
        rows = hidden_rows.shape[0]
        out = np.empty((rows, self.cfg["vocab_size"]), dtype=act_np_dtype(self.act))
        _L.orc_model_logits(C.byref(self._m), _ptr(hidden_rows), rows, _ptr(out))
        return out

    def decode(self, conv, ssd, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        batch = ids.size
        logits = np.empty((batch, self.cfg["vocab_size"]), dtype=act_np_dtype(self.act))
        _L.orc_model_decode(C.byref(self._m), _ptr(conv), _ptr(ssd), _ptr(ids), batch, _ptr(logits))
        return logits


def num_threads():
    return int(_L.orc_num_threads())


def set_num_threads(n):
    _L.orc_set_num_threads(int(n))


def set_accum(f32):
    """Summation of the linears' dot products: False = double (default),
    True = float32 in sixteen partial sums (see lssm_oracle.c)."""
    _L.orc_set_accum(1 if f32 else 0)


class accum_f32:
    """with O.accum_f32(): ... runs the oracle with float32 sums."""

    def __enter__(self):
        self._old = int(_L.orc_accum())
        _L.orc_set_accum(1)

    def __exit__(self, *exc):
        _L.orc_set_accum(self._old)

""".ssm weight files through the C ABI (``lssm_ssm_*`` in include/lssm.h).

:class:`SSMFile` mirrors the reference's ``SSMFile`` (include/lite_ssm/model.hpp:40-62,
src/core/ssm_loader.cpp): open + validate, ``find`` / ``at``, the header's model
hyperparameters; ``upload`` copies the file into HBM once and ``model`` resolves
``Mamba2Model``'s weight lookups (src/model/mamba2_model.cpp:62-116) into an object
:class:`lite_ssm_amd.model.Engine` accepts.  :class:`Writer` is the write path of
tools/ssm_format.py; :func:`write_random` writes a random-initialised model and
:func:`write_device_model` writes the tensors of a :class:`~lite_ssm_amd.model.DeviceModel`.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import (BF16, F16, F32, W_DENSE, W_Q4_B32, W_Q4_G64, W_Q8_G32, LayerWeights, LssmError,
               ModelConfig, SsmHeader, SsmTensor, check, lib)
from .model import GROUP, Shape

# tensor dtype codes (include/lite_ssm/ssm_format.hpp:29-41, + this build's 7 and 8)
DTYPE_F16, DTYPE_BF16, DTYPE_F32, DTYPE_I8, DTYPE_U8, DTYPE_I32 = 0, 1, 2, 3, 4, 5
DTYPE_INT4_B32, DTYPE_Q4_G64, DTYPE_Q8_G32 = 6, 7, 8
BLOCK_DTYPES = (DTYPE_INT4_B32, DTYPE_Q4_G64, DTYPE_Q8_G32)
_NP = {DTYPE_F16: np.uint16, DTYPE_BF16: np.uint16, DTYPE_F32: np.float32, DTYPE_I8: np.int8,
       DTYPE_U8: np.uint8, DTYPE_I32: np.int32}

HEADER_FIELDS = ("d_model", "n_layer", "d_state", "d_conv", "expand", "vocab_size", "n_heads",
                 "d_head", "chunk_size", "default_dtype", "n_groups", "norm_before_gate")


def packed_nbytes(dtype: int, numel: int) -> int:
    """dtype_packed_nbytes (ssm_format.hpp:45-69) with codes 7 and 8."""
    return int(lib.lssm_ssm_packed_nbytes(dtype, numel))


def layer_names(i: int):
    """Names of layer i's tensors in the exporter's order, keyed by the engine's field."""
    p = f"backbone.layers.{i}."
    return {"dt_bias": p + "mixer.dt_bias", "A_log": p + "mixer.A_log", "D": p + "mixer.D",
            "conv1d_w": p + "mixer.conv1d.weight", "conv1d_b": p + "mixer.conv1d.bias",
            "in_proj_w": p + "mixer.in_proj.weight", "mixer_norm_w": p + "mixer.norm.weight",
            "out_proj_w": p + "mixer.out_proj.weight", "norm_w": p + "norm.weight"}


class SSMFile:
    """A validated, read-only mapping of one .ssm file."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib.lssm_ssm_open(C.byref(h), str(path).encode()))
        self.h = h
        self.path = str(path)
        self.header = SsmHeader()
        check(lib.lssm_ssm_get_header(self.h, C.byref(self.header)))

    def close(self):
        if getattr(self, "h", None):
            lib.lssm_ssm_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- index ------------------------------------------------------------
    def config(self) -> dict:
        return {k: getattr(self.header, k) for k in HEADER_FIELDS}

    def __len__(self):
        return self.header.n_tensors

    def entries(self):
        """[(name, SsmTensor)] in file order."""
        out = []
        buf = C.create_string_buffer(4096)
        for i in range(len(self)):
            t = SsmTensor()
            check(lib.lssm_ssm_tensor_at(self.h, i, buf, len(buf), C.byref(t)))
            out.append((buf.value.decode(), t))
        return out

    def names(self):
        return [n for n, _ in self.entries()]

    def find(self, name: str):
        t = SsmTensor()
        rc = lib.lssm_ssm_find(self.h, name.encode(), C.byref(t))
        if rc == 4:   # LSSM_ENOTFOUND
            return None
        check(rc)
        return t

    def at(self, name: str) -> SsmTensor:
        t = SsmTensor()
        check(lib.lssm_ssm_find(self.h, name.encode(), C.byref(t)))
        return t

    def raw(self, name: str) -> np.ndarray:
        """Copy of a payload's bytes."""
        t = self.at(name)
        if t.nbytes == 0:
            return np.zeros(0, np.uint8)
        return np.ctypeslib.as_array((C.c_uint8 * t.nbytes).from_address(t.host)).copy()

    def array(self, name: str):
        """Host copy of a tensor: an array of its shape (16-bit floats as uint16 bit
        patterns), or for block formats (packed [N, K/2 or K] uint8, scales [N, K/G] uint16)."""
        t = self.at(name)
        shape = tuple(t.shape[i] for i in range(t.rank))
        b = self.raw(name)
        if t.dtype in BLOCK_DTYPES:
            N, K = shape[0], int(np.prod(shape[1:]))
            pb = N * K if t.dtype == DTYPE_Q8_G32 else N * K // 2
            G = 64 if t.dtype == DTYPE_Q4_G64 else 32
            return b[:pb].reshape(N, -1), b[pb:].view(np.uint16).reshape(N, K // G)
        return b.view(_NP[t.dtype]).reshape(shape)

    # -- device -----------------------------------------------------------
    def upload(self, ctx) -> int:
        """Device address of the file's HBM copy (made on the first call)."""
        p = C.c_void_p()
        check(lib.lssm_ssm_upload(self.h, ctx.h, C.byref(p)))
        return p.value

    def model(self, ctx) -> "FileModel":
        """Uploads the file (once) and resolves the model's weights in HBM."""
        return FileModel(self, self.upload(ctx))


class FileModel:
    """Weights of an uploaded .ssm file, in the form Engine and the oracle take
    (the interface of DeviceModel: config(), layer_structs(), embed / norm_f /
    lm_head device pointers, shape, act, wfmt, to_host())."""

    def __init__(self, f: SSMFile, device_base: int):
        self.file, self.device_base = f, device_base
        cfg = ModelConfig()
        e, n, h = C.c_void_p(), C.c_void_p(), C.c_void_p()
        n_layer = f.header.n_layer
        self._layers = (LayerWeights * max(n_layer, 1))()
        check(lib.lssm_ssm_model(f.h, device_base, C.byref(cfg), C.byref(e), C.byref(n),
                                 C.byref(h), self._layers, n_layer))
        self._cfg = cfg
        self.embed, self.norm_f, self.lm_head = e.value, n.value, h.value
        self.act, self.wfmt, self.device = cfg.act, cfg.wfmt, "cuda"
        self.shape = Shape(cfg.d_model, cfg.n_layer, cfg.d_state, cfg.d_conv, cfg.expand,
                           cfg.vocab_size, cfg.n_heads, cfg.d_head, cfg.chunk_size, cfg.n_groups)

    def config(self) -> ModelConfig:
        return self._cfg

    def layer_structs(self):
        return self._layers

    def to_host(self):
        """Host copies in DeviceModel.to_host()'s layout, for the CPU oracle."""
        f = self.file
        layers = []
        for i in range(self.shape.n_layer):
            Lw = {}
            for key, name in layer_names(i).items():
                a = f.array(name)
                if isinstance(a, tuple):
                    Lw[key], Lw[key[:-1] + "s"] = a
                else:
                    Lw[key] = a.reshape(a.shape[0], -1) if key == "conv1d_w" else a
            if self.wfmt == W_DENSE:
                Lw["in_proj_s"] = Lw["out_proj_s"] = None
            layers.append(Lw)
        emb = f.array("backbone.embeddings.weight")
        head = f.array("lm_head.weight") if f.find("lm_head.weight") is not None else emb
        return {"embed": emb, "norm_f": f.array("backbone.norm_f.weight"), "lm_head": head,
                "layers": layers}


class Writer:
    """Streaming .ssm writer: declare every tensor, then put payloads."""

    def __init__(self, path: str, **hparams):
        hp = SsmHeader()
        for k in HEADER_FIELDS:
            setattr(hp, k, int(hparams.get(k, 0)))
        h = C.c_void_p()
        check(lib.lssm_ssm_writer_create(C.byref(h), str(path).encode(), C.byref(hp)))
        self.h = h

    def declare(self, name: str, dtype: int, shape):
        shp = (C.c_uint64 * 4)(*[int(s) for s in shape])
        check(lib.lssm_ssm_writer_declare(self.h, name.encode(), dtype, len(shape), shp))

    def put(self, name: str, data):
        b = np.ascontiguousarray(data)
        check(lib.lssm_ssm_writer_put(self.h, name.encode(), b.ctypes.data, b.nbytes))

    def finish(self):
        h, self.h = self.h, None
        if h:
            check(lib.lssm_ssm_writer_finish(h))

    def __del__(self):
        if getattr(self, "h", None):
            lib.lssm_ssm_writer_finish(self.h)
            self.h = None


def quantize(w: np.ndarray, wfmt: int):
    """lssm_quantize: fp32 [N, K] -> (packed uint8 [N, K/2 or K], fp16 scale bits [N, K/G])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    packed = np.empty((N, K if wfmt == W_Q8_G32 else K // 2), np.uint8)
    scales = np.empty((N, K // GROUP[wfmt]), np.uint16)
    check(lib.lssm_quantize(w.ctypes.data, N, K, wfmt, packed.ctypes.data, scales.ctypes.data))
    return packed, scales


def model_config(sh: Shape, act: int, wfmt: int) -> ModelConfig:
    return ModelConfig(sh.d_model, sh.n_layer, sh.d_state, sh.d_conv, sh.expand, sh.vocab_size,
                       sh.n_heads, sh.d_head, sh.chunk_size, sh.n_groups, act, wfmt)


def write_random(path: str, sh: Shape, act: int = BF16, wfmt: int = W_Q4_G64, seed: int = 0):
    """lssm_ssm_write_random: a random-initialised model file of shape `sh`."""
    cfg = model_config(sh, act, wfmt)
    check(lib.lssm_ssm_write_random(str(path).encode(), C.byref(cfg), seed))


def write_device_model(path: str, m, lm_head: bool = False):
    """Write a DeviceModel's tensors (exporter names and order; lm_head tied unless
    `lm_head`)."""
    sh, act, wfmt = m.shape, m.act, m.wfmt
    host = m.to_host()
    wdt = act if wfmt == W_DENSE else wfmt
    w = Writer(path, **{k: getattr(sh, k) for k in HEADER_FIELDS if hasattr(sh, k)},
               default_dtype=act)
    plan = [("backbone.embeddings.weight", act, (sh.vocab_size, sh.d_model), host["embed"])]
    for i, Lw in enumerate(host["layers"]):
        names = layer_names(i)
        for key, name in names.items():
            if key in ("in_proj_w", "out_proj_w"):
                N, K = (sh.proj, sh.d_model) if key == "in_proj_w" else (sh.d_model, sh.d_inner)
                data = Lw[key].reshape(-1).view(np.uint8)
                if wfmt != W_DENSE:
                    data = np.concatenate([data, Lw[key[:-1] + "s"].reshape(-1).view(np.uint8)])
                plan.append((name, wdt, (N, K), data))
            elif key == "conv1d_w":
                plan.append((name, act, (sh.xbc, 1, sh.d_conv), Lw[key]))
            else:
                plan.append((name, act, Lw[key].shape, Lw[key]))
    plan.append(("backbone.norm_f.weight", act, (sh.d_model,), host["norm_f"]))
    if lm_head:
        plan.append(("lm_head.weight", act, (sh.vocab_size, sh.d_model), host["lm_head"]))
    for name, dt, shape, _ in plan:
        w.declare(name, dt, shape)
    for name, _, _, data in plan:
        w.put(name, data)
    w.finish()


__all__ = ["SSMFile", "FileModel", "Writer", "packed_nbytes", "quantize", "write_random",
           "write_device_model", "model_config", "layer_names", "LssmError",
           "DTYPE_F16", "DTYPE_BF16", "DTYPE_F32", "DTYPE_INT4_B32", "DTYPE_Q4_G64",
           "DTYPE_Q8_G32", "F16", "BF16", "F32", "W_Q4_B32", "W_Q4_G64", "W_Q8_G32"]

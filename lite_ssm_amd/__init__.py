"""lite_ssm_amd — MI355X (gfx950) Mamba-2 inference backend, Python host bindings.

The product is the C-ABI shared library ``liblssm_hip.so`` built from
``lite_ssm_amd/csrc`` (see ``include/lssm.h``).  This module binds it with
ctypes.  There is no CPU fallback: importing the package without the built
library raises, and every call that fails on the device raises
:class:`LssmError` with the library's own message.

Device memory and streams come from PyTorch (plumbing only): pass tensors'
``data_ptr()`` and a stream handle, or let :class:`Ctx` create its own stream.
"""
from __future__ import annotations

import ctypes as C
import os

__all__ = [
    "LIB_PATH", "lib", "LssmError", "Ctx", "check", "F16", "BF16", "F32",
    "W_DENSE", "W_Q4_B32", "W_Q4_G64", "W_Q8_G32", "EPI_NONE", "EPI_SILU", "EPI_ADD",
    "LinearDims", "RMSNormDims", "RMSLinearDims", "Conv1dDims", "SSDDims", "SSDStepDims",
    "FusedInProjDims", "ModelConfig", "LayerWeights", "SsmHeader", "SsmTensor",
    "exported_symbols",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblssm_hip.so")

# dtype / format / epilogue codes (include/lssm.h)
F16, BF16, F32 = 0, 1, 2
W_DENSE, W_Q4_B32, W_Q4_G64, W_Q8_G32 = 0, 6, 7, 8
EPI_NONE, EPI_SILU, EPI_ADD = 0, 1, 2
DEBUG_STALE_WAIT = 1   # lssm_ctx_set_debug: fused decode waits give up (failure-handling tests)


class LssmError(RuntimeError):
    """A failed lssm_* call; carries the status code and lssm_last_error()."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"lssm error {code}: {msg}")
        self.code = code
        self.msg = msg


class LinearDims(C.Structure):
    _fields_ = [("M", C.c_uint32), ("N", C.c_uint32), ("K", C.c_uint32)]


class RMSNormDims(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("dim", C.c_uint32), ("eps", C.c_float)]


class RMSLinearDims(C.Structure):
    _fields_ = [("N", C.c_uint32), ("K", C.c_uint32), ("eps", C.c_float)]


class Conv1dDims(C.Structure):
    _fields_ = [("B", C.c_uint32), ("L", C.c_uint32), ("D", C.c_uint32), ("K", C.c_uint32)]


class SSDDims(C.Structure):
    _fields_ = [("L", C.c_uint32), ("H", C.c_uint32), ("P", C.c_uint32), ("N", C.c_uint32),
                ("n_groups", C.c_uint32), ("chunk_size", C.c_uint32), ("dt_min", C.c_float),
                ("dt_max", C.c_float), ("has_D", C.c_uint32)]


class SSDStepDims(C.Structure):
    _fields_ = [("H", C.c_uint32), ("P", C.c_uint32), ("N", C.c_uint32), ("n_groups", C.c_uint32),
                ("dt_min", C.c_float), ("dt_max", C.c_float), ("has_D", C.c_uint32)]


class FusedInProjDims(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("L", "d_model", "d_inner", "d_state", "n_groups", "n_heads", "d_conv", "proj_dim")]


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("d_model", "n_layer", "d_state", "d_conv", "expand", "vocab_size", "n_heads",
                 "d_head", "chunk_size", "n_groups", "act", "wfmt")]


class LayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("norm_w", "in_proj_w", "in_proj_s", "conv1d_w", "conv1d_b", "dt_bias", "A_log",
                 "D", "mixer_norm_w", "out_proj_w", "out_proj_s")]


class SsmHeader(C.Structure):
    """lssm_ssm_header: .ssm FileHeader fields (include/lite_ssm/ssm_format.hpp:73-110)."""
    _fields_ = ([(n, C.c_uint32) for n in ("version", "header_size", "n_tensors")] +
                [(n, C.c_uint64) for n in ("index_offset", "data_offset", "file_size")] +
                [(n, C.c_uint32) for n in
                 ("d_model", "n_layer", "d_state", "d_conv", "expand", "vocab_size", "n_heads",
                  "d_head", "chunk_size", "default_dtype", "n_groups", "norm_before_gate")])


class SsmTensor(C.Structure):
    """lssm_ssm_tensor: one index entry (lite_ssm::Tensor)."""
    _fields_ = [("dtype", C.c_uint32), ("rank", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("host", C.c_void_p)]


_vp, _u32, _i, _f, _sz = C.c_void_p, C.c_uint32, C.c_int, C.c_float, C.c_size_t
_SIGS = {
    "lssm_last_error": ([], C.c_char_p),
    "lssm_ctx_create": ([C.POINTER(_vp), _vp], _i),
    "lssm_ctx_destroy": ([_vp], _i),
    "lssm_ctx_stream": ([_vp, C.POINTER(_vp)], _i),
    "lssm_begin_batch": ([_vp], _i),
    "lssm_commit_and_wait": ([_vp], _i),
    "lssm_batch_active": ([_vp], _i),
    "lssm_sync": ([_vp], _i),
    "lssm_ctx_set_debug": ([_vp, _u32], _i),
    "lssm_library_loaded": ([], _i),
    "lssm_has_kernel": ([C.c_char_p], _i),
    "lssm_library_path": ([], C.c_char_p),
    "lssm_kernel_count": ([], _i),
    "lssm_kernel_name": ([_i], C.c_char_p),
    "lssm_malloc": ([C.POINTER(_vp), _sz], _i),
    "lssm_malloc_host": ([C.POINTER(_vp), _sz], _i),
    "lssm_free": ([_vp], _i),
    "lssm_free_host": ([_vp], _i),
    "lssm_memcpy_h2d": ([_vp, _vp, _vp, _sz], _i),
    "lssm_memcpy_d2h": ([_vp, _vp, _vp, _sz], _i),
    "lssm_memcpy_d2d": ([_vp, _vp, _vp, _sz], _i),
    "lssm_memset": ([_vp, _vp, _i, _sz], _i),
    # reference-named
    "lssm_rmsnorm_f16": ([_vp, _vp, _vp, _vp, RMSNormDims], _i),
    "lssm_linear_f16_gemv": ([_vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_linear_silu_f16_gemv": ([_vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_rmsnorm_linear_f16_gemv": ([_vp, _vp, _vp, _vp, _vp, RMSLinearDims], _i),
    "lssm_linear_f16_gemm": ([_vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_linear_silu_f16_gemm": ([_vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_linear_int4_gemv": ([_vp, _vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_linear_int4_gemm": ([_vp, _vp, _vp, _vp, _vp, LinearDims], _i),
    "lssm_silu_f16": ([_vp, _vp, _vp, _u32], _i),
    "lssm_add_inplace_f16": ([_vp, _vp, _vp, _u32], _i),
    "lssm_split_silu_xBC_f16": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32], _i),
    "lssm_silu_gated_f16": ([_vp, _vp, _vp, _vp, _u32], _i),
    "lssm_causal_conv1d_f16": ([_vp, _vp, _vp, _vp, _vp, Conv1dDims], _i),
    "lssm_causal_conv1d_update_f16": ([_vp, _vp, _vp, _vp, _vp, _vp, Conv1dDims], _i),
    "lssm_seed_conv_state_f16": ([_vp, _vp, _vp, _u32, _u32, _u32], _i),
    "lssm_inproj_fused_f16": ([_vp] + [_vp] * 10 + [FusedInProjDims], _i),
    "lssm_ssd_chunked_f16": ([_vp] + [_vp] * 9 + [SSDDims], _i),
    "lssm_ssd_step_f16": ([_vp] + [_vp] * 9 + [SSDStepDims], _i),
    # generic
    "lssm_rmsnorm": ([_vp, _vp, _vp, _vp, _u32, _u32, _f, _i], _i),
    "lssm_linear": ([_vp, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _i, _i, _i], _i),
    "lssm_dequant": ([_vp, _vp, _vp, _vp, _u32, _u32, _i], _i),
    "lssm_silu": ([_vp, _vp, _vp, _u32, _i], _i),
    "lssm_add_inplace": ([_vp, _vp, _vp, _u32, _i], _i),
    "lssm_silu_gated": ([_vp, _vp, _vp, _vp, _u32, _i], _i),
    "lssm_split_silu_xbc": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _i], _i),
    "lssm_conv1d": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _i], _i),
    "lssm_conv1d_update": ([_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _i], _i),
    "lssm_conv1d_seed": ([_vp, _vp, _vp, _u32, _u32, _u32, _u32, _i], _i),
    "lssm_gated_rmsnorm": ([_vp, _vp, _vp, _vp, _vp, _u32, _u32, _f, _i], _i),
    "lssm_norm_linear_decode": ([_vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _i, _i, _i], _i),
    "lssm_ssd_chunked": ([_vp] + [_vp] * 9 + [_u32, SSDDims, _i], _i),
    "lssm_ssd_step": ([_vp] + [_vp] * 9 + [_u32, SSDStepDims, _i], _i),
    "lssm_inproj_decode": ([_vp] * 11 + [_u32] * 7 + [_f, _i, _i], _i),
    "lssm_inproj_ssd_decode": ([_vp] * 14 + [_u32] * 8 + [_f, _i, _i], _i),
    "lssm_inproj_ssd_decode_noalloc": ([_vp] * 13 + [_u32] * 7 + [_f, _i, _i], _i),
    "lssm_mixer_decode": ([_vp] * 16 + [_u32] * 8 + [_f, _i, _i], _i),
    "lssm_embed": ([_vp, _vp, _vp, _vp, _u32, _u32, _u32, _i], _i),
    "lssm_argmax": ([_vp, _vp, _vp, _u32, _u32, _i], _i),
    # engine
    "lssm_engine_create": ([C.POINTER(_vp), _vp, C.POINTER(ModelConfig), _vp, _vp, _vp,
                            C.POINTER(LayerWeights), _u32, _u32], _i),
    "lssm_engine_destroy": ([_vp], _i),
    "lssm_engine_reset": ([_vp], _i),
    "lssm_engine_prefill": ([_vp, _vp, _u32, _u32, _vp], _i),
    "lssm_engine_decode": ([_vp, _vp, _u32, _vp], _i),
    "lssm_engine_decode_graph": ([_vp, _vp, _u32, _vp, _u32], _i),
    "lssm_engine_logits": ([_vp, C.POINTER(_vp)], _i),
    "lssm_engine_set_trace": ([_vp, _vp, C.c_uint64], _i),
    "lssm_engine_set_id_log": ([_vp, _vp, _u32], _i),
    "lssm_engine_state": ([_vp, C.POINTER(_vp), C.POINTER(_vp)], _i),
    "lssm_engine_fused_layers": ([_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)], _i),
    # .ssm files
    "lssm_ssm_packed_nbytes": ([_u32, C.c_uint64], C.c_uint64),
    "lssm_ssm_open": ([C.POINTER(_vp), C.c_char_p], _i),
    "lssm_ssm_close": ([_vp], _i),
    "lssm_ssm_get_header": ([_vp, C.POINTER(SsmHeader)], _i),
    "lssm_ssm_tensor_at": ([_vp, _u32, C.c_char_p, _sz, C.POINTER(SsmTensor)], _i),
    "lssm_ssm_find": ([_vp, C.c_char_p, C.POINTER(SsmTensor)], _i),
    "lssm_ssm_upload": ([_vp, _vp, C.POINTER(_vp)], _i),
    "lssm_ssm_model": ([_vp, _vp, C.POINTER(ModelConfig), C.POINTER(_vp), C.POINTER(_vp),
                        C.POINTER(_vp), C.POINTER(LayerWeights), _u32], _i),
    "lssm_ssm_writer_create": ([C.POINTER(_vp), C.c_char_p, C.POINTER(SsmHeader)], _i),
    "lssm_ssm_writer_declare": ([_vp, C.c_char_p, _u32, _u32, C.POINTER(C.c_uint64)], _i),
    "lssm_ssm_writer_put": ([_vp, C.c_char_p, _vp, C.c_uint64], _i),
    "lssm_ssm_writer_finish": ([_vp], _i),
    "lssm_quantize": ([_vp, _u32, _u32, _u32, _vp, _vp], _i),
    "lssm_ssm_write_random": ([C.c_char_p, C.POINTER(ModelConfig), C.c_uint64], _i),
}


def exported_symbols():
    """Names of every entry point this binding declares (== include/lssm.h)."""
    return sorted(_SIGS)


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"lite_ssm_amd: {LIB_PATH} is not built; run __graft_entry__.build() "
            "(make -C lite_ssm_amd/csrc).  There is no CPU fallback.")
    L = C.CDLL(LIB_PATH)
    for name, (args, ret) in _SIGS.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ret
    return L


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise LssmError(rc, lib.lssm_last_error().decode(errors="replace"))


def _p(x):
    """Device pointer of a torch tensor, an int, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


class Ctx:
    """One lssm_ctx: a HIP stream plus the batch flag (MetalOps analogue).

    ``stream`` may be a HIP stream handle (int) to borrow, e.g.
    ``torch.cuda.current_stream().cuda_stream``; by default a stream is created.
    """

    def __init__(self, stream: int | None = None):
        h = C.c_void_p()
        check(lib.lssm_ctx_create(C.byref(h), stream))
        self.h = h

    def close(self):
        if self.h:
            lib.lssm_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        s = C.c_void_p()
        check(lib.lssm_ctx_stream(self.h, C.byref(s)))
        return s.value or 0

    def sync(self):
        check(lib.lssm_sync(self.h))

    def set_debug(self, flags: int):
        check(lib.lssm_ctx_set_debug(self.h, flags))

    def begin_batch(self):
        check(lib.lssm_begin_batch(self.h))

    def commit_and_wait(self):
        check(lib.lssm_commit_and_wait(self.h))

    def batch_active(self) -> bool:
        return bool(lib.lssm_batch_active(self.h))

    # thin op helpers (pointers may be torch tensors or ints) ----------------
    def rmsnorm(self, x, w, y, rows, dim, eps, act):
        check(lib.lssm_rmsnorm(self.h, _p(x), _p(w), _p(y), rows, dim, eps, act))

    def linear(self, x, w, s, y, M, N, K, wfmt, act, epi=EPI_NONE, residual=None,
               x_stride=0, y_stride=0):
        check(lib.lssm_linear(self.h, _p(x), x_stride, _p(w), _p(s), _p(y), y_stride,
                              _p(residual), M, N, K, wfmt, act, epi))

    def dequant(self, w, s, out, N, K, wfmt):
        check(lib.lssm_dequant(self.h, _p(w), _p(s), _p(out), N, K, wfmt))

    def ssd_chunked(self, X, B, Cm, dt, dt_bias, A_log, D, Y, state, batch, dims, act):
        check(lib.lssm_ssd_chunked(self.h, _p(X), _p(B), _p(Cm), _p(dt), _p(dt_bias), _p(A_log),
                                   _p(D), _p(Y), _p(state), batch, dims, act))

    def ssd_step(self, x, B, Cm, dt, dt_bias, A_log, D, state, y, batch, dims, act):
        check(lib.lssm_ssd_step(self.h, _p(x), _p(B), _p(Cm), _p(dt), _p(dt_bias), _p(A_log),
                                _p(D), _p(state), _p(y), batch, dims, act))

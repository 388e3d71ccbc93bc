"""ctypes binding of the C ABI in ``include/imq.h`` and ``include/imq_weights.h``
(``aestrix_amd/libimq.so``).

The library is built in-tree by ``aestrix_amd/build.py``.  Loading never
builds and never falls back: a missing library raises ``ImqLibraryMissing``.
"""

from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libimq.so")

IMQ_OK = 0
IMQ_EINVAL = 1
IMQ_EUNSUPPORTED = 2
IMQ_EHIP = 3
IMQ_ENOMEM = 4

IMQ_BF16 = 0
IMQ_F16 = 1
IMQ_F32 = 2

IMQ_ST_MAX_DIMS = 8
# safetensors dtype strings in imq_st_dtype order, with element sizes.
ST_DTYPES = ["BOOL", "U8", "I8", "U16", "I16", "F16", "BF16", "U32", "I32", "F32", "U64", "I64",
             "F64", "F8_E4M3", "F8_E5M2"]
ST_SIZES = [1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8, 1, 1]


class StInfo(ctypes.Structure):
    """imq_st_info."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * IMQ_ST_MAX_DIMS), ("data", ctypes.c_void_p),
                ("bytes", ctypes.c_size_t), ("shard", ctypes.c_int)]


class QWeight(ctypes.Structure):
    """imq_qweight."""
    _fields_ = [("w", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("n", ctypes.c_int), ("k", ctypes.c_int), ("dtype", ctypes.c_int),
                ("base", ctypes.c_void_p)]


class Plan(ctypes.Structure):
    """imq_plan."""
    _fields_ = [("kernel", ctypes.c_int), ("tile_rows", ctypes.c_int), ("splits", ctypes.c_int),
                ("workspace_bytes", ctypes.c_size_t), ("tile_cols", ctypes.c_int)]


IMQ_ENTRY_QMM_T, IMQ_ENTRY_QGEMM, IMQ_ENTRY_QGEMV, IMQ_ENTRY_FUSED, IMQ_ENTRY_SWIGLU = 0, 1, 2, 3, 4
KERNEL_NAMES = {0: "qgemv", 1: "few_row", 2: "tile", 3: "tile_reg"}


class DitDims(ctypes.Structure):
    """imq_dit_dims."""
    _fields_ = [("l_img", ctypes.c_int), ("l_txt", ctypes.c_int), ("dim", ctypes.c_int),
                ("ff_inner", ctypes.c_int), ("n_double", ctypes.c_int), ("n_single", ctypes.c_int)]


# Every entry point the headers declare, with its ctypes signature.
_p = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_s = ctypes.c_char_p
_QMM = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]
SIGNATURES = {
    "imq_abi_version": ([], _i),
    "imq_status_string": ([_i], ctypes.c_char_p),
    "imq_create": ([_i, ctypes.POINTER(_p)], _i),
    "imq_destroy": ([_p], _i),
    "imq_last_error": ([_p], ctypes.c_char_p),
    "imq_stream_create": ([_p, ctypes.POINTER(_p)], _i),
    "imq_stream_destroy": ([_p, _p], _i),
    "imq_stream_sync": ([_p, _p], _i),
    "imq_malloc": ([_p, _sz, ctypes.POINTER(_p)], _i),
    "imq_free": ([_p, _p], _i),
    "imq_memcpy_h2d": ([_p, _p, _p, _sz, _p], _i),
    "imq_memcpy_d2h": ([_p, _p, _p, _sz, _p], _i),
    "imq_memcpy_d2d": ([_p, _p, _p, _sz, _p], _i),
    "imq_dequantize": ([_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "imq_qmm_t": (_QMM, _i),
    "imq_qmm_t_noalloc": (_QMM, _i),
    "imq_qmm_plan": ([_p, _i, _i, _i, _i, _i, ctypes.POINTER(Plan)], _i),
    "imq_qgemv": (_QMM, _i),
    "imq_qgemm": (_QMM, _i),
    "imq_cast_prescale": ([_p, _p, _p, _sz, ctypes.c_float, _i, _p], _i),
    "imq_qmm_postscale": ([_p, _p, _p, _p, _p, _p, _i, _i, _i, ctypes.c_float, _i, _i, _i, _p], _i),
    "imq_dynamic_scale": ([_p, _p, _sz, ctypes.c_float, _p, _p], _i),
    "imq_cast_prescale_ex": ([_p, _p, _p, _sz, ctypes.c_float, _p, _i, _p], _i),
    "imq_qmm_postscale_ex": ([_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, ctypes.c_float, _p, _i, _i,
                              _i, _p], _i),
    "imq_dequantize_rows": ([_p, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _p], _i),
    "imq_rmsnorm": ([_p, _p, _i, _p, _p, _i, _i, _i, ctypes.c_float, _p], _i),
    "imq_qmm_add": ([_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p], _i),
    "imq_qmm_gate_add": ([_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, ctypes.c_float, _i, _i, _i,
                          _p], _i),
    "imq_qmm_swiglu": ([_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float,
                        ctypes.c_float, _i, _i, _i, _p], _i),
    # imq_weights.h
    "imq_st_open": ([ctypes.POINTER(_s), _i, ctypes.POINTER(_p)], _i),
    "imq_st_open_dir": ([_s, ctypes.POINTER(_p)], _i),
    "imq_st_close": ([_p], _i),
    "imq_st_last_error": ([_p], _s),
    "imq_st_shard_count": ([_p], _i),
    "imq_st_shard_path": ([_p, _i], _s),
    "imq_st_metadata": ([_p, _i, _s], _s),
    "imq_st_count": ([_p], _i),
    "imq_st_info_at": ([_p, _i, ctypes.POINTER(StInfo)], _i),
    "imq_st_find": ([_p, _s, ctypes.POINTER(StInfo)], _i),
    "imq_upload": ([_p, _p, _p, _sz, _p], _i),
    "imq_st_upload": ([_p, _p, _s, _i, _p, _sz, _p], _i),
    "imq_load_qlinear": ([_p, _p, _s, _i, ctypes.POINTER(QWeight), _p], _i),
    "imq_load_qlinear_cat": ([_p, _p, ctypes.POINTER(_s), _i, _i, ctypes.POINTER(QWeight), _p], _i),
    "imq_qweight_free": ([_p, ctypes.POINTER(QWeight)], _i),
    # imq_step.h
    "imq_dit_step_create": ([_p, ctypes.POINTER(DitDims), ctypes.POINTER(QWeight), _i, _i,
                             ctypes.POINTER(_p)], _i),
    "imq_dit_step_set_conditioning": ([_p, _p, _p, _p], _i),
    "imq_dit_step_run": ([_p, _p, _p, _p, _i, _p], _i),
    "imq_dit_step_set_head": ([_p, ctypes.POINTER(QWeight), ctypes.POINTER(QWeight)], _i),
    "imq_dit_step_denoise": ([_p, _p, _p, _p, ctypes.c_float, _i, _p], _i),
    "imq_dit_step_launches": ([_p], _i),
    "imq_dit_double_attn_in": ([_p, _i, _p, _p, _p, _p, _p, _p], _i),
    "imq_dit_double_attn_out": ([_p, _i, _p, _p, _p], _i),
    "imq_dit_double_mlp": ([_p, _i, _p, _p, _p], _i),
    "imq_dit_single_attn_in": ([_p, _i, _p, _p, _p, _p, _p], _i),
    "imq_dit_single_attn_out": ([_p, _i, _p, _p, _p], _i),
    "imq_dit_head_embed": ([_p, _p, _p, _p], _i),
    "imq_dit_head_out": ([_p, _p, _p, _p, _p, ctypes.c_float, _p], _i),
    "imq_te_create": ([_p, _p, _i, _i, ctypes.c_float, _p], _i),
    "imq_te_attn_in": ([_p, _i, _p, _p, _i, _p], _i),
    "imq_te_attn_out_mlp": ([_p, _i, _p, _p, _p, _i, _p], _i),
    "imq_te_dims": ([_p, _p, _p, _p, _p], _i),
    "imq_te_destroy": ([_p], _i),
    "imq_cond_create": ([_p, _p, _p, _p, _p], _i),
    "imq_cond_step_conditioning": ([_p, _p, _i, _p, _p, _p], _i),
    "imq_cond_sinusoid": ([_p, _i, _i, _p], _i),
    "imq_cond_destroy": ([_p], _i),
    "imq_dit_step_destroy": ([_p], _i),
}


class ImqLibraryMissing(RuntimeError):
    """libimq.so is not built; run ``python -m aestrix_amd.build``."""


class ImqError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{_status_name(status)}: {message}")
        self.status = status


class ImqInvalid(ImqError, ValueError):
    pass


class ImqUnsupported(ImqError, NotImplementedError):
    pass


def _status_name(status: int) -> str:
    return {0: "IMQ_OK", 1: "IMQ_EINVAL", 2: "IMQ_EUNSUPPORTED", 3: "IMQ_EHIP",
            4: "IMQ_ENOMEM"}.get(status, f"status {status}")


_lib = None


def load():
    """Load libimq.so (no compute call is made)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImqLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m aestrix_amd.build` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = L
    return _lib


def check(status: int, ctx) -> None:
    if status == IMQ_OK:
        return
    msg = load().imq_last_error(ctx)
    text = msg.decode() if msg else ""
    if status == IMQ_EINVAL:
        raise ImqInvalid(status, text)
    if status == IMQ_EUNSUPPORTED:
        raise ImqUnsupported(status, text)
    raise ImqError(status, text)

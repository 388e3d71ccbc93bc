"""torch-facing mirror of the reference's quantized-linear operator surface.

The reference reaches the path through MLX ops and its direct engine:

* ``dequantized(w, scales:, biases:, groupSize: 64, bits: 4)``
  (``Sources/ImarelloDirect/DirectTEEncoder.swift:129-134``)      -> ``dequantize``
* ``quantizedMM(x, w, scales:, biases:, transpose: true, groupSize: 64, bits: 4)``
  (``Sources/ImarelloDiT/AttentionUtils.swift:212-221``,
  ``Sources/ImarelloDirect/DirectQmmSpike.swift:55-58``)          -> ``quantized_matmul``
* ``QuantizedLinear`` built by ``quantize(model:groupSize:64,bits:4)``
  (``Sources/ImarelloDiT/TransformerWeights.swift:20``)            -> ``QuantizedLinear``
* ``applyLinear`` / ``applyLinearCore`` with ``linearF16`` on
  (``Sources/ImarelloDiT/AttentionUtils.swift:140-150,198-230``)  -> ``apply_linear``
  (``cast_prescale`` + ``qmm_postscale``)
* ``DirectDiTStep.qmm(enc, q, x:, xOff:, y:, yOff:, m:)``
  (``Sources/ImarelloDirect/DirectDiTStep.swift:374-406``)         -> ``qmm``

Every call goes through the C ABI of ``libimq.so`` on torch's current HIP
stream.  torch is used for device memory and streams only; there is no
CPU or torch fallback for any computation.

Tensors: packed weights are ``torch.int32`` (or ``torch.uint32``) ``[N, K/8]``
holding the raw uint32 words; scales, biases, x and y share one element type
T: bfloat16 (the text encoder), float16 (the reference's DiT kernels,
``DirectDiTStep.swift:82-85``) or float32 (its M=1 conditioner kernels,
``DirectConditioner.swift:48``; no MFMA kernel, so ``qgemm`` rejects it and
``quantized_matmul`` runs any M on the qGEMV kernel).
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import torch

from . import _lib

GROUP_SIZE = 64
BITS = 4

_ctx_lock = threading.Lock()
_ctxs: dict[int, ctypes.c_void_p] = {}

_DTYPES = {torch.bfloat16: _lib.IMQ_BF16, torch.float16: _lib.IMQ_F16,
           torch.float32: _lib.IMQ_F32}
_WORD_DTYPES = (torch.int32,) + ((torch.uint32,) if hasattr(torch, "uint32") else ())


def device_index(device: int | str | torch.device | None) -> int:
    """Ordinal of a HIP device given as an int, a string or a torch.device."""
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    d = torch.device(device)
    if d.type != "cuda":
        raise ValueError(f"not a HIP device: {d}")
    return d.index if d.index is not None else torch.cuda.current_device()


def context(device: int | str | torch.device | None = None) -> ctypes.c_void_p:
    """The library context of a HIP device (created once, kept for the process)."""
    idx = device_index(device)
    with _ctx_lock:
        ctx = _ctxs.get(idx)
        if ctx is None:
            L = _lib.load()
            out = ctypes.c_void_p()
            _lib.check(L.imq_create(idx, ctypes.byref(out)), None)
            ctx = out
            _ctxs[idx] = ctx
        return ctx


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_weight(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                  group_size: int, bits: int) -> tuple[int, int]:
    _require(w.is_cuda and scales.is_cuda and biases.is_cuda, "tensors must be on a HIP device")
    _require(w.dtype in _WORD_DTYPES, f"packed weight must be int32/uint32 words, got {w.dtype}")
    _require(w.dim() == 2 and scales.dim() == 2 and biases.dim() == 2,
             "w, scales and biases must be 2-D")
    _require(w.is_contiguous() and scales.is_contiguous() and biases.is_contiguous(),
             "w, scales and biases must be contiguous")
    _require(scales.dtype == biases.dtype, "scales and biases must share a dtype")
    if group_size != GROUP_SIZE or bits != BITS:
        # the same answer the C ABI gives (IMQ_EUNSUPPORTED)
        raise _lib.ImqUnsupported(_lib.IMQ_EUNSUPPORTED,
                                  f"group_size={group_size} bits={bits}: only 64 / 4 are provided")
    n, k = w.shape[0], w.shape[1] * 8
    _require(tuple(scales.shape) == (n, k // GROUP_SIZE) and scales.shape == biases.shape,
             f"scales/biases must be [{n}, {k // GROUP_SIZE}] for w {tuple(w.shape)}, "
             f"got {tuple(scales.shape)} / {tuple(biases.shape)}")
    return n, k


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = GROUP_SIZE, bits: int = BITS,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """deq(W) [N, K] in the scales' dtype: RNE(fl32(scale * q + bias)), bit-exact."""
    n, k = _check_weight(w, scales, biases, group_size, bits)
    if out is None:
        out = torch.empty((n, k), dtype=scales.dtype, device=w.device)
    _require(out.is_contiguous() and tuple(out.shape) == (n, k) and out.dtype == scales.dtype,
             "out must be a contiguous [N, K] tensor of the scales' dtype")
    dtype = _DTYPES.get(scales.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_dequantize(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                                        k, n, group_size, bits, dtype, _stream(w))
    _lib.check(st, ctx)
    return out


def _qmm_call(entry: str, x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
              biases: torch.Tensor, group_size: int, bits: int,
              out: torch.Tensor | None) -> torch.Tensor:
    n, k = _check_weight(w, scales, biases, group_size, bits)
    _require(x.is_cuda and x.device == w.device, "x must be on the weight's device")
    _require(x.dim() >= 1 and x.shape[-1] == k, f"x's last dim must be K={k}, got {tuple(x.shape)}")
    _require(x.dtype == scales.dtype, f"x ({x.dtype}) and scales ({scales.dtype}) must share T")
    lead = tuple(x.shape[:-1])
    m = 1
    for d in lead:
        m *= d
    if not x.is_contiguous():
        x = x.contiguous()
    if out is None:
        out = torch.empty(lead + (n,), dtype=x.dtype, device=x.device)
    _require(out.is_contiguous() and tuple(out.shape) == lead + (n,) and out.dtype == x.dtype,
             "out must be a contiguous [..., N] tensor of x's dtype")
    if m == 0:
        return out
    dtype = _DTYPES.get(x.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = getattr(_lib.load(), entry)(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(x),
                                         _ptr(out), k, n, m, group_size, bits, dtype, _stream(x))
    _lib.check(st, ctx)
    return out


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True,
                     group_size: int = GROUP_SIZE, bits: int = BITS,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """y[..., N] = x[..., K] . deq(W)^T (MLX quantizedMM with transpose=true).

    3 <= M <= 16 rows with K % 128 == 0 run the few-row matrix-core kernel
    (17 <= M <= 32 its K split, where fewer than 512 row tiles allow it),
    other M <= 4 (and f32) the qGEMV kernel, larger M the MFMA qGEMM kernel,
    with K split over a per-stream workspace when its output tiles are too few
    to fill the GPU (deterministic; another fp32 summation order than qgemm)."""
    if not transpose:
        raise NotImplementedError("only transpose=true (y = x . deq(w)^T) is on the path")
    return _qmm_call("imq_qmm_t", x, w, scales, biases, group_size, bits, out)


def qgemv(x, w, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS, out=None):
    """The skinny-M kernel alone (1 <= M <= 16)."""
    return _qmm_call("imq_qgemv", x, w, scales, biases, group_size, bits, out)


def qgemm(x, w, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS, out=None):
    """The MFMA kernel alone (any M)."""
    return _qmm_call("imq_qgemm", x, w, scales, biases, group_size, bits, out)


def _epi_args(x, w, scales, biases, group_size, bits):
    n, k = _check_weight(w, scales, biases, group_size, bits)
    _require(x.is_cuda and x.device == w.device, "x must be on the weight's device")
    _require(x.dim() >= 1 and x.shape[-1] == k, f"x's last dim must be K={k}, got {tuple(x.shape)}")
    _require(x.dtype == scales.dtype, f"x ({x.dtype}) and scales ({scales.dtype}) must share T")
    lead = tuple(x.shape[:-1])
    m = 1
    for d in lead:
        m *= d
    return n, k, m, lead, (x if x.is_contiguous() else x.contiguous())


def _f32_out(out, shape, device, what):
    if out is None:
        return torch.empty(shape, dtype=torch.float32, device=device)
    _require(out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == shape,
             f"{what} must be a contiguous float32 tensor of shape {shape}")
    return out


def cast_prescale(x: torch.Tensor, scale: float = 16.0, dtype: torch.dtype = torch.float16,
                  out: torch.Tensor | None = None,
                  scale_dev: torch.Tensor | None = None) -> torch.Tensor:
    """T y = T(x / scale) for float32 x (``AttentionUtils.compiledPreScale``,
    ``Sources/ImarelloDiT/AttentionUtils.swift:155-160``): bit-exact, one HIP kernel.
    ``scale_dev`` (a one-element float32 device tensor, e.g. ``dynamic_scale``'s)
    replaces ``scale`` and is read when the kernel runs."""
    _require(x.is_cuda and x.dtype == torch.float32, "x must be a float32 HIP tensor")
    _require(dtype in (torch.float16, torch.bfloat16), f"dtype {dtype}: float16 or bfloat16")
    x = x if x.is_contiguous() else x.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
    _require(out.dtype == dtype and out.is_contiguous() and out.shape == x.shape
             and out.device == x.device, f"out must be a contiguous {dtype} tensor shaped like x")
    sd = _scale_dev(scale_dev, x.device)
    ctx = context(x.device)
    with torch.cuda.device(x.device):
        st = _lib.load().imq_cast_prescale_ex(ctx, _ptr(x), _ptr(out), x.numel(), float(scale), sd,
                                              _DTYPES[dtype], _stream(x))
    _lib.check(st, ctx)
    return out


def _scale_dev(t: torch.Tensor | None, device) -> ctypes.c_void_p:
    if t is None:
        return ctypes.c_void_p(0)
    _require(t.is_cuda and t.device == device and t.dtype == torch.float32 and t.numel() == 1,
             "scale_dev must be a one-element float32 tensor on x's device")
    return _ptr(t)


def dynamic_scale(x: torch.Tensor, target: float = 64.0,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """One-element float32 device tensor max(amax|x| / target, 1): the per-tensor
    dynamic scale of ``applyLinearCore`` (``AttentionUtils.swift:173-178,208-210``,
    ``linearDynamicScaleTarget`` 64), computed on the device without a host sync."""
    _require(x.is_cuda and x.dtype == torch.float32, "x must be a float32 HIP tensor")
    x = x if x.is_contiguous() else x.contiguous()
    if out is None:
        out = torch.empty(1, dtype=torch.float32, device=x.device)
    _scale_dev(out, x.device)
    ctx = context(x.device)
    with torch.cuda.device(x.device):
        st = _lib.load().imq_dynamic_scale(ctx, _ptr(x), x.numel(), float(target), _ptr(out),
                                           _stream(x))
    _lib.check(st, ctx)
    return out


def qmm_postscale(x, w, scales, biases, scale: float, group_size: int = GROUP_SIZE,
                  bits: int = BITS, out=None, out_dtype: torch.dtype = torch.float32,
                  scale_dev: torch.Tensor | None = None) -> torch.Tensor:
    """y = float(T(x . deq(W)^T)) * scale in one kernel (the reference's qmm +
    dd_cast_postscale, ``DirectDiTKernels.swift:199-209``).  ``out_dtype`` float16
    keeps the result in f16 without the f32 upcast (``compiledPostScaleF16``,
    ``AttentionUtils.swift:166-171``: f16(y * f16(scale)), the f16 qmm only);
    ``scale_dev`` replaces ``scale`` (read when the kernel runs)."""
    n, k, m, lead, x = _epi_args(x, w, scales, biases, group_size, bits)
    _require(out_dtype in (torch.float32, torch.float16), "out_dtype: float32 or float16")
    if out is None:
        out = torch.empty(lead + (n,), dtype=out_dtype, device=x.device)
    _require(out.dtype == out_dtype and out.is_contiguous() and tuple(out.shape) == lead + (n,),
             f"out must be a contiguous {out_dtype} tensor of shape {lead + (n,)}")
    sd = _scale_dev(scale_dev, x.device)
    dtype = _DTYPES.get(x.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_qmm_postscale_ex(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(x),
                                              _ptr(out), _DTYPES[out_dtype], k, n, m,
                                              float(scale), sd, group_size, bits, dtype,
                                              _stream(x))
    _lib.check(st, ctx)
    return out


def qmm_gate_add(x, w, scales, biases, residual: torch.Tensor, gate: torch.Tensor, scale: float,
                 group_size: int = GROUP_SIZE, bits: int = BITS, out=None) -> torch.Tensor:
    """float32 y = residual + gate * float(T(x . deq(W)^T)) * scale in one kernel
    (qmm + dd_gate_add, ``DirectDiTKernels.swift:211-224``); ``out=residual``
    updates the residual stream in place."""
    n, k, m, lead, x = _epi_args(x, w, scales, biases, group_size, bits)
    _require(residual.dtype == torch.float32 and residual.is_contiguous()
             and tuple(residual.shape) == lead + (n,), "residual must be float32 [..., N]")
    _require(gate.dtype == torch.float32 and gate.is_contiguous() and tuple(gate.shape) == (n,),
             "gate must be float32 [N]")
    out = _f32_out(out, lead + (n,), x.device, "out")
    dtype = _DTYPES.get(x.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_qmm_gate_add(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(x),
                                          _ptr(residual), _ptr(gate), _ptr(out), k, n, m,
                                          float(scale), group_size, bits, dtype, _stream(x))
    _lib.check(st, ctx)
    return out


def dequantize_rows(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                    rows: torch.Tensor, group_size: int = GROUP_SIZE, bits: int = BITS,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """deq(W)[rows] [len(rows), K] in the scales' dtype: ``DirectTEEncoder.embedRow``
    (``DirectTEEncoder.swift:106-123``) for a batch of token ids, one launch.
    Ids are checked against [0, N) here (the kernel clamps them)."""
    n, k = _check_weight(w, scales, biases, group_size, bits)
    _require(rows.dim() == 1 and rows.dtype in (torch.int32, torch.int64), "rows: 1-D integer ids")
    if rows.numel():
        lo, hi = int(rows.min()), int(rows.max())
        _require(0 <= lo and hi < n, f"ids must lie in [0, {n}), got [{lo}, {hi}]")
    ids = rows.to(device=w.device, dtype=torch.int32).contiguous()
    if out is None:
        out = torch.empty((ids.numel(), k), dtype=scales.dtype, device=w.device)
    _require(out.dtype == scales.dtype and out.is_contiguous() and tuple(out.shape) == (ids.numel(), k),
             f"out must be a contiguous {scales.dtype} [{ids.numel()}, {k}] tensor")
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_dequantize_rows(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(ids),
                                             ids.numel(), _ptr(out), k, n, group_size, bits,
                                             _DTYPES[scales.dtype], _stream(ids))
    _lib.check(st, ctx)
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5,
            out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row RMSNorm to T: x * rsqrt(mean(x^2) + eps) * weight with an fp32 sum of
    squares and fp32 weight; x float32 (the DiT's residual, ``dd_rmsnorm_pitched``,
    ``DirectDiTKernels.swift:61-99``, eps 1e-5) or T itself (the text encoder's
    ``dq_rmsnorm``, ``DirectGlueKernels.swift:14-49``, eps 1e-6)."""
    _require(x.is_cuda and x.dtype in (torch.float32, torch.bfloat16, torch.float16),
             "x must be a float32, bfloat16 or float16 HIP tensor")
    out_dtype = out_dtype or (x.dtype if x.dtype != torch.float32 else torch.bfloat16)
    _require(out_dtype in (torch.bfloat16, torch.float16), "out_dtype: bfloat16 or float16")
    x = x if x.is_contiguous() else x.contiguous()
    cols = x.shape[-1]
    _require(weight.dtype == torch.float32 and weight.is_contiguous() and weight.numel() == cols
             and weight.device == x.device, f"weight must be float32 [{cols}] on x's device")
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    _require(out.dtype == out_dtype and out.is_contiguous() and out.shape == x.shape,
             f"out must be a contiguous {out_dtype} tensor shaped like x")
    ctx = context(x.device)
    with torch.cuda.device(x.device):
        st = _lib.load().imq_rmsnorm(ctx, _ptr(x), _DTYPES[x.dtype], _ptr(weight), _ptr(out),
                                     _DTYPES[out_dtype], x.numel() // cols, cols, float(eps),
                                     _stream(x))
    _lib.check(st, ctx)
    return out


def qmm_add(x, w, scales, biases, residual: torch.Tensor, group_size: int = GROUP_SIZE,
            bits: int = BITS, out=None) -> torch.Tensor:
    """T y = T(float(residual) + float(T(x . deq(W)^T))) in one kernel: the text
    encoder's qmm + dq_add (``DirectTEEncoder.swift:390-392,409-411``,
    ``DirectGlueKernels.swift:88-96``); residual has x's dtype, ``out=residual``
    updates it in place."""
    n, k, m, lead, x = _epi_args(x, w, scales, biases, group_size, bits)
    _require(residual.dtype == x.dtype and residual.is_contiguous()
             and tuple(residual.shape) == lead + (n,), f"residual must be {x.dtype} [..., N]")
    if out is None:
        out = torch.empty(lead + (n,), dtype=x.dtype, device=x.device)
    _require(out.dtype == x.dtype and out.is_contiguous() and tuple(out.shape) == lead + (n,),
             f"out must be a contiguous {x.dtype} tensor of shape {lead + (n,)}")
    dtype = _DTYPES.get(x.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_qmm_add(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(x),
                                     _ptr(residual), _ptr(out), k, n, m, group_size, bits, dtype,
                                     _stream(x))
    _lib.check(st, ctx)
    return out


def qmm_swiglu(x, w, scales, biases, width: int, gate_row: int, up_row: int,
               in_scale: float = 1.0, out_scale: float = 1.0, group_size: int = GROUP_SIZE,
               bits: int = BITS, out=None) -> torch.Tensor:
    """y[..., j] = T(g * sigmoid(g) * u * out_scale) for j < width, with g and u
    the T-rounded products of x with weight rows gate_row + j and up_row + j
    times in_scale (qmm + dd_swiglu_pitched, ``DirectDiTKernels.swift:137-157``).
    ``out`` may be a column slice of a wider 2-D buffer (unit column stride)."""
    n, k, m, lead, x = _epi_args(x, w, scales, biases, group_size, bits)
    if out is None:
        out = torch.empty(lead + (width,), dtype=x.dtype, device=x.device)
    _require(out.dtype == x.dtype and tuple(out.shape) == lead + (width,) and out.stride(-1) == 1,
             "out must be [..., width] of x's dtype with unit column stride")
    if out.dim() >= 2:
        ldy = out.stride(-2)
        _require(all(out.stride(i) == out.stride(i + 1) * out.shape[i + 1]
                     for i in range(out.dim() - 2)), "out's leading dims must be packed")
    else:
        ldy = width
    dtype = _DTYPES.get(x.dtype, -1)
    ctx = context(w.device)
    with torch.cuda.device(w.device):
        st = _lib.load().imq_qmm_swiglu(ctx, _ptr(w), _ptr(scales), _ptr(biases), _ptr(x),
                                        _ptr(out), ldy, k, n, m, width, gate_row, up_row,
                                        float(in_scale), float(out_scale), group_size, bits,
                                        dtype, _stream(x))
    _lib.check(st, ctx)
    return out


_ENTRIES = {"qmm_t": _lib.IMQ_ENTRY_QMM_T, "qgemm": _lib.IMQ_ENTRY_QGEMM,
            "qgemv": _lib.IMQ_ENTRY_QGEMV, "fused": _lib.IMQ_ENTRY_FUSED,
            "swiglu": _lib.IMQ_ENTRY_SWIGLU}


def qmm_plan(m: int, n: int, k: int, dtype: torch.dtype = torch.bfloat16, entry: str = "qmm_t",
             device=None) -> dict:
    """The kernel, tile height and K split a call of ``entry`` ("qmm_t", "qgemm",
    "qgemv", "fused": the post-scale and gated-residual stages over n weight
    rows, "swiglu": n = 2 width) would run for these sizes, without launching
    anything (``imq_qmm_plan``)."""
    _require(entry in _ENTRIES, f"entry must be one of {sorted(_ENTRIES)}")
    ctx = context(device)
    out = _lib.Plan()
    _lib.check(_lib.load().imq_qmm_plan(ctx, _ENTRIES[entry], k, n, m, _DTYPES.get(dtype, -1),
                                        ctypes.byref(out)), ctx)
    return {"kernel": _lib.KERNEL_NAMES[out.kernel], "tile_rows": out.tile_rows,
            "tile_cols": out.tile_cols,
            "splits": out.splits, "workspace_bytes": out.workspace_bytes}


@dataclass
class Q:
    """A resident packed projection, the reference's ``Q(w:s:b:n:k:)``
    (``Sources/ImarelloDirect/DirectDiTStep.swift:278-284``)."""

    w: torch.Tensor
    s: torch.Tensor
    b: torch.Tensor
    n: int
    k: int


def qmm(q: Q, x: torch.Tensor, x_off: int, y: torch.Tensor, y_off: int, m: int) -> None:
    """``DirectDiTStep.qmm``: y rows [y_off, y_off + m) = x rows [x_off, x_off + m) . deq(W)^T.

    The reference binds x and y with byte offsets (row halves,
    ``DirectDiTStep.swift:573-580,597-611``); here offsets are in rows of the
    2-D buffers x [*, K] and y [*, N]."""
    _require(x.dim() == 2 and y.dim() == 2 and x.shape[1] == q.k and y.shape[1] == q.n,
             "x must be [*, K] and y [*, N]")
    _require(0 <= x_off and x_off + m <= x.shape[0] and 0 <= y_off and y_off + m <= y.shape[0],
             "row range out of bounds")
    quantized_matmul(x[x_off:x_off + m], q.w, q.s, q.b, out=y[y_off:y_off + m])


class QuantizedLinear:
    """Bias-free affine 4-bit Linear (every Linear on the path is bias-free,
    ``Sources/ImarelloDiT/AttentionUtils.swift:223-228``); forward = quantized_matmul."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = GROUP_SIZE, bits: int = BITS):
        _check_weight(weight, scales, biases, group_size, bits)
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits

    @property
    def in_features(self) -> int:
        return self.weight.shape[1] * 8

    @property
    def out_features(self) -> int:
        return self.weight.shape[0]

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return quantized_matmul(x, self.weight, self.scales, self.biases, True,
                                self.group_size, self.bits)

    def dequantized(self) -> torch.Tensor:
        return dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits)


def apply_linear(linear: QuantizedLinear, x: torch.Tensor, scale: float = 16.0,
                 output_f16: bool = False, dynamic_target: float | None = None) -> torch.Tensor:
    """y = linear(x) through the f16 sandwich of ``AttentionUtils.applyLinear`` /
    ``applyLinearCore`` with ``linearF16`` on (``Sources/ImarelloDiT/AttentionUtils.swift:140-150,
    198-230``): x / scale rounded to f16 (``cast_prescale``), then the f16 qmm and the
    x scale rescale in one kernel (``qmm_postscale``).  x is float32 of any leading shape; the
    linear's scales and biases must be float16 (the DiT pack casts them at load,
    ``TransformerWeights.swift:40-54``, exact for that pack; ``load_qlinear(..., IMQ_F16)``
    does the same).

    * ``scale``: the static scale (``AttentionTuning.linearF16Scale``, 16);
    * ``dynamic_target``: the per-tensor dynamic scale instead (``linearDynamicScale``:
      max(amax|x| / target, 1), ``linearDynamicScaleTarget`` 64), computed on the device;
    * ``output_f16``: an f16 result without the f32 upcast (``outputF16`` /
      ``linearF16FullEpilogue``, ``compiledPostScaleF16``), else float32.

    ``linearChunkedSequence`` (``:233-261``) runs this in 512-row chunks to bound MLX
    temporaries; rows are independent, so one launch over all rows gives the same values
    (with the dynamic scale, the reference's chunks would each take their own amax)."""
    _require(linear.scales.dtype == torch.float16,
             f"the f16 path needs float16 scales and biases, got {linear.scales.dtype}")
    sd = dynamic_scale(x, dynamic_target) if dynamic_target is not None else None
    x16 = cast_prescale(x, scale, torch.float16, scale_dev=sd)
    return qmm_postscale(x16, linear.weight, linear.scales, linear.biases, scale,
                         linear.group_size, linear.bits,
                         out_dtype=torch.float16 if output_f16 else torch.float32, scale_dev=sd)

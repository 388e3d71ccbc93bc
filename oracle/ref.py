"""numpy restatement of the affine 4-bit quantized linear path (test oracle).

TEST INFRASTRUCTURE ONLY -- see the package docstring.  All bf16 values are
carried as ``uint16`` bit patterns; f16 and f32 values as numpy float16 /
float32 arrays (the ``*_as`` functions).
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 64
BITS = 4
PACK = 8  # codes per uint32 word


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """bf16 bits -> float32 (``DirectTEEncoder.swift:44-46``: bits << 16)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(v: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, RNE by the integer formula of
    ``DirectTEEncoder.swift:39-43`` (wrapping add, no NaN special case)."""
    bits = np.asarray(v, dtype=np.float32).view(np.uint32)
    rounded = bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def f64_to_bf16(v: np.ndarray) -> np.ndarray:
    """Correctly rounded float64 -> bf16 (RNE), via round-to-odd at float32."""
    v = np.asarray(v, dtype=np.float64)
    f = v.astype(np.float32)
    bits = f.view(np.uint32).copy()
    inexact = (f.astype(np.float64) != v) & np.isfinite(v)
    away = np.abs(f.astype(np.float64)) > np.abs(v)
    bits = np.where(inexact & away, bits - np.uint32(1), bits)
    bits = np.where(inexact, bits | np.uint32(1), bits)
    return f32_to_bf16(bits.view(np.float32))


def unpack_codes(w: np.ndarray) -> np.ndarray:
    """uint32 [N, K/8] -> uint8 codes [N, K]; code k = nibble k%8 of word k/8,
    low nibble first (``DirectTEEncoder.swift:116-118``)."""
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(PACK, dtype=np.uint32) * np.uint32(4))
    codes = (w[..., None] >> shifts) & np.uint32(0xF)
    return codes.reshape(*w.shape[:-1], w.shape[-1] * PACK).astype(np.uint8)


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """uint8 codes [N, K] (values 0..15) -> uint32 [N, K/8], low nibble first."""
    codes = np.asarray(codes, dtype=np.uint32)
    n, k = codes.shape
    assert k % PACK == 0
    c = codes.reshape(n, k // PACK, PACK)
    shifts = (np.arange(PACK, dtype=np.uint32) * np.uint32(4))
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def dequantize(w: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """bf16 bits [N, K] = RNE_bf16(fl32(s*q + b)) (``DirectTEEncoder.swift:106-123``).

    Two float32 operations, like the reference's ``scale * q + bias`` on Float:
    the product is exact unless it overflows (then +-inf), the sum rounds once."""
    q = unpack_codes(w).astype(np.float32)
    n, k = q.shape
    assert k % GROUP_SIZE == 0
    s = np.repeat(bf16_to_f32(scales), GROUP_SIZE, axis=-1).reshape(n, k)
    b = np.repeat(bf16_to_f32(biases), GROUP_SIZE, axis=-1).reshape(n, k)
    with np.errstate(over="ignore", invalid="ignore"):
        return f32_to_bf16(s * q + b)


def qmm_t_f64(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """Unrounded float64 y = x . deq(w)^T with the bit-exact bf16 dequant."""
    xd = bf16_to_f32(x).astype(np.float64)
    wd = bf16_to_f32(dequantize(w, scales, biases)).astype(np.float64)
    return xd @ wd.T


def qmm_t(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """bf16 bits y[M, N] = RNE_bf16(x . deq(w)^T) -- the parity oracle
    (``DirectQmmSpike.swift:55-58``: quantizedMM with transpose=true)."""
    return f64_to_bf16(qmm_t_f64(x, w, scales, biases))


def dequantize_as(w: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                  dtype) -> np.ndarray:
    """deq(W) [N, K] in T = float16 or float32, with scales and biases given in T:
    RNE_T(fl32(fl32(s*q) + b)); for float32 the weight is fl32(fl32(s*q) + b)
    itself.  Two rounded float32 operations, as in ``dequantize``; with f16
    scales the product is exact, with f32 scales it is not.

    The element type of the reference's DiT kernels (``affine_qmm_t_float16_t``,
    ``DirectDiTStep.swift:82-85``, scales precast to f16 by
    ``TransformerWeights.swift:40-54``) and of its conditioner kernels
    (``affine_qmm_t_float``, f32 scales, ``DirectConditioner.swift:48,75-84``).
    numpy's float32 -> float16 cast rounds to nearest even."""
    dtype = np.dtype(dtype)
    assert dtype in (np.float16, np.float32)
    q = unpack_codes(w).astype(np.float32)
    n, k = q.shape
    assert k % GROUP_SIZE == 0
    s = np.repeat(np.asarray(scales).astype(np.float32), GROUP_SIZE, axis=-1).reshape(n, k)
    b = np.repeat(np.asarray(biases).astype(np.float32), GROUP_SIZE, axis=-1).reshape(n, k)
    with np.errstate(over="ignore", invalid="ignore"):
        return (s * q + b).astype(dtype)


def qmm_t_as(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray,
             dtype) -> np.ndarray:
    """y[M, N] = RNE_T(x . deq_T(w)^T accumulated in float64), T = float16 or
    float32 (numpy's float64 -> float16 / float32 casts round once, to nearest
    even)."""
    dtype = np.dtype(dtype)
    xd = np.asarray(x).astype(np.float64)
    wd = dequantize_as(w, scales, biases, dtype).astype(np.float64)
    return (xd @ wd.T).astype(dtype)


def error_stats_values(y: np.ndarray, o: np.ndarray) -> dict:
    """error_stats for float16 / float32 outputs (values, not bit patterns)."""
    stats = _stats(np.asarray(y).astype(np.float64), np.asarray(o).astype(np.float64))
    stats["bit_exact_frac"] = float(np.mean(np.asarray(y) == np.asarray(o))) if o.size else 1.0
    return stats


def error_stats(y_bits: np.ndarray, oracle_bits: np.ndarray) -> dict:
    """Tolerance metrics: MAE, normwise max error, floored elementwise error."""
    y = bf16_to_f32(y_bits).astype(np.float64)
    o = bf16_to_f32(oracle_bits).astype(np.float64)
    stats = _stats(y, o)
    stats["bit_exact_frac"] = float(np.mean(y_bits == oracle_bits)) if o.size else 1.0
    return stats


def _stats(y: np.ndarray, o: np.ndarray) -> dict:
    d = np.abs(y - o)
    omax = float(np.max(np.abs(o))) if o.size else 0.0
    rms = float(np.sqrt(np.mean(o * o))) if o.size else 0.0
    floor = np.maximum(np.abs(o), 1e-3 * rms) if o.size else o
    # Cosine similarity of the flattened outputs: the reference's own qmm
    # parity criterion is cosine >= 0.99999 (DirectQmmSpike.swift:141-153).
    ny, no = float(np.linalg.norm(y)), float(np.linalg.norm(o))
    cosine = float(np.dot(y.ravel(), o.ravel()) / (ny * no)) if ny > 0 and no > 0 else \
        (1.0 if ny == no else 0.0)
    return {
        "cosine": cosine,
        "mae": float(np.mean(d)) if d.size else 0.0,
        "max_abs": float(np.max(d)) if d.size else 0.0,
        "max_rel_normwise": float(np.max(d) / omax) if d.size and omax > 0 else 0.0,
        "max_rel_floored": float(np.max(d / np.where(floor > 0, floor, 1.0))) if d.size else 0.0,
    }


# ------------------------------------------------------------- glue stages
def glue_prescale(x: np.ndarray, scale: float, dtype: str) -> np.ndarray:
    """AttentionUtils.compiledPreScale (Sources/ImarelloDiT/AttentionUtils.swift:155-160):
    ``(x / s).asType(T)`` on float32 x -- the fp32 quotient (IEEE, correctly
    rounded), then RNE to T.  Returns float16 values ("f16") or bf16 bits ("bf16")."""
    q = (np.asarray(x, dtype=np.float32) / np.float32(scale)).astype(np.float32)
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return q.astype(np.float16)
    return f32_to_bf16(q)


# The reference's post-qmm glue kernels (Sources/ImarelloDirect/DirectDiTKernels.swift)
# on the T output of a qmm, in fp32 (the Metal kernels compute in float).
# `y_t` is the qmm output as float32 values of T.

def glue_postscale(y_t: np.ndarray, scale: float) -> np.ndarray:
    """dd_cast_postscale (DirectDiTKernels.swift:199-209): float(y) * s."""
    return (np.asarray(y_t, dtype=np.float32) * np.float32(scale)).astype(np.float32)


def glue_postscale_f16(y_f16: np.ndarray, scale: float) -> np.ndarray:
    """AttentionUtils.compiledPostScaleF16 (Sources/ImarelloDiT/AttentionUtils.swift:166-171):
    ``y * s.asType(.float16)`` on the f16 qmm output -- the scale rounded to f16,
    then the f16 product, correctly rounded once (the product of two f16 values
    is exact in float32).  Returns float16 values."""
    s16 = np.float32(np.float16(np.float32(scale)))
    with np.errstate(over="ignore"):
        return (np.asarray(y_f16, dtype=np.float16).astype(np.float32) * s16).astype(np.float16)


def dynamic_scale(x: np.ndarray, target: float) -> np.float32:
    """AttentionUtils.compiledDynamicScale (AttentionUtils.swift:173-178):
    ``maximum(abs(x).max() / target, 1)`` in float32 -- the fp32 quotient
    (correctly rounded), at least 1; a NaN anywhere in x gives NaN.  An empty x
    has amax 0 and so scale 1."""
    a = np.abs(np.asarray(x, dtype=np.float32)).ravel()
    amax = np.float32(0.0) if a.size == 0 else np.float32(np.max(a))
    q = np.float32(amax / np.float32(target))
    return q if np.isnan(q) else np.float32(max(q, np.float32(1.0)))


def glue_gate_add(y_t: np.ndarray, residual: np.ndarray, gate: np.ndarray,
                  scale: float) -> np.ndarray:
    """dd_gate_add (DirectDiTKernels.swift:211-224): fma(gate[j], float(v) * s, x)."""
    v = (np.asarray(y_t, dtype=np.float32) * np.float32(scale)).astype(np.float64)
    exact = np.asarray(gate, np.float64)[None, :] * v + np.asarray(residual, np.float64)
    return exact.astype(np.float32)


def glue_add_t(y_t: np.ndarray, r_t: np.ndarray, dtype: str) -> np.ndarray:
    """dq_add (Sources/ImarelloDirect/DirectGlueKernels.swift:88-96) after a qmm:
    T(float(r) + float(y)) -- the float32 sum of two T values, rounded to T.
    y_t, r_t are float32 values of T; returns float16 values ("f16") or bf16
    bits ("bf16")."""
    s = (np.asarray(r_t, dtype=np.float32) + np.asarray(y_t, dtype=np.float32)).astype(np.float32)
    if dtype == "f16":
        with np.errstate(over="ignore"):
            return s.astype(np.float16)
    return f32_to_bf16(s)


def glue_swiglu(g_t: np.ndarray, u_t: np.ndarray, in_scale: float, out_scale: float) -> np.ndarray:
    """dd_swiglu_pitched (DirectDiTKernels.swift:137-157): g, u = float(.) * inScale;
    g * sigmoid(g) * u * outScale, as float64 (to be rounded to T by the caller)."""
    g = np.asarray(g_t, np.float64) * np.float32(in_scale)
    u = np.asarray(u_t, np.float64) * np.float32(in_scale)
    return g / (1.0 + np.exp(-g)) * u * np.float32(out_scale)


def rmsnorm_rows(x: np.ndarray, w: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """Row RMSNorm in float64: x * 1/sqrt(mean(x^2) + eps) * w (the shape of the
    reference's dd_rmsnorm_pitched, DirectDiTKernels.swift:61-99, eps 1e-5 at
    DirectDiTStep.swift:416); the caller rounds to T."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(w, np.float64)


# The conditioning chain of DirectConditioner.stepConditioning
# (Sources/ImarelloDirect/DirectConditioner.swift:152-213), f32 throughout.

def cond_sinusoid(t: np.ndarray, sin_dim: int) -> np.ndarray:
    """DirectConditioner.sinusoid (:152-166) for each t: freq_i = expf(-logf(10000)
    * i / half), arg = t * freq_i, [cosf(arg) | sinf(arg)].  Every float operation
    rounds to float32 in the reference's order; the transcendental functions are
    evaluated in float64 and rounded once (correctly rounded float32 results)."""
    t = np.asarray(t, dtype=np.float32).reshape(-1)
    half = sin_dim // 2
    ln = np.float32(np.log(np.float64(10000.0)))
    i = np.arange(half, dtype=np.float32)
    e = ((-ln) * i).astype(np.float32) / np.float32(half)
    freq = np.exp(e.astype(np.float64)).astype(np.float32)
    arg = (t[:, None] * freq[None, :]).astype(np.float32).astype(np.float64)
    return np.concatenate([np.cos(arg).astype(np.float32), np.sin(arg).astype(np.float32)], axis=1)


def silu_f32(v: np.ndarray) -> np.ndarray:
    """dd_silu_f32 (DirectDiTKernels.swift:176-184): v / (1 + exp(-v)), evaluated in
    float64 and rounded once to float32."""
    vd = np.asarray(v, dtype=np.float32).astype(np.float64)
    with np.errstate(over="ignore"):
        return (vd / (1.0 + np.exp(-vd))).astype(np.float32)


def cond_chain(t: np.ndarray, l1, l2, heads, head_rows=None):
    """stepConditioning (:168-213) on the CPU for timesteps t: l1, l2, heads are
    (w uint32, scales f32, biases f32) triples; returns (temb, heads_out), each
    qmm the f32 oracle qmm (f32 dequant, float64 accumulation, one rounding).
    head_rows restricts the heads' output columns to those weight rows."""
    sin = cond_sinusoid(t, l1[0].shape[1] * 8)
    t1 = silu_f32(qmm_t_as(sin, *l1, np.float32))
    temb = qmm_t_as(t1, *l2, np.float32)
    hw, hs, hb = heads
    if head_rows is not None:
        hw, hs, hb = hw[head_rows], hs[head_rows], hb[head_rows]
    return temb, qmm_t_as(silu_f32(temb), hw, hs, hb, np.float32)


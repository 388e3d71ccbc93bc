"""The text encoder's quantized-linear layer halves (include/imq_te.h) from Python.

Mirrors ``DirectTEEncoder.encodeLayer`` (``Sources/ImarelloDirect/DirectTEEncoder.swift:364-412``)
over the layers ``DirectTEForward.loadLayers`` uploads (``DirectTEForward.swift:97-138``):
``attn_in`` is RMSNorm + the q/k/v projections (one launch), ``attn_out_mlp`` is
o_proj + dq_add, RMSNorm, gate/up with dq_silu_mul (one launch) and down_proj +
dq_add.  The attention core between them (per-head norms, RoPE, attention) is
the caller's.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .ops import Q, _require, context, device_index
from .step import _qweight

# Qwen3 4B text encoder (DirectTEForward.swift:12-22).
HIDDEN, N_HEADS, N_KV, HEAD_DIM, INTER, N_LAYERS, EPS = 2560, 32, 8, 128, 9728, 27, 1e-6


@dataclass
class TeLayer:
    """One layer's resident projections and norm weights: q/k/v and gate/up
    concatenated along N (rows q | k | v, gate | up)."""

    qkv: Q
    o: Q
    gate_up: Q
    down: Q
    norm_in: torch.Tensor    # input_layernorm.weight, float32 [hidden]
    norm_post: torch.Tensor  # post_attention_layernorm.weight, float32 [hidden]


def _rand_q(n, k, dtype, g, dev) -> Q:
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev, generator=g)
    unit = 1.0 / (4.0 * k ** 0.5)
    s = torch.randn((n, k // 64), device=dev, generator=g).abs() * unit
    b = -8.0 * s + torch.randn((n, k // 64), device=dev, generator=g) * (0.1 * unit)
    return Q(w=w, s=s.to(dtype), b=b.to(dtype), n=n, k=k)


def random_te_layers(n_layers: int = 1, hidden: int = HIDDEN, nq: int = N_HEADS * HEAD_DIM,
                     nkv: int = N_KV * HEAD_DIM, inter: int = INTER,
                     dtype: torch.dtype = torch.bfloat16, seed: int = 0,
                     device=None) -> list[TeLayer]:
    """Synthetic layers of the given shapes (scale law of ``step.random_projections``:
    outputs at the scale of the normalized input) and norm weights 1 + N(0, 0.1)."""
    dev = torch.device("cuda", device_index(device))
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for _ in range(n_layers):
        out.append(TeLayer(
            qkv=_rand_q(nq + 2 * nkv, hidden, dtype, g, dev), o=_rand_q(hidden, nq, dtype, g, dev),
            gate_up=_rand_q(2 * inter, hidden, dtype, g, dev), down=_rand_q(hidden, inter, dtype, g, dev),
            norm_in=1.0 + 0.1 * torch.randn(hidden, device=dev, generator=g),
            norm_post=1.0 + 0.1 * torch.randn(hidden, device=dev, generator=g)))
    return out


def load_te_layers(st, n_layers: int = N_LAYERS, prefix: str = "layers",
                   scales: torch.dtype = torch.bfloat16, device=None) -> list[TeLayer]:
    """``DirectTEForward.loadLayers`` (``:97-138``) from an opened ``SafetensorsSet``:
    ``<prefix>.<i>.self_attn.{q,k,v,o}_proj``, ``mlp.{gate,up,down}_proj`` with their
    scales and biases kept in ``scales`` (the TE's raw bf16 by default), the norm
    weights as float32."""
    from .weights import load_qlinear, load_qlinear_cat
    out = []
    for i in range(n_layers):
        p = f"{prefix}.{i}"
        qkv = load_qlinear_cat(st, [f"{p}.self_attn.{n}_proj" for n in "qkv"], scales, device)
        gate_up = load_qlinear_cat(st, [f"{p}.mlp.gate_proj", f"{p}.mlp.up_proj"], scales, device)
        out.append(TeLayer(
            qkv=qkv, o=load_qlinear(st, f"{p}.self_attn.o_proj", scales, device), gate_up=gate_up,
            down=load_qlinear(st, f"{p}.mlp.down_proj", scales, device),
            norm_in=st.upload(f"{p}.input_layernorm.weight", torch.float32, device),
            norm_post=st.upload(f"{p}.post_attention_layernorm.weight", torch.float32, device)))
    return out


class TeLayerWeights(ctypes.Structure):
    """imq_te_layer_weights."""
    _fields_ = [("qkv", _lib.QWeight), ("o", _lib.QWeight), ("gate_up", _lib.QWeight),
                ("down", _lib.QWeight), ("norm_in", ctypes.c_void_p), ("norm_post", ctypes.c_void_p)]


class TextEncoderLayers:
    """A created plan over resident layers (kept alive here)."""

    def __init__(self, layers: list[TeLayer], max_rows: int = 512, eps: float = EPS, device=None):
        self.layers = layers
        self.device = torch.device("cuda", device_index(device))
        self.dtype = layers[0].qkv.s.dtype
        self.max_rows = max_rows
        self._L = _lib.load()
        self._ctx = context(self.device)
        arr = (TeLayerWeights * len(layers))()
        for i, l in enumerate(layers):
            for name in ("qkv", "o", "gate_up", "down"):
                setattr(arr[i], name, _qweight(getattr(l, name)))
            _require(l.norm_in.dtype == torch.float32 and l.norm_post.dtype == torch.float32,
                     "norm weights must be float32")
            arr[i].norm_in = l.norm_in.data_ptr()
            arr[i].norm_post = l.norm_post.data_ptr()
        out = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_te_create(self._ctx, arr, len(layers), max_rows, float(eps),
                                             ctypes.byref(out)), self._ctx)
        self._h = out
        dims = [ctypes.c_int() for _ in range(4)]
        _lib.check(self._L.imq_te_dims(self._h, *[ctypes.byref(d) for d in dims]), self._ctx)
        self.hidden, self.nq, self.nkv, self.inter = (d.value for d in dims)

    def close(self) -> None:
        if self._h:
            self._L.imq_te_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _rows(self, x: torch.Tensor, width: int, name: str) -> int:
        _require(x.dim() == 2 and x.shape[1] == width and x.dtype == self.dtype and x.is_contiguous()
                 and x.device == self.device,
                 f"{name} must be a contiguous {self.dtype} [rows, {width}] tensor on {self.device}")
        return x.shape[0]

    def attn_in(self, layer: int, x: torch.Tensor, qkv: torch.Tensor | None = None) -> torch.Tensor:
        """qkv [rows, nq + 2 nkv] (q | k | v columns) = RMSNorm(x) . [Wq; Wk; Wv]^T."""
        rows = self._rows(x, self.hidden, "x")
        width = self.nq + 2 * self.nkv
        if qkv is None:
            qkv = torch.empty((rows, width), dtype=self.dtype, device=self.device)
        _require(self._rows(qkv, width, "qkv") == rows, "qkv rows must match x")
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_te_attn_in(self._h, layer, ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(qkv.data_ptr()), rows,
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                       self._ctx)
        return qkv

    def attn_out_mlp(self, layer: int, x: torch.Tensor, attn_o: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
        """The layer output [rows, hidden] from its input x and the attention output
        attn_o [rows, nq]; ``out=x`` updates x in place."""
        rows = self._rows(x, self.hidden, "x")
        _require(self._rows(attn_o, self.nq, "attn_o") == rows, "attn_o rows must match x")
        if out is None:
            out = torch.empty_like(x)
        _require(self._rows(out, self.hidden, "out") == rows, "out rows must match x")
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_te_attn_out_mlp(
                self._h, layer, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(attn_o.data_ptr()),
                ctypes.c_void_p(out.data_ptr()), rows,
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), self._ctx)
        return out

"""The DiT's per-step conditioning chain (include/imq_cond.h) from Python.

Mirrors ``DirectConditioner`` (``Sources/ImarelloDirect/DirectConditioner.swift``):
``Conditioner.from_safetensors`` loads the projections the reference loads with
f32 scales and biases (``:75-95``), ``step_conditioning`` is
``stepConditioning(timesteps:)`` (``:168-213``) and returns the same per-step
pieces (``Flux2StepConditioning``: temb, the double blocks' img / txt
modulation triples, the single blocks' triple, norm_out's scale and shift).
All timesteps of a call run as rows of one pass on the device.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import Q, _require, context, device_index
from .step import _qweight

TIME_L1 = "time_guidance_embed.linear_1"
TIME_L2 = "time_guidance_embed.linear_2"
# The modulation heads in the order of their concatenation, with their rows in
# units of dim (DirectConditioner.swift:89-92).
HEADS = (("double_stream_modulation_img.linear", 6), ("double_stream_modulation_txt.linear", 6),
         ("single_stream_modulation.linear", 3), ("norm_out.linear", 2))


@dataclass
class StepConditioning:
    """``Flux2StepConditioning`` of one timestep (``DirectConditioner.swift:186-208``):
    each triple is three consecutive dim-wide slices of its head's output."""

    temb: torch.Tensor
    double_img: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
    double_txt: list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]
    single: tuple[torch.Tensor, torch.Tensor, torch.Tensor]
    out_scale: torch.Tensor
    out_shift: torch.Tensor


def split_heads(temb: torch.Tensor, heads: torch.Tensor, dim: int) -> StepConditioning:
    """One timestep's temb [dim] and concatenated head outputs [17 dim] as the
    reference's per-step structure (``triples(_:sets:)``, ``:186-197``)."""
    _require(heads.shape[-1] == 17 * dim, f"heads must be [{17 * dim}] for dim {dim}")

    def triples(base: int, sets: int):
        return [tuple(heads[base + (3 * i + j) * dim: base + (3 * i + j + 1) * dim]
                      for j in range(3)) for i in range(sets)]

    return StepConditioning(temb=temb, double_img=triples(0, 2), double_txt=triples(6 * dim, 2),
                            single=triples(12 * dim, 1)[0], out_scale=heads[15 * dim:16 * dim],
                            out_shift=heads[16 * dim:17 * dim])


def sinusoid(timesteps, sin_dim: int = 256) -> np.ndarray:
    """The chain's host sinusoid (``DirectConditioner.sinusoid``, ``:152-166``) as
    float32 [count, sin_dim]."""
    t = np.ascontiguousarray(np.asarray(timesteps, dtype=np.float32).reshape(-1))
    out = np.empty((t.size, sin_dim), dtype=np.float32)
    _lib.check(_lib.load().imq_cond_sinusoid(t.ctypes.data_as(ctypes.c_void_p), t.size, sin_dim,
                                             out.ctypes.data_as(ctypes.c_void_p)), None)
    return out


def random_conditioner(dim: int = 3072, sin_dim: int = 256, seed: int = 0,
                       device=None) -> tuple[Q, Q, Q]:
    """Synthetic time_guidance_embed.linear_1 [dim, sin_dim], linear_2 [dim, dim]
    and the concatenated heads [17 dim, dim], f32 scales and biases holding
    bf16 values (as the hub pack's bf16 parameters cast to f32): random packed
    words, scale = |N(0, 1)| / (4 sqrt(K)), bias = -8 scale + N(0, 1) / (40 sqrt(K))."""
    dev = torch.device("cuda", device_index(device))
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for n, k in ((dim, sin_dim), (dim, dim), (17 * dim, dim)):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev,
                          generator=g)
        unit = 1.0 / (4.0 * k ** 0.5)
        s = torch.randn((n, k // 64), device=dev, generator=g).abs() * unit
        b = -8.0 * s + torch.randn((n, k // 64), device=dev, generator=g) * (0.1 * unit)
        out.append(Q(w=w, s=s.bfloat16().float(), b=b.bfloat16().float(), n=n, k=k))
    return out[0], out[1], out[2]


class Conditioner:
    """A created conditioning chain over resident f32-parameter projections
    (kept alive here)."""

    def __init__(self, time_l1: Q, time_l2: Q, heads: Q, device=None):
        self.projections = (time_l1, time_l2, heads)
        self.device = torch.device("cuda", device_index(device))
        self.dim = time_l1.n
        self.sin_dim = time_l1.k
        self.n_heads = heads.n
        self._L = _lib.load()
        self._ctx = context(self.device)
        a, b, c = _qweight(time_l1), _qweight(time_l2), _qweight(heads)
        out = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_cond_create(self._ctx, ctypes.byref(a), ctypes.byref(b),
                                               ctypes.byref(c), ctypes.byref(out)), self._ctx)
        self._h = out

    @classmethod
    def from_safetensors(cls, st, device=None) -> "Conditioner":
        """The reference's loads (``DirectConditioner.swift:86-95``) from an opened
        ``SafetensorsSet``: f32 scales and biases, the heads concatenated."""
        from .weights import load_qlinear, load_qlinear_cat
        l1 = load_qlinear(st, TIME_L1, torch.float32, device)
        l2 = load_qlinear(st, TIME_L2, torch.float32, device)
        heads = load_qlinear_cat(st, [p for p, _ in HEADS], torch.float32, device)
        return cls(l1, l2, heads, device)

    def close(self) -> None:
        if self._h:
            self._L.imq_cond_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run(self, timesteps, temb: torch.Tensor | None = None,
            heads: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """temb [count, dim] and the concatenated heads [count, n_heads] for the
        timesteps, fp32 on the device (asynchronous on the current stream)."""
        t = np.ascontiguousarray(np.asarray(timesteps, dtype=np.float32).reshape(-1))
        _require(t.size > 0, "no timesteps")
        if temb is None:
            temb = torch.empty((t.size, self.dim), dtype=torch.float32, device=self.device)
        if heads is None:
            heads = torch.empty((t.size, self.n_heads), dtype=torch.float32, device=self.device)
        for name, buf, width in (("temb", temb, self.dim), ("heads", heads, self.n_heads)):
            _require(buf.dtype == torch.float32 and buf.is_contiguous() and buf.device == self.device
                     and tuple(buf.shape) == (t.size, width),
                     f"{name} must be a contiguous float32 [{t.size}, {width}] tensor on {self.device}")
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_cond_step_conditioning(
                self._h, t.ctypes.data_as(ctypes.c_void_p), t.size, ctypes.c_void_p(temb.data_ptr()),
                ctypes.c_void_p(heads.data_ptr()), stream), self._ctx)
        return temb, heads

    def step_conditioning(self, timesteps) -> list[StepConditioning]:
        """``stepConditioning(timesteps:)``: one ``StepConditioning`` per timestep."""
        _require(self.n_heads == 17 * self.dim,
                 f"the FLUX.2 heads are 17 dim rows; this chain has {self.n_heads}")
        temb, heads = self.run(timesteps)
        return [split_heads(temb[i], heads[i], self.dim) for i in range(temb.shape[0])]

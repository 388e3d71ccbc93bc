"""Whole-step replay of a DiT step's quantized linear layers (include/imq_step.h).

``DitStep`` mirrors the reference's ``DirectDiTStep`` call surface
(``Sources/ImarelloDirect/DirectDiTStep.swift``): created once over resident
projections (``loadBlocks``), per-step conditioning (``setStepConditioning``),
and ``run`` = ``encodeStep`` (one graph launch instead of ~25 encoders).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .ops import Q, _DTYPES, context, device_index
from .weights import dit_double_linears, dit_single_linears


@dataclass(frozen=True)
class DitDims:
    l_img: int = 4096
    l_txt: int = 512
    dim: int = 3072
    ff_inner: int = 9216
    n_double: int = 5
    n_single: int = 20

    @property
    def joint(self) -> int:
        return self.l_img + self.l_txt

    def projection_shapes(self) -> list[tuple[str, int, int]]:
        """(name, N, K) of every projection in the plan's order."""
        out = []
        for i in range(self.n_double):
            for name, n, k in dit_double_linears(self.dim, self.ff_inner, 2 * self.ff_inner):
                out.append((f"transformer_blocks.{i}.{name}", n, k))
        for i in range(self.n_single):
            for name, n, k in dit_single_linears(self.dim, 3 * self.dim + 2 * self.ff_inner,
                                                 self.dim + self.ff_inner):
                out.append((f"single_transformer_blocks.{i}.{name}", n, k))
        return out

    def rows_of(self, name: str) -> int:
        """M of a projection: image rows, text rows (double-block add_* /
        to_add_out / ff_context.*) or all joint rows (single blocks)."""
        if name.startswith("single_transformer_blocks."):
            return self.joint
        txt = (".add_", ".to_add_out", ".ff_context.")
        return self.l_txt if any(t in name for t in txt) else self.l_img

    def step_flops(self) -> float:
        """2 M N K summed over the step's projections (the SwiGLU-fused
        projections count their full 2 ff_inner rows; the single blocks'
        to_qkv_mlp_proj its full width)."""
        return sum(2.0 * self.rows_of(name) * n * k for name, n, k in self.projection_shapes())


def random_projections(dims: DitDims, dtype: torch.dtype = torch.float16, seed: int = 0,
                       device=None) -> list[Q]:
    """Synthetic resident projections of the plan's shapes, generated on the
    device: random packed words, scale = |N(0, 1)| / (4 sqrt(K)), bias = -8 scale
    + N(0, 1) / (40 sqrt(K)).  Weights of rms about 1.2 / sqrt(K) keep a
    projection's output at the scale of its normalized input, so the residual
    stream stays finite in f16 through all blocks, as trained weights do."""
    dev = torch.device("cuda", device_index(device))
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for _, n, k in dims.projection_shapes():
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev,
                          generator=g)
        unit = 1.0 / (4.0 * k ** 0.5)
        s = torch.randn((n, k // 64), device=dev, generator=g).abs() * unit
        b = -8.0 * s + torch.randn((n, k // 64), device=dev, generator=g) * (0.1 * unit)
        out.append(Q(w=w, s=s.to(dtype), b=b.to(dtype), n=n, k=k))
    return out


def random_head(dims: DitDims, channels: int = 128, dtype: torch.dtype = torch.float16,
                seed: int = 0, device=None) -> tuple[Q, Q]:
    """Synthetic x_embedder [dim, channels] and proj_out [channels, dim] with the
    scale law of ``random_projections`` (``loadHead``, DirectDiTStep.swift:844-884)."""
    dev = torch.device("cuda", device_index(device))
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for n, k in ((dims.dim, channels), (channels, dims.dim)):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32, device=dev,
                          generator=g)
        unit = 1.0 / (4.0 * k ** 0.5)
        s = torch.randn((n, k // 64), device=dev, generator=g).abs() * unit
        b = -8.0 * s + torch.randn((n, k // 64), device=dev, generator=g) * (0.1 * unit)
        out.append(Q(w=w, s=s.to(dtype), b=b.to(dtype), n=n, k=k))
    return out[0], out[1]


def _qweight(q: Q) -> "_lib.QWeight":
    r = _lib.QWeight()
    r.w, r.scales, r.biases = q.w.data_ptr(), q.s.data_ptr(), q.b.data_ptr()
    r.n, r.k = q.n, q.k
    r.dtype = _DTYPES.get(q.s.dtype, -1)
    r.base = None
    return r


class DitStep:
    """A created step plan over resident projections (kept alive here)."""

    def __init__(self, dims: DitDims, projections: list[Q], device=None):
        self.dims = dims
        self.projections = projections
        self.device = torch.device("cuda", device_index(device))
        dt = projections[0].s.dtype
        self.dtype = dt
        L = _lib.load()
        self._L = L
        self._ctx = context(self.device)
        arr = (_lib.QWeight * len(projections))()
        for i, q in enumerate(projections):
            arr[i].w = q.w.data_ptr()
            arr[i].scales = q.s.data_ptr()
            arr[i].biases = q.b.data_ptr()
            arr[i].n = q.n
            arr[i].k = q.k
            arr[i].dtype = _DTYPES.get(q.s.dtype, -1)
            arr[i].base = None
        d = _lib.DitDims(dims.l_img, dims.l_txt, dims.dim, dims.ff_inner, dims.n_double,
                         dims.n_single)
        out = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(L.imq_dit_step_create(self._ctx, ctypes.byref(d), arr, len(projections),
                                             _DTYPES.get(dt, -1), ctypes.byref(out)), self._ctx)
        self._h = out

    def close(self) -> None:
        if self._h:
            self._L.imq_dit_step_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_conditioning(self, norm_weight: torch.Tensor | None = None,
                         gates: torch.Tensor | None = None) -> None:
        d = self.dims
        if norm_weight is not None:
            assert norm_weight.dtype == torch.float32 and norm_weight.numel() == d.dim
            assert norm_weight.is_contiguous()
        if gates is not None:
            assert gates.dtype == torch.float32 and gates.is_contiguous()
            assert gates.numel() == (4 * d.n_double + d.n_single) * d.dim
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_dit_step_set_conditioning(
                self._h, ctypes.c_void_p(norm_weight.data_ptr() if norm_weight is not None else 0),
                ctypes.c_void_p(gates.data_ptr() if gates is not None else 0),
                ctypes.c_void_p(st)), self._ctx)

    def run(self, h: torch.Tensor, e: torch.Tensor, out: torch.Tensor | None = None,
            use_graph: bool = True) -> torch.Tensor:
        """x_out [l_txt + l_img, dim] fp32 (text rows first) from h [l_img, dim]
        and e [l_txt, dim] fp32."""
        d = self.dims
        assert h.dtype == torch.float32 and tuple(h.shape) == (d.l_img, d.dim) and h.is_contiguous()
        assert e.dtype == torch.float32 and tuple(e.shape) == (d.l_txt, d.dim) and e.is_contiguous()
        if out is None:
            out = torch.empty((d.joint, d.dim), dtype=torch.float32, device=self.device)
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_dit_step_run(self._h, ctypes.c_void_p(h.data_ptr()),
                                                ctypes.c_void_p(e.data_ptr()),
                                                ctypes.c_void_p(out.data_ptr()), int(use_graph),
                                                ctypes.c_void_p(st)), self._ctx)
        return out

    def set_head(self, x_embedder: Q, proj_out: Q) -> None:
        """``loadHead``: the x_embedder [dim, C] and proj_out [C, dim] projections
        of ``denoise`` (kept alive here)."""
        self.head = (x_embedder, proj_out)
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_dit_step_set_head(self._h, ctypes.byref(_qweight(x_embedder)),
                                                     ctypes.byref(_qweight(proj_out))), self._ctx)

    def denoise(self, lat_in: torch.Tensor, e: torch.Tensor, dt: float,
                out: torch.Tensor | None = None, use_graph: bool = True) -> torch.Tensor:
        """``encodeDenoiseStep``: lat_out [l_img, C] fp32 = lat_in + 16 dt times the
        head's prediction, after the embedder, the blocks and proj_out."""
        d = self.dims
        assert lat_in.dtype == torch.float32 and lat_in.dim() == 2 and lat_in.shape[0] == d.l_img
        assert lat_in.is_contiguous()
        assert e.dtype == torch.float32 and tuple(e.shape) == (d.l_txt, d.dim) and e.is_contiguous()
        if out is None:
            out = torch.empty_like(lat_in)
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_dit_step_denoise(
                self._h, ctypes.c_void_p(lat_in.data_ptr()), ctypes.c_void_p(e.data_ptr()),
                ctypes.c_void_p(out.data_ptr()), float(dt), int(use_graph),
                ctypes.c_void_p(st)), self._ctx)
        return out

    # ---- block halves around the caller's attention (imq_dit_double_attn_in ...)

    def _call(self, name: str, *args) -> None:
        st = torch.cuda.current_stream(self.device).cuda_stream
        ptrs = [a if isinstance(a, (int, float)) else
                ctypes.c_void_p(a.data_ptr() if a is not None else 0) for a in args]
        with torch.cuda.device(self.device):
            _lib.check(getattr(self._L, name)(self._h, *ptrs, ctypes.c_void_p(st)), self._ctx)

    def _joint(self, t: torch.Tensor | None, width: int, dtype: torch.dtype, what: str) -> None:
        if t is None:
            return
        assert t.is_cuda and t.is_contiguous(), f"{what} must be a contiguous device tensor"
        assert t.dtype == dtype, f"{what} must be {dtype}"
        assert tuple(t.shape) == (self.dims.joint, width), f"{what} must be [J, {width}]"

    def double_attn_in(self, block: int, x: torch.Tensor | None, q: torch.Tensor, k: torch.Tensor,
                       v: torch.Tensor, nx: torch.Tensor | None = None) -> None:
        """Double block ``block`` before attention: q, k, v [J, dim] (T, text rows
        first) from nx (T [J, dim]) or, with nx None, the stand-in RMSNorm(x)."""
        d = self.dims
        self._joint(x, d.dim, torch.float32, "x")
        self._joint(nx, d.dim, self.dtype, "nx")
        for t, n in ((q, "q"), (k, "k"), (v, "v")):
            self._joint(t, d.dim, self.dtype, n)
        self._call("imq_dit_double_attn_in", int(block), x, nx, q, k, v)

    def double_attn_out(self, block: int, attn: torch.Tensor, x: torch.Tensor) -> None:
        """Double block ``block`` after attention: x += gated to_out / to_add_out of attn."""
        self._joint(attn, self.dims.dim, self.dtype, "attn")
        self._joint(x, self.dims.dim, torch.float32, "x")
        self._call("imq_dit_double_attn_out", int(block), attn, x)

    def double_mlp(self, block: int, x: torch.Tensor, nx: torch.Tensor | None = None) -> None:
        """Double block ``block``'s two MLPs with their gated residual adds into x."""
        self._joint(x, self.dims.dim, torch.float32, "x")
        self._joint(nx, self.dims.dim, self.dtype, "nx")
        self._call("imq_dit_double_mlp", int(block), nx, x)

    def single_attn_in(self, block: int, x: torch.Tensor | None, qkv: torch.Tensor,
                       concat: torch.Tensor, nx: torch.Tensor | None = None) -> None:
        """Single block ``block`` before attention: qkv [J, 3 dim] and the MLP half
        (columns [dim, dim + ff_inner)) of concat [J, dim + ff_inner]."""
        d = self.dims
        self._joint(x, d.dim, torch.float32, "x")
        self._joint(nx, d.dim, self.dtype, "nx")
        self._joint(qkv, 3 * d.dim, self.dtype, "qkv")
        self._joint(concat, d.dim + d.ff_inner, self.dtype, "concat")
        self._call("imq_dit_single_attn_in", int(block), x, nx, qkv, concat)

    def single_attn_out(self, block: int, concat: torch.Tensor, x: torch.Tensor) -> None:
        """Single block ``block`` after attention (concat[:, :dim] holds it): x +=
        gated to_out of concat."""
        d = self.dims
        self._joint(concat, d.dim + d.ff_inner, self.dtype, "concat")
        self._joint(x, d.dim, torch.float32, "x")
        self._call("imq_dit_single_attn_out", int(block), concat, x)

    def head_embed(self, lat: torch.Tensor, x: torch.Tensor) -> None:
        """The image rows of x = float(T(T(lat / 16) . x_embedder^T)) * 16."""
        assert lat.dtype == torch.float32 and lat.is_contiguous() and lat.shape[0] == self.dims.l_img
        self._joint(x, self.dims.dim, torch.float32, "x")
        self._call("imq_dit_head_embed", lat, x)

    def head_out(self, x: torch.Tensor | None, lat_in: torch.Tensor, dt: float,
                 lat_out: torch.Tensor, nh: torch.Tensor | None = None) -> None:
        """lat_out = lat_in + float(T(nh . proj_out^T)) * 16 dt, nh the caller's
        norm_out output / 16 or, with nh None, the stand-in T(RMSNorm(x image rows) / 16)."""
        self._joint(x, self.dims.dim, torch.float32, "x")
        if nh is not None:
            assert nh.dtype == self.dtype and nh.is_contiguous()
            assert tuple(nh.shape) == (self.dims.l_img, self.dims.dim)
        assert lat_in.is_contiguous() and lat_out.is_contiguous()
        assert lat_in.dtype == lat_out.dtype == torch.float32 and lat_in.shape == lat_out.shape
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(self._L.imq_dit_head_out(
                self._h, ctypes.c_void_p(x.data_ptr() if x is not None else 0),
                ctypes.c_void_p(nh.data_ptr() if nh is not None else 0),
                ctypes.c_void_p(lat_in.data_ptr()), ctypes.c_void_p(lat_out.data_ptr()),
                float(dt), ctypes.c_void_p(st)), self._ctx)

    @property
    def launches(self) -> int:
        return self._L.imq_dit_step_launches(self._h)

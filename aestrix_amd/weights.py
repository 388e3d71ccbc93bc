"""Packed-tensor loader: safetensors shards -> resident packed projections.

The reference's weight path for the quantized layers, over the C ABI of
``include/imq_weights.h`` (shards memory-mapped and parsed in C++, staged
uploads through pinned buffers):

* ``SafetensorsSet.open_dir``  -- ``SafetensorsLoader.shardFileNames`` + ``loadMergedArrays``
  (``Sources/ImarelloWeights/SafetensorsLoader.swift:6-25``,
  ``Sources/ImarelloWeights/SafetensorsLoader+MLX.swift:7-17``)
* ``load_qlinear``            -- ``DirectDiTStep.quant`` (``Sources/ImarelloDirect/DirectDiTStep.swift:278-284``)
* ``load_dit_blocks`` / ``load_dit_head`` -- ``DirectDiTStep.loadBlocks`` / ``loadHead``
  (``DirectDiTStep.swift:294-336,844-884``): scales and biases cast bf16 -> f16
* ``load_text_encoder``       -- ``DirectTEForward.loadLayers`` (``DirectTEForward.swift:97-138``)
* ``load_conditioner``        -- ``DirectConditioner`` init (``DirectConditioner.swift:75-91``):
  f32 scales, except ``context_embedder`` (bf16)
* ``text_encoder_keys``       -- ``TextEncoderWeights.sanitize``
  (``Sources/ImarelloText/TextEncoderWeights.swift:36-60``)

The f16 cast of the DiT's scales is the reference's choice (exact for its
4-bit pack, ``Sources/ImarelloDiT/TransformerWeights.swift:24-54``); bf16 is
kept when ``scales=torch.bfloat16`` is asked for.
"""

from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .ops import Q, context, device_index

_TORCH_ST = {torch.bfloat16: 6, torch.float16: 5, torch.float32: 9, torch.int32: 8,
             torch.uint8: 1, torch.int8: 2, torch.int16: 4, torch.float64: 12, torch.int64: 11,
             torch.bool: 0}
_NP = {"BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16,
       "F16": np.float16, "BF16": np.uint16, "U32": np.uint32, "I32": np.int32,
       "F32": np.float32, "U64": np.uint64, "I64": np.int64, "F64": np.float64,
       "F8_E4M3": np.uint8, "F8_E5M2": np.uint8}
# Stored dtype -> the torch dtype its raw bytes upload as (U32 words go to int32).
_RAW_TORCH = {"BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "U16": torch.int16,
              "I16": torch.int16, "F16": torch.float16, "BF16": torch.bfloat16,
              "U32": torch.int32, "I32": torch.int32, "F32": torch.float32,
              "U64": torch.int64, "I64": torch.int64, "F64": torch.float64,
              "F8_E4M3": torch.uint8, "F8_E5M2": torch.uint8}


class WeightsError(ValueError):
    """A shard or tensor that cannot be read (missing, malformed, wrong shape)."""


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    nbytes: int
    shard: int


class SafetensorsSet:
    """An opened, memory-mapped set of safetensors shards (one merged name map)."""

    def __init__(self, handle: ctypes.c_void_p):
        self._h = handle
        self._lib = _lib.load()

    @classmethod
    def open(cls, paths) -> "SafetensorsSet":
        L = _lib.load()
        paths = [os.fspath(p) for p in paths]
        arr = (ctypes.c_char_p * len(paths))(*[p.encode() for p in paths])
        out = ctypes.c_void_p()
        if L.imq_st_open(arr, len(paths), ctypes.byref(out)) != _lib.IMQ_OK:
            raise WeightsError(L.imq_st_last_error(None).decode())
        return cls(out)

    @classmethod
    def open_dir(cls, directory) -> "SafetensorsSet":
        L = _lib.load()
        out = ctypes.c_void_p()
        if L.imq_st_open_dir(os.fspath(directory).encode(), ctypes.byref(out)) != _lib.IMQ_OK:
            raise WeightsError(L.imq_st_last_error(None).decode())
        return cls(out)

    def close(self) -> None:
        if self._h:
            self._lib.imq_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        if not self._h:
            raise WeightsError("the shard set is closed")
        return self._h

    @property
    def shard_paths(self) -> list[str]:
        return [self._lib.imq_st_shard_path(self.handle, i).decode()
                for i in range(self._lib.imq_st_shard_count(self.handle))]

    def metadata(self, shard: int, key: str) -> str | None:
        v = self._lib.imq_st_metadata(self.handle, shard, key.encode())
        return v.decode() if v is not None else None

    def _info(self, st_info: _lib.StInfo) -> TensorInfo:
        return TensorInfo(st_info.name.decode(), _lib.ST_DTYPES[st_info.dtype],
                          tuple(st_info.shape[i] for i in range(st_info.ndim)),
                          st_info.bytes, st_info.shard)

    def names(self) -> list[str]:
        out = []
        info = _lib.StInfo()
        for i in range(self._lib.imq_st_count(self.handle)):
            self._lib.imq_st_info_at(self.handle, i, ctypes.byref(info))
            out.append(info.name.decode())
        return out

    def __contains__(self, name: str) -> bool:
        info = _lib.StInfo()
        return self._lib.imq_st_find(self.handle, name.encode(), ctypes.byref(info)) == _lib.IMQ_OK

    def _find(self, name: str) -> _lib.StInfo:
        info = _lib.StInfo()
        if self._lib.imq_st_find(self.handle, name.encode(), ctypes.byref(info)) != _lib.IMQ_OK:
            raise WeightsError(self._lib.imq_st_last_error(self.handle).decode())
        return info

    def info(self, name: str) -> TensorInfo:
        return self._info(self._find(name))

    def numpy(self, name: str) -> np.ndarray:
        """Read-only zero-copy view of a tensor's bytes in the mapping (BF16 as
        uint16 bit patterns); valid while the set is open."""
        info = self._find(name)
        t = self._info(info)
        if t.nbytes == 0:
            a = np.zeros(t.shape, dtype=_NP[t.dtype])
            a.flags.writeable = False
            return a
        buf = (ctypes.c_char * t.nbytes).from_address(info.data)
        a = np.frombuffer(buf, dtype=_NP[t.dtype]).reshape(t.shape)
        a.flags.writeable = False
        return a

    def upload(self, name: str, dtype: torch.dtype | None = None, device=None,
               stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """The tensor on a HIP device, converted to dtype (BF16 -> F16 / F32 and
        F16 -> F32 are the conversions provided; None keeps the stored type)."""
        t = self.info(name)
        target = dtype if dtype is not None else _RAW_TORCH[t.dtype]
        if target not in _TORCH_ST:
            raise WeightsError(f"{name}: no upload to {target}")
        dev = torch.device("cuda", device_index(device))
        out = torch.empty(t.shape, dtype=target, device=dev)
        return self.upload_into(name, out, stream)

    def upload_into(self, name: str, out: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Upload the tensor into ``out`` (contiguous, its shape, converted to
        out's dtype as ``upload`` does) -- e.g. a row range of a larger buffer."""
        t = self.info(name)
        target = out.dtype
        if target not in _TORCH_ST:
            raise WeightsError(f"{name}: no upload to {target}")
        if tuple(out.shape) != tuple(t.shape) or not out.is_contiguous() or not out.is_cuda:
            raise WeightsError(f"{name}: destination must be a contiguous HIP tensor of shape "
                               f"{t.shape}, got {tuple(out.shape)}")
        dev = out.device
        ctx = context(dev)
        st = stream if stream is not None else torch.cuda.current_stream(dev)
        dst_st = _TORCH_ST[target]
        if t.dtype == "U32" and target == torch.int32:
            dst_st = 7  # the raw words, viewed as int32
        rc = self._lib.imq_st_upload(ctx, self.handle, name.encode(), dst_st,
                                     ctypes.c_void_p(out.data_ptr()),
                                     out.numel() * out.element_size(),
                                     ctypes.c_void_p(st.cuda_stream))
        _lib.check(rc, ctx)
        return out


def load_qlinear(st: SafetensorsSet, prefix: str, scales: torch.dtype = torch.bfloat16,
                 device=None, n: int | None = None, k: int | None = None) -> Q:
    """``<prefix>.weight / .scales / .biases`` as a resident ``Q``; scales and
    biases converted to ``scales``.  When n and k are given the packed shape
    must match them (the reference passes them from its model constants)."""
    info = st.info(f"{prefix}.weight")
    if info.dtype != "U32" or len(info.shape) != 2:
        raise WeightsError(f"{prefix}.weight must be U32 [N, K/8], got {info.dtype} {info.shape}")
    nn, kk = info.shape[0], info.shape[1] * 8
    if (n is not None and n != nn) or (k is not None and k != kk):
        raise WeightsError(f"{prefix}: packed shape N={nn} K={kk}, expected N={n} K={k}")
    for suf in ("scales", "biases"):
        si = st.info(f"{prefix}.{suf}")
        if si.shape != (nn, kk // 64):
            raise WeightsError(f"{prefix}.{suf} must be [{nn}, {kk // 64}], got {si.shape}")
    w = st.upload(f"{prefix}.weight", torch.int32, device)
    s = st.upload(f"{prefix}.scales", scales, device)
    b = st.upload(f"{prefix}.biases", scales, device)
    return Q(w=w, s=s, b=b, n=nn, k=kk)


def load_qlinear_cat(st: SafetensorsSet, prefixes: list[str],
                     scales: torch.dtype = torch.bfloat16, device=None) -> Q:
    """Projections sharing K as one resident ``Q`` whose rows are theirs in order
    (q/k/v or gate/up of a text-encoder layer): one call then streams all of
    their weights in one launch.  Rows [sum(n_0..n_{i-1}), +n_i) are projection i."""
    if not prefixes:
        raise WeightsError("no projections to concatenate")
    metas = []
    for prefix in prefixes:
        info = st.info(f"{prefix}.weight")
        if info.dtype != "U32" or len(info.shape) != 2:
            raise WeightsError(f"{prefix}.weight must be U32 [N, K/8], got {info.dtype} {info.shape}")
        nn, kk = info.shape[0], info.shape[1] * 8
        for suf in ("scales", "biases"):
            si = st.info(f"{prefix}.{suf}")
            if si.shape != (nn, kk // 64):
                raise WeightsError(f"{prefix}.{suf} must be [{nn}, {kk // 64}], got {si.shape}")
        metas.append((prefix, nn, kk))
    k = metas[0][2]
    if any(m[2] != k for m in metas):
        raise WeightsError(f"projections disagree on K: {[(m[0], m[2]) for m in metas]}")
    n = sum(m[1] for m in metas)
    dev = torch.device("cuda", device_index(device))
    w = torch.empty((n, k // 8), dtype=torch.int32, device=dev)
    s = torch.empty((n, k // 64), dtype=scales, device=dev)
    b = torch.empty((n, k // 64), dtype=scales, device=dev)
    row = 0
    for prefix, nn, _ in metas:
        st.upload_into(f"{prefix}.weight", w[row:row + nn])
        st.upload_into(f"{prefix}.scales", s[row:row + nn])
        st.upload_into(f"{prefix}.biases", b[row:row + nn])
        row += nn
    return Q(w=w, s=s, b=b, n=n, k=k)


# ------------------------------------------------------------- key maps
# FLUX.2 klein 4B DiT (DirectDiTStep.swift:16-22, DirectDiTBlock.swift:15-21,
# DirectDiTDoubleBlock.swift:16-20).
DIT_DIM = 3072
DIT_FF_INNER = 9216
DIT_FF_WIDE = 18432
DIT_PROJ_WIDTH = 27648
DIT_CONCAT_WIDTH = 12288
DIT_N_DOUBLE = 5
DIT_N_SINGLE = 20


def dit_double_linears(dim: int = DIT_DIM, ff_inner: int = DIT_FF_INNER,
                       ff_wide: int = DIT_FF_WIDE) -> list[tuple[str, int, int]]:
    """(name, N, K) of a double block's projections (DirectDiTStep.swift:310-323)."""
    return [("attn.to_q", dim, dim), ("attn.to_k", dim, dim), ("attn.to_v", dim, dim),
            ("attn.add_q_proj", dim, dim), ("attn.add_k_proj", dim, dim),
            ("attn.add_v_proj", dim, dim), ("attn.to_out", dim, dim),
            ("attn.to_add_out", dim, dim), ("ff.linear_in", ff_wide, dim),
            ("ff.linear_out", dim, ff_inner), ("ff_context.linear_in", ff_wide, dim),
            ("ff_context.linear_out", dim, ff_inner)]


def dit_single_linears(dim: int = DIT_DIM, proj_width: int = DIT_PROJ_WIDTH,
                       concat_width: int = DIT_CONCAT_WIDTH) -> list[tuple[str, int, int]]:
    """(name, N, K) of a single block's projections (DirectDiTStep.swift:328-333)."""
    return [("attn.to_qkv_mlp_proj", proj_width, dim), ("attn.to_out", dim, concat_width)]


def load_dit_blocks(st: SafetensorsSet, n_double: int = DIT_N_DOUBLE,
                    n_single: int = DIT_N_SINGLE, scales: torch.dtype = torch.float16,
                    device=None, dims: dict | None = None) -> dict[str, Q]:
    """Every quantized projection of the DiT blocks, keyed by its full prefix
    (``transformer_blocks.{i}.attn.to_q`` ...); scales cast to f16 like
    ``loadBlocks``'s ``sub()`` (DirectDiTStep.swift:296-307)."""
    dims = dims or {}
    out = {}
    for i in range(n_double):
        for name, n, k in dit_double_linears(**{key: dims[key] for key in
                                                 ("dim", "ff_inner", "ff_wide") if key in dims}):
            p = f"transformer_blocks.{i}.{name}"
            out[p] = load_qlinear(st, p, scales, device, n, k)
    for i in range(n_single):
        for name, n, k in dit_single_linears(**{key: dims[key] for key in
                                                 ("dim", "proj_width", "concat_width")
                                                 if key in dims}):
            p = f"single_transformer_blocks.{i}.{name}"
            out[p] = load_qlinear(st, p, scales, device, n, k)
    return out


def load_dit_head(st: SafetensorsSet, scales: torch.dtype = torch.float16, device=None) -> dict[str, Q]:
    """``x_embedder`` and ``proj_out``, shapes taken from the tensors
    (``loadHead``'s ``conv``, DirectDiTStep.swift:845-857)."""
    return {p: load_qlinear(st, p, scales, device) for p in ("x_embedder", "proj_out")}


# Qwen3 text encoder as the reference drives it (DirectTEForward.swift:11-18).
TE_HIDDEN = 2560
TE_N_HEADS = 32
TE_N_KV = 8
TE_HEAD_DIM = 128
TE_INTER = 9728
TE_N_LAYERS = 27


def te_linears(hidden: int = TE_HIDDEN, n_heads: int = TE_N_HEADS, n_kv: int = TE_N_KV,
               head_dim: int = TE_HEAD_DIM, inter: int = TE_INTER) -> list[tuple[str, int, int]]:
    """(name, N, K) of a layer's projections (DirectTEForward.swift:98-106)."""
    return [("self_attn.q_proj", n_heads * head_dim, hidden),
            ("self_attn.k_proj", n_kv * head_dim, hidden),
            ("self_attn.v_proj", n_kv * head_dim, hidden),
            ("self_attn.o_proj", hidden, n_heads * head_dim),
            ("mlp.gate_proj", inter, hidden), ("mlp.up_proj", inter, hidden),
            ("mlp.down_proj", hidden, inter)]


def load_text_encoder(st: SafetensorsSet, n_layers: int = TE_N_LAYERS,
                      raw_scales: bool = False, device=None,
                      dims: dict | None = None) -> dict[str, Q]:
    """Every quantized projection of the first n_layers layers
    (``layers.{i}.self_attn.q_proj`` ...).  ``raw_scales=False`` casts scales
    and biases to f16 as ``loadLayers`` does by default; True keeps bf16."""
    scales = None if raw_scales else torch.float16
    out = {}
    for i in range(n_layers):
        for name, n, k in te_linears(**(dims or {})):
            p = f"layers.{i}.{name}"
            sd = scales if scales is not None else _RAW_TORCH[st.info(f"{p}.scales").dtype]
            out[p] = load_qlinear(st, p, sd, device, n, k)
    return out


# Conditioner (DirectConditioner.swift:16-17,85-91): f32 scales for the M=1
# kernels, bf16 for context_embedder (fed bf16 prompt embeddings).
COND_DIM = 3072
COND_SIN_DIM = 256
COND_CONTEXT_K = 7680


def conditioner_linears(dim: int = COND_DIM, sin_dim: int = COND_SIN_DIM,
                        context_k: int = COND_CONTEXT_K) -> list[tuple[str, int, int, torch.dtype]]:
    return [("time_guidance_embed.linear_1", dim, sin_dim, torch.float32),
            ("time_guidance_embed.linear_2", dim, dim, torch.float32),
            ("double_stream_modulation_img.linear", 6 * dim, dim, torch.float32),
            ("double_stream_modulation_txt.linear", 6 * dim, dim, torch.float32),
            ("single_stream_modulation.linear", 3 * dim, dim, torch.float32),
            ("norm_out.linear", 2 * dim, dim, torch.float32),
            ("context_embedder", dim, context_k, torch.bfloat16)]


def load_conditioner(st: SafetensorsSet, device=None, dims: dict | None = None) -> dict[str, Q]:
    return {name: load_qlinear(st, name, dt, device, n, k)
            for name, n, k, dt in conditioner_linears(**(dims or {}))}


_SWIFT_INT = re.compile(r"[+-]?[0-9]+")


def text_encoder_keys(names, max_layer: int) -> list[str]:
    """``TextEncoderWeights.sanitize``: drop the rotary cache, the final norm,
    the LM head, ``layers.<i>.`` keys whose index does not parse as an integer,
    and layers at or past ``max_layer``; keep the rest."""
    keep = []
    for key in names:
        if key.startswith("rotary_emb") or key == "norm.weight" or key.startswith("norm."):
            continue
        if key.startswith("lm_head"):
            continue
        if key.startswith("layers."):
            rest = key[len("layers."):]
            dot = rest.find(".")
            if dot < 0 or not _SWIFT_INT.fullmatch(rest[:dot]):
                continue
            if int(rest[:dot]) >= max_layer:
                continue
        keep.append(key)
    return keep

"""Seeded synthetic inputs in the MLX affine 4-bit format (group 64).

One documented generator, numpy ``Generator(PCG64(seed))``, drawing in this
fixed order so that the GPU kernels and the CPU baseline see the same bytes:

1. x = RNE_bf16(float32 N(0, 1))                         [M, K]
2. packed codes: uniform uint32 words (eight independent
   uniform 4-bit codes each, low nibble first)            [N, K/8]
3. scales s = RNE_bf16(|N(0, 0.02)|)                      [N, K/64]
4. biases b = RNE_bf16(-8 s + N(0, 0.002))                [N, K/64]

MLX's own RNG streams are not reproducible here, so "seed 0" means this
generator.  bf16 values are uint16 bit patterns.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GROUP_SIZE = 64


def _f32_to_bf16(v: np.ndarray) -> np.ndarray:
    bits = np.asarray(v, dtype=np.float32).view(np.uint32)
    return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1)))
            >> np.uint32(16)).astype(np.uint16)


def _bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclass
class Problem:
    x: np.ndarray       # uint16 bf16 bits [M, K]
    w: np.ndarray       # uint32 [N, K/8]
    scales: np.ndarray  # uint16 bf16 bits [N, K/64]
    biases: np.ndarray  # uint16 bf16 bits [N, K/64]

    @property
    def m(self) -> int:
        return self.x.shape[0]

    @property
    def n(self) -> int:
        return self.w.shape[0]

    @property
    def k(self) -> int:
        return self.w.shape[1] * 8


def make_weight(rng: np.random.Generator, n: int, k: int):
    if k % GROUP_SIZE:
        raise ValueError("K must be a multiple of 64")
    w = rng.integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint32)
    s = _f32_to_bf16(np.abs(rng.normal(0.0, 0.02, size=(n, k // GROUP_SIZE))).astype(np.float32))
    noise = rng.normal(0.0, 0.002, size=(n, k // GROUP_SIZE)).astype(np.float32)
    b = _f32_to_bf16(np.float32(-8.0) * _bf16_to_f32(s) + noise)
    return w, s, b


def make_problem(m: int, n: int, k: int, seed: int = 0) -> Problem:
    rng = np.random.Generator(np.random.PCG64(seed))
    x = _f32_to_bf16(rng.standard_normal(size=(m, k), dtype=np.float32)) if m > 0 else \
        np.zeros((0, k), dtype=np.uint16)
    w, s, b = make_weight(rng, n, k)
    return Problem(x=x, w=w, scales=s, biases=b)


def to_device(p: Problem, device="cuda"):
    """(x, w, scales, biases) as torch tensors on a HIP device: x, s, b bf16, w int32."""
    import torch

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)

    w = torch.from_numpy(np.ascontiguousarray(p.w).view(np.int32)).to(device)
    return bf(p.x), w, bf(p.scales), bf(p.biases)


def bf16_bits(t) -> np.ndarray:
    """bf16 torch tensor -> numpy uint16 bit patterns (on the host)."""
    import torch

    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)

"""Seeded random shapes through the regime dispatcher, against the oracle.

imq_qmm_t picks the qGEMV, the few-row kernel (whole K, multi-tile or K
split) or the tile kernel (buffer-load or register-staged, with or without a
K split) from M, N and K.  The fixed-shape tests pin each kernel at the shapes
the model runs; this sweep draws 32 shapes per dtype with M log-uniform in
[1, 700], N in [1, 3000] and K a multiple of 64 up to 5120 (seeded, so the
same shapes every run), crossing the regime boundaries at arbitrary sizes:
partial row and column tiles, K % 256 != 0 and K % 128 != 0, split plans.

Oracle: RNE_T of the double-accumulated product with the bit-exact T dequant
(oracle.cref.qmm_t_f64).  Bars as in the other GPU tests: MAE <= 1e-3,
normwise max error <= 1e-2, cosine >= 0.99999; and a second call returns the
same bits (every plan sums in a fixed order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import synth
from oracle import cref, ref

pytestmark = pytest.mark.gpu

MAE_TOL = 1e-3
NORMWISE_TOL = 1e-2
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)
MAX_MACS = 1_500_000_000  # bounds the oracle's CPU time per case


def sweep_shapes(seed: int, count: int) -> list[tuple[int, int, int]]:
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        m = int(np.exp(rng.uniform(0.0, np.log(700.0))))
        n = int(rng.integers(1, 3001))
        k = 64 * int(rng.integers(1, 81))
        if m >= 1 and m * n * k <= MAX_MACS:
            out.append((m, n, k))
    return out


SHAPES = sweep_shapes(2026, 32)
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def t_values(bits: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return ref.bf16_to_f32(bits).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def round_t(v: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return ref.f64_to_bf16(v)
    return np.asarray(v, np.float64).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("case", SHAPES, ids=[f"M{m}_N{n}_K{k}" for m, n, k in SHAPES])
def test_dispatcher_random_shape(dtype, case):
    m, n, k = case
    plan = imq.qmm_plan(m, n, k, TDT[dtype])
    print(f"sweep {dtype} M={m} N={n} K={k} plan={plan}", flush=True)
    p = synth.make_problem(m, n, k, seed=m * 7919 + n * 31 + k)
    x, w, s, b = synth.to_device(p)
    if dtype == "f16":
        x, s, b = x.half(), s.half(), b.half()
    y1 = imq.quantized_matmul(x, w, s, b)
    y2 = imq.quantized_matmul(x, w, s, b)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "two calls of one plan differ"
    xb, sb, bb = host_bits(x), host_bits(s), host_bits(b)
    want = t_values(round_t(cref.qmm_t_f64(xb, p.w, sb, bb, dtype), dtype), dtype)
    got = t_values(host_bits(y1), dtype)
    assert np.all(np.isfinite(got))
    st = ref.error_stats_values(got, want)
    print(f"  mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g} "
          f"bit_exact={st['bit_exact_frac']:.4f} cosine={st['cosine']:.7f}", flush=True)
    assert st["mae"] <= MAE_TOL and st["max_rel_normwise"] <= NORMWISE_TOL, st
    assert st["cosine"] >= COSINE_MIN, st

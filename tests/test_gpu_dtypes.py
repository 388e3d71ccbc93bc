"""GPU parity of the f16 and f32 element types against the CPU oracle.

The reference's DiT kernels run in f16 (`affine_qmm_t_float16_t`,
Sources/ImarelloDirect/DirectDiTStep.swift:82-85) and its conditioner kernels
in f32 (`affine_qmm_t_float`, Sources/ImarelloDirect/DirectConditioner.swift:48,75-84);
x, scales, biases and y share the element type T.

Bars (as for bf16):
* dequantize: bit-exact against RNE_T(fl32(fl32(s*q) + b)) (f32: fl32(s*q + b));
* qGEMV / qGEMM: against RNE_T(x . deq_T(W)^T accumulated in double):
  mean |y - oracle| <= MAE_TOL and max |y - oracle| / max |oracle| <= NORMWISE_TOL;
* one-hot activations make y a column of deq_T(W): bit-exact.

Scales and biases carry full f16 / f32 significands (not bf16-derived ones,
for which s*q + b is exact in f16), so the kernels' own rounding of the
dequantized weight to T is exercised.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import _lib, synth
from oracle import ref

pytestmark = pytest.mark.gpu

MAE_TOL = 1e-3
NORMWISE_TOL = 1e-2
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)
TORCH = {np.float16: torch.float16, np.float32: torch.float32}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def problem(m: int, n: int, k: int, dtype, seed: int):
    """x ~ N(0,1), codes uniform, s = |N(0,0.02)|, b = -8 s + N(0,0.002), all in T."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(dtype)
    w = rng.integers(0, 2 ** 32, size=(n, k // 8), dtype=np.uint32)
    s64 = np.abs(rng.standard_normal((n, k // 64)) * 0.02)
    s = s64.astype(dtype)
    b = (-8.0 * s.astype(np.float64) + rng.standard_normal((n, k // 64)) * 0.002).astype(dtype)
    return x, w, s, b


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_close(y: np.ndarray, want: np.ndarray, what: str) -> None:
    st = ref.error_stats_values(y, want)
    note(f"  {what}: mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g} "
         f"bit_exact={st['bit_exact_frac']:.4f} cosine={st['cosine']:.7f}")
    assert np.all(np.isfinite(y)), what
    assert st["mae"] <= MAE_TOL, (what, st)
    assert st["max_rel_normwise"] <= NORMWISE_TOL, (what, st)
    assert st["cosine"] >= COSINE_MIN, (what, st)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("n,k", [(96, 512), (1000, 3072)])
def test_dequant_bit_exact(dtype, n, k):
    note(f"dequant {np.dtype(dtype).name} N={n} K={k}")
    _, w, s, b = problem(0, n, k, dtype, seed=31)
    out = host(imq.dequantize(dev(w), dev(s), dev(b)))
    want = ref.dequantize_as(w, s, b, dtype)
    assert out.dtype == dtype
    assert np.array_equal(out.view(np.uint16 if dtype == np.float16 else np.uint32),
                          want.view(np.uint16 if dtype == np.float16 else np.uint32))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("m", [1, 3, 16])
@pytest.mark.parametrize("n,k", [(1000, 768), (33, 4160), (2560, 9728)])
def test_qgemv(dtype, m, n, k):
    note(f"qgemv {np.dtype(dtype).name} M={m} N={n} K={k}")
    x, w, s, b = problem(m, n, k, dtype, seed=32)
    y = host(imq.qgemv(dev(x), dev(w), dev(s), dev(b)))
    assert_close(y, ref.qmm_t_as(x, w, s, b, dtype), f"qgemv {np.dtype(dtype).name}")


@pytest.mark.parametrize("m,n,k", [(17, 32, 64), (129, 200, 192), (300, 257, 3072),
                                   (512, 4096, 2560)])
def test_qgemm_f16(m, n, k):
    note(f"qgemm f16 M={m} N={n} K={k}")
    x, w, s, b = problem(m, n, k, np.float16, seed=33)
    y = host(imq.qgemm(dev(x), dev(w), dev(s), dev(b)))
    assert_close(y, ref.qmm_t_as(x, w, s, b, np.float16), "qgemm f16")


def test_qmm_t_f32_beyond_16_rows():
    """f32 has no MFMA kernel: the dispatcher runs any M on the qGEMV kernel,
    16 rows at a time (the conditioner's multi-row calls)."""
    note("qmm_t f32 M=40 N=384 K=3072")
    x, w, s, b = problem(40, 384, 3072, np.float32, seed=34)
    y = host(imq.quantized_matmul(dev(x), dev(w), dev(s), dev(b)))
    assert_close(y, ref.qmm_t_as(x, w, s, b, np.float32), "qmm_t f32 M=40")


def test_qgemm_f32_is_unsupported():
    x, w, s, b = problem(32, 64, 128, np.float32, seed=35)
    with pytest.raises(_lib.ImqUnsupported):
        imq.qgemm(dev(x), dev(w), dev(s), dev(b))


@pytest.mark.parametrize("dtype,fn_name,m", [(np.float16, "qgemm", 40), (np.float16, "qgemv", 16),
                                             (np.float32, "qgemv", 16), (np.float32, "qgemv", 1)])
def test_one_hot_rows_reproduce_dequant_bit_exact(dtype, fn_name, m):
    n, k = 320, 3072
    note(f"{fn_name} {np.dtype(dtype).name} one-hot M={m} N={n} K={k}")
    _, w, s, b = problem(0, n, k, dtype, seed=36)
    rng = np.random.default_rng(36)
    cols = rng.choice(k, size=m, replace=False)
    x = np.zeros((m, k), dtype=dtype)
    x[np.arange(m), cols] = 1.0
    y = host(getattr(imq, fn_name)(dev(x), dev(w), dev(s), dev(b)))
    deq = host(imq.dequantize(dev(w), dev(s), dev(b)))
    assert np.array_equal(y, deq[:, cols].T)
    assert np.array_equal(deq, ref.dequantize_as(w, s, b, dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_rows_equals_dequantize(dtype):
    """imq_dequantize_rows (embedRow for a batch of ids, DirectTEEncoder.swift:106-123):
    the rows of imq_dequantize bit for bit, ids repeated and at both ends, an
    empty batch; ids out of range are refused on the host and clamped by the
    kernel when passed straight to the C ABI."""
    p = synth.make_problem(1, 1000, 2560, seed=81)
    _, w, s, b = synth.to_device(p)
    s, b = s.to(dtype), b.to(dtype)
    full = imq.dequantize(w, s, b)
    ids = torch.tensor([5, 0, 999, 5, 17, 998, 0, 512], dtype=torch.int32, device="cuda")
    got = imq.dequantize_rows(w, s, b, ids)
    torch.cuda.synchronize()
    assert torch.equal(got, full[ids.long()])
    assert imq.dequantize_rows(w, s, b, ids[:0]).shape == (0, 2560)
    with pytest.raises(ValueError, match="ids"):
        imq.dequantize_rows(w, s, b, torch.tensor([3, 1000], device="cuda"))
    # straight to the C ABI: -7 reads row 0, 1003 reads row 999
    from aestrix_amd import _lib, ops
    bad = torch.tensor([-7, 1003, 4], dtype=torch.int32, device="cuda")
    out = torch.empty((3, 2560), dtype=dtype, device="cuda")
    ctx = ops.context(w.device)
    st = _lib.load().imq_dequantize_rows(ctx, ops._ptr(w), ops._ptr(s), ops._ptr(b), ops._ptr(bad), 3,
                                         ops._ptr(out), 2560, 1000, 64, 4, ops._DTYPES[dtype],
                                         ops._stream(out))
    _lib.check(st, ctx)
    torch.cuda.synchronize()
    assert torch.equal(out, full[torch.tensor([0, 999, 4], device="cuda")])

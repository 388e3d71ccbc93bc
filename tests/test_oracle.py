"""Pins the CPU oracle (oracle/) against checks that do not restate it.

The reference holds no golden vectors for this path (its only quantization
test checks key presence, Tests/ImarelloDiTTests/TransformerStructureTests.swift:40-48)
and its implementation (Swift + MLX + Metal) cannot run here.  The oracle is
therefore pinned by:

* exact rational arithmetic (fractions.Fraction) with an independent
  round-to-nearest-even, over all 16 codes and a grid of (scale, bias) bf16
  patterns (negative, zero, subnormal, huge, ties);
* torch's own float32 arithmetic and bf16 conversion;
* known-answer words and closed forms (q = 0 -> bias, scale = 0 -> bias,
  all-equal codes -> rank-1 product);
* brute-force exact dot products on tiny shapes, torch float64 matmul,
  K-split additivity;
* planted mutants (plausible mistakes) that must fail those same checks.
"""

from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from aestrix_amd import synth
from oracle import cref, ref

# ---------------------------------------------------------------- exact RNE


def _rne(v: Fraction, p: int, emin: int = -126, emax: int = 127):
    """Round a rational to the nearest p-bit binary float (ties to even),
    with subnormals below 2^emin; returns a Fraction or +-inf (float)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = -v if v < 0 else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - p + 1)
    n = a / quantum
    f = n.numerator // n.denominator
    r = n - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2 == 1):
        f += 1
    res = f * quantum
    if res >= Fraction(2) ** (emax + 1):
        return sign * float("inf")
    return sign * res


def _bf16_bits_of(v) -> int:
    """bf16 bits of a value that is exactly representable in bf16 (or +-inf)."""
    f = float(v)
    bits = struct.unpack("<I", struct.pack("<f", f))[0]
    assert bits & 0xFFFF == 0, "not a bf16 value"
    return bits >> 16


def _bf16_value(bits: int) -> Fraction:
    f = struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]
    return Fraction(f)


def exact_dequant_bits(s_bits: int, b_bits: int, q: int) -> int:
    """RNE_bf16(fl32(fl32(s*q) + b)) computed with exact rationals: the
    reference's `scale * q + bias` on Float is two rounded operations
    (DirectTEEncoder.swift:119).  The product is exact unless it overflows."""
    prod = _rne(_bf16_value(s_bits) * q, 24)
    if isinstance(prod, float):  # product overflowed to +-inf; a finite bias keeps it
        return _bf16_bits_of(prod)
    f32 = _rne(prod + _bf16_value(b_bits), 24)
    if isinstance(f32, float):  # sum overflowed
        return _bf16_bits_of(f32)
    return _bf16_bits_of(_rne(f32, 8))


# (scale, bias) bf16 bit patterns: ordinary, negative, zero, subnormal,
# tiny normal, huge, and values whose sums land on bf16 ties.
S_PATTERNS = [0x3F80, 0x3F00, 0x3EAB, 0x3CA4, 0x3B80, 0xBCA4, 0x0000, 0x0001, 0x0050, 0x0080,
              0x00FF, 0x7E00, 0x7F00, 0x3D4D, 0x3F81, 0x4000, 0x3E4D, 0xC000]
B_PATTERNS = [0x0000, 0x3F80, 0xBF80, 0xBE24, 0xC0A0, 0x3B00, 0x0001, 0x8080, 0x7F00, 0xFF00,
              0xBD4D, 0x4100, 0x3C00, 0x2000]


def _grid():
    rows = []
    for s in S_PATTERNS:
        for b in B_PATTERNS:
            rows.append((s, b))
    return rows


def _grid_problem():
    """One weight row per (s, b) pair, each row holding codes 0..15 four times."""
    grid = _grid()
    n = len(grid)
    codes = np.tile(np.arange(16, dtype=np.uint8), 4)[None, :].repeat(n, axis=0)  # [n, 64]
    w = ref.pack_codes(codes)
    s = np.array([[g[0]] for g in grid], dtype=np.uint16)
    b = np.array([[g[1]] for g in grid], dtype=np.uint16)
    return grid, codes, w, s, b


def _exact_grid_expected():
    grid, codes, w, s, b = _grid_problem()
    exp = np.empty(codes.shape, dtype=np.uint16)
    for i, (sb, bb) in enumerate(grid):
        for k in range(codes.shape[1]):
            exp[i, k] = exact_dequant_bits(sb, bb, int(codes[i, k]))
    return exp


_EXACT_CACHE: dict = {}


def exact_grid():
    if "v" not in _EXACT_CACHE:
        _EXACT_CACHE["v"] = _exact_grid_expected()
    return _EXACT_CACHE["v"]


# ------------------------------------------------------------ bf16 rounding


def test_f32_to_bf16_matches_torch_on_random_finite_patterns():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    ours = ref.f32_to_bf16(f)
    theirs = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


def test_f32_to_bf16_ties_and_overflow():
    cases = {
        0x3F808000: 0x3F80,  # tie, even stays
        0x3F818000: 0x3F82,  # tie, odd rounds up
        0x3F807FFF: 0x3F80,  # below tie
        0x3F808001: 0x3F81,  # above tie
        0x7F7FFFFF: 0x7F80,  # largest float rounds to inf
        0x00008000: 0x0000,  # subnormal tie to even (zero)
        0x00018000: 0x0002,  # subnormal tie to even (up)
        0x80000000: 0x8000,  # negative zero
    }
    for fbits, want in cases.items():
        v = np.array([fbits], dtype=np.uint32).view(np.float32)
        assert int(ref.f32_to_bf16(v)[0]) == want, hex(fbits)
        assert int(cref.lib().oracle_f32_to_bf16(float(v[0]))) == want, hex(fbits)


def test_f64_to_bf16_is_correctly_rounded():
    rng = np.random.default_rng(3)
    vals = rng.standard_normal(20_000) * np.exp(rng.uniform(-20, 20, 20_000))
    got = ref.f64_to_bf16(vals)
    for v, g in zip(vals[:3000], got[:3000]):
        want = _rne(Fraction(float(v)), 8)
        assert int(g) == _bf16_bits_of(want)
    # a double just above a bf16 tie must round up even when its float32 cast lands on the tie
    tie = 1.0 + 2.0 ** -8          # exact midpoint between 1.0 and 1 + 2^-7
    above = tie + 2.0 ** -40       # float32 cast rounds back to the tie
    assert int(ref.f64_to_bf16(np.array([above]))[0]) == 0x3F81
    assert int(ref.f64_to_bf16(np.array([tie]))[0]) == 0x3F80


# --------------------------------------------------------------- dequantize


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(11)
    w = rng.integers(0, 1 << 32, size=(17, 24), dtype=np.uint32)
    assert np.array_equal(ref.pack_codes(ref.unpack_codes(w)), w)
    codes = rng.integers(0, 16, size=(5, 64), dtype=np.uint8)
    assert np.array_equal(ref.unpack_codes(ref.pack_codes(codes)), codes)


def test_known_answer_words_low_nibble_first():
    w = np.array([[0x76543210, 0xFEDCBA98] * 4], dtype=np.uint32)
    codes = ref.unpack_codes(w)[0]
    assert list(codes[:16]) == list(range(16))
    one = np.array([[0x3F80]], dtype=np.uint16)      # scale 1.0
    zero = np.array([[0x0000]], dtype=np.uint16)     # bias 0
    deq = ref.dequantize(w, one, zero)[0]
    want = [_bf16_bits_of(float(v)) for v in range(16)] * 4
    assert list(deq) == want
    assert list(cref.dequantize(w, one, zero)[0]) == want
    # scale 0.5, bias -4: 0.5 q - 4 is exact
    half = np.array([[0x3F00]], dtype=np.uint16)
    m4 = np.array([[0xC080]], dtype=np.uint16)
    want2 = [_bf16_bits_of(0.5 * v - 4) for v in range(16)] * 4
    assert list(ref.dequantize(w, half, m4)[0]) == want2


def test_dequant_matches_exact_rational_grid():
    _, _, w, s, b = _grid_problem()
    exp = exact_grid()
    assert np.array_equal(ref.dequantize(w, s, b), exp)
    assert np.array_equal(cref.dequantize(w, s, b), exp)


def test_dequant_matches_torch_arithmetic():
    _, codes, w, s, b = _grid_problem()
    sf = torch.from_numpy(ref.bf16_to_f32(s))
    bf = torch.from_numpy(ref.bf16_to_f32(b))
    q = torch.from_numpy(codes.astype(np.float32))
    want = (sf * q + bf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(ref.bf16_to_f32(want))
    assert np.array_equal(ref.dequantize(w, s, b)[finite], want[finite])


def test_dequant_special_cases():
    rng = np.random.default_rng(5)
    p = synth.make_problem(0, 8, 256, seed=9)
    # q = 0 -> bias exactly
    w0 = np.zeros_like(p.w)
    d0 = ref.dequantize(w0, p.scales, p.biases)
    assert np.array_equal(d0, np.repeat(p.biases, 64, axis=1))
    # scale = 0 -> bias exactly
    z = np.zeros_like(p.scales)
    assert np.array_equal(ref.dequantize(p.w, z, p.biases), np.repeat(p.biases, 64, axis=1))
    # group index is k // 64: changing group g's scale changes exactly columns [64g, 64g+64)
    s2 = p.scales.copy()
    s2[:, 2] = ref.f32_to_bf16(ref.bf16_to_f32(s2[:, 2]) * np.float32(2.0))
    diff = ref.dequantize(p.w, s2, p.biases) != ref.dequantize(p.w, p.scales, p.biases)
    cols = np.nonzero(diff.any(axis=0))[0]
    assert cols.min() >= 128 and cols.max() < 192
    del rng


def test_c_and_numpy_dequant_agree_on_random_packs():
    p = synth.make_problem(0, 300, 1024, seed=4)
    assert np.array_equal(ref.dequantize(p.w, p.scales, p.biases),
                          cref.dequantize(p.w, p.scales, p.biases))


def test_dequant_rejects_bad_shapes():
    w = np.zeros((4, 5), dtype=np.uint32)  # K = 40, not a multiple of 64
    s = np.zeros((4, 1), dtype=np.uint16)
    with pytest.raises(ValueError):
        cref.dequantize(w, s, s)


# ------------------------------------------------------- dequant-then-matmul


def _exact_qmm_bits(x, w, s, b):
    deq = ref.dequantize(w, s, b)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.uint16)
    for i in range(m):
        for j in range(n):
            acc = Fraction(0)
            for t in range(k):
                acc += _bf16_value(int(x[i, t])) * _bf16_value(int(deq[j, t]))
            r = _rne(acc, 8)
            out[i, j] = _bf16_bits_of(r)
    return out


def test_qmm_brute_force_exact_tiny():
    p = synth.make_problem(3, 4, 128, seed=21)
    want = _exact_qmm_bits(p.x, p.w, p.scales, p.biases)
    assert np.array_equal(cref.qmm_t(p.x, p.w, p.scales, p.biases), want)
    assert np.array_equal(ref.qmm_t(p.x, p.w, p.scales, p.biases), want)


def test_qmm_matches_torch_float64():
    p = synth.make_problem(33, 70, 320, seed=22)
    deq = torch.from_numpy(ref.bf16_to_f32(ref.dequantize(p.w, p.scales, p.biases))).double()
    x = torch.from_numpy(ref.bf16_to_f32(p.x)).double()
    want = (x @ deq.T).numpy()
    got = ref.qmm_t_f64(p.x, p.w, p.scales, p.biases)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    c = cref.qmm_t(p.x, p.w, p.scales, p.biases, threads=2)
    assert np.array_equal(c, ref.f64_to_bf16(want))


def test_qmm_rank1_known_answer():
    """All codes equal c: deq(W) is one value per group, so
    y[m, n] = sum_g w_g * sum_{k in g} x[m, k]."""
    p = synth.make_problem(6, 5, 256, seed=23)
    c = 11
    word = 0
    for i in range(8):
        word |= c << (4 * i)
    w = np.full_like(p.w, word)
    wg = ref.bf16_to_f32(ref.f32_to_bf16(ref.bf16_to_f32(p.scales) * np.float32(c)
                                         + ref.bf16_to_f32(p.biases))).astype(np.float64)
    xs = ref.bf16_to_f32(p.x).astype(np.float64).reshape(6, 4, 64).sum(axis=2)  # [M, G]
    want = xs @ wg.T
    np.testing.assert_allclose(ref.qmm_t_f64(p.x, w, p.scales, p.biases), want,
                               rtol=1e-12, atol=1e-12)


def test_qmm_k_split_additivity():
    p = synth.make_problem(7, 9, 384, seed=24)
    full = ref.qmm_t_f64(p.x, p.w, p.scales, p.biases)
    k1 = 128
    a = ref.qmm_t_f64(p.x[:, :k1], p.w[:, :k1 // 8], p.scales[:, :k1 // 64], p.biases[:, :k1 // 64])
    b = ref.qmm_t_f64(p.x[:, k1:], p.w[:, k1 // 8:], p.scales[:, k1 // 64:], p.biases[:, k1 // 64:])
    np.testing.assert_allclose(full, a + b, rtol=1e-12, atol=1e-12)


def test_c_f32acc_baseline_within_tolerance_of_oracle():
    p = synth.make_problem(16, 64, 1024, seed=25)
    o = cref.qmm_t(p.x, p.w, p.scales, p.biases)
    c = cref.qmm_t_f32acc(p.x, p.w, p.scales, p.biases)
    st = ref.error_stats(c, o)
    assert st["mae"] <= 1e-3 and st["max_rel_normwise"] <= 1e-2, st


# ---------------------------------------------------------- planted mutants
# Each plausible mistake in a restatement must fail a check above.


def _deq_high_nibble_first(w, s, b):
    codes = ref.unpack_codes(w).reshape(w.shape[0], -1, 8)[:, :, ::-1].reshape(w.shape[0], -1)
    return _deq_from_codes(codes, s, b)


def _deq_from_codes(codes, s, b, group=64):
    q = codes.astype(np.float32)
    n, k = q.shape
    sf = np.repeat(ref.bf16_to_f32(s), group, axis=-1)[:, :k]
    bf = np.repeat(ref.bf16_to_f32(b), group, axis=-1)[:, :k]
    return ref.f32_to_bf16(sf * q + bf)


def _deq_group32(w, s, b):
    """Group index k // 32 into the row-major [N, K/64] tables (reads the next
    groups, and past the row end into the next row)."""
    codes = ref.unpack_codes(w)
    n, k = codes.shape
    g = k // 64
    idx = (np.arange(n)[:, None] * g + np.arange(k)[None, :] // 32) % (n * g)
    sf = ref.bf16_to_f32(s.reshape(-1)[idx])
    bf = ref.bf16_to_f32(b.reshape(-1)[idx])
    with np.errstate(over="ignore", invalid="ignore"):
        return ref.f32_to_bf16(sf * codes.astype(np.float32) + bf)


def _deq_per_op_rounding(w, s, b):
    q = ref.unpack_codes(w).astype(np.float32)
    n, k = q.shape
    sf = np.repeat(ref.bf16_to_f32(s), 64, axis=-1)
    bf = np.repeat(ref.bf16_to_f32(b), 64, axis=-1)
    prod = ref.bf16_to_f32(ref.f32_to_bf16(sf * q))
    return ref.f32_to_bf16(prod + bf)


def _deq_truncating(w, s, b):
    q = ref.unpack_codes(w).astype(np.float32)
    sf = np.repeat(ref.bf16_to_f32(s), 64, axis=-1)
    bf = np.repeat(ref.bf16_to_f32(b), 64, axis=-1)
    return ((sf * q + bf).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


@pytest.mark.parametrize("mutant", [_deq_high_nibble_first, _deq_group32, _deq_per_op_rounding,
                                    _deq_truncating])
def test_dequant_checks_catch_mutants(mutant):
    _, _, w, s, b = _grid_problem()
    exact = exact_grid()
    p = synth.make_problem(0, 64, 512, seed=31)
    caught = (not np.array_equal(mutant(w, s, b), exact)
              or not np.array_equal(mutant(p.w, p.scales, p.biases),
                                    ref.dequantize(p.w, p.scales, p.biases)))
    # the grid alone must already expose every mutant
    assert not np.array_equal(mutant(w, s, b), exact)
    assert caught


def test_qmm_checks_catch_mutants():
    p = synth.make_problem(3, 4, 128, seed=21)
    want = _exact_qmm_bits(p.x, p.w, p.scales, p.biases)
    deq = ref.bf16_to_f32(ref.dequantize(p.w, p.scales, p.biases)).astype(np.float64)
    x = ref.bf16_to_f32(p.x).astype(np.float64)
    # a dropped bias term, and the K order of one operand reversed
    no_bias = ref.f64_to_bf16(x @ (deq - np.repeat(ref.bf16_to_f32(p.biases), 64, axis=1)).T)
    wrong_order = ref.f64_to_bf16(x[:, ::-1] @ deq.T)
    for mutant in (no_bias, wrong_order):
        assert not np.array_equal(mutant, want)


# ------------------------------------------- f16 / f32 element types (DiT, conditioner)
# The reference's DiT kernels run in f16 (DirectDiTStep.swift:82-85) and its
# conditioner kernels in f32 (DirectConditioner.swift:48,75-84).  The oracle's
# *_as functions are pinned here by the same exact-rational rounding.

F16 = dict(p=11, emin=-14, emax=15)
F32 = dict(p=24, emin=-126, emax=127)


def _f16_param_values() -> np.ndarray:
    vals = [0.0, -0.0, 1.0, -1.0, 0.02, -0.0175, 3.0517578125e-05, 6.1035156e-05, 5.96e-08,
            -5.96e-08, 1.5e-05, 0.333, 1000.0, -4096.0, 65504.0, 0.5 + 2 ** -11, 2 ** -14]
    return np.array(vals, dtype=np.float16)


def _exact_deq(s: float, b: float, q: int, fmt: dict):
    prod = _rne(Fraction(float(s)) * q, 24)
    if isinstance(prod, float):
        return prod
    f32 = _rne(prod + Fraction(float(b)), 24)
    if isinstance(f32, float):
        return f32
    return _rne(f32, **fmt)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_dequant_as_matches_exact_rational_grid(dtype):
    vals = _f16_param_values().astype(dtype)
    if dtype == np.float32:
        vals = np.concatenate([vals, np.array([3.4e38, -1e-40, 7.0e-39, 1.0000001], np.float32)])
    fmt = F16 if dtype == np.float16 else F32
    s = np.repeat(vals, len(vals)).reshape(-1, 1)
    b = np.tile(vals, len(vals)).reshape(-1, 1)
    n = s.shape[0]
    codes = np.tile(np.arange(16, dtype=np.uint8), (n, 4))  # K = 64: every code 4 times
    w = ref.pack_codes(codes)
    got = ref.dequantize_as(w, s, b, dtype)
    for i in range(n):
        for c in range(16):
            want = _exact_deq(s[i, 0], b[i, 0], c, fmt)
            g = got[i, c]
            if isinstance(want, float):
                assert np.isinf(g) and np.sign(g) == np.sign(want), (s[i, 0], b[i, 0], c)
            else:
                assert Fraction(float(g)) == want, (s[i, 0], b[i, 0], c, g, want)


def test_f64_to_f16_and_f32_casts_round_once():
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 5, 3000),
                        # f16 halfway points nudged by less than an f32 ulp: a cast through
                        # float32 would round these twice
                        (1 + (2 * rng.integers(0, 1024, 500) + 1) * 2.0 ** -11) * (1 + 2.0 ** -40),
                        (1 + (2 * rng.integers(0, 1024, 500) + 1) * 2.0 ** -11) * (1 - 2.0 ** -40)])
    for dtype, fmt in ((np.float16, F16), (np.float32, F32)):
        got = v.astype(dtype)
        for a, g in zip(v, got):
            want = _rne(Fraction(float(a)), **fmt)
            if isinstance(want, float):
                assert np.isinf(g)
            else:
                assert Fraction(float(g)) == want, (dtype, a, g)


def _exact_qmm_as(x, w, s, b, dtype, fmt):
    deq = ref.dequantize_as(w, s, b, dtype)
    m, n = x.shape[0], w.shape[0]
    y = np.empty((m, n), dtype=dtype)
    for i in range(m):
        for j in range(n):
            acc = sum(Fraction(float(a)) * Fraction(float(c)) for a, c in zip(x[i], deq[j]))
            r = _rne(acc, **fmt)
            y[i, j] = float(r)
    return y


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_qmm_as_brute_force_exact_tiny(dtype):
    fmt = F16 if dtype == np.float16 else F32
    p = synth.make_problem(3, 5, 128, seed=21)
    x = ref.bf16_to_f32(p.x).astype(dtype)
    s = ref.bf16_to_f32(p.scales).astype(dtype)
    b = ref.bf16_to_f32(p.biases).astype(dtype)
    got = ref.qmm_t_as(x, p.w, s, b, dtype)
    want = _exact_qmm_as(x, p.w, s, b, dtype, fmt)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_qmm_as_rank1_known_answer(dtype):
    """All codes equal c: deq is constant per group, y = sum_g w_g * sum_{k in g} x_k."""
    n, k, c = 4, 192, 11
    codes = np.full((n, k), c, dtype=np.uint8)
    w = ref.pack_codes(codes)
    s = np.array([[0.02, 0.5, -0.25]] * n, dtype=dtype)
    b = np.array([[-0.16, 1.0, 2.0]] * n, dtype=dtype)
    x = np.linspace(-1, 1, 2 * k).reshape(2, k).astype(dtype)
    wg = [float(np.float32(np.float32(s[0, g]) * c) + np.float32(b[0, g])) for g in range(3)]
    wg = [float(np.asarray(v, np.float32).astype(dtype)) for v in wg]
    for i in range(2):
        exact = sum(Fraction(wg[g]) * sum(Fraction(float(v)) for v in x[i, 64 * g:64 * g + 64])
                    for g in range(3))
        want = float(_rne(exact, **(F16 if dtype == np.float16 else F32)))
        got = ref.qmm_t_as(x, w, s, b, dtype)
        assert np.all(got[i] == np.asarray(want, dtype=dtype))


def test_f16_checks_catch_unrounded_dequant_mutant():
    """Skipping the f16 rounding of deq(W) (keeping fl32(s*q+b)) must fail the
    brute-force check on a small case.  Scales and biases carry full 11-bit
    significands here: bf16-derived ones (8 bits) make s*q + b exact in f16,
    which is why the reference's f16 precast of the bf16 pack loses nothing
    (TransformerWeights.swift:40-54)."""
    rng = np.random.default_rng(5)
    p = synth.make_problem(4, 16, 256, seed=21)
    x = ref.bf16_to_f32(p.x).astype(np.float16)
    s = (rng.random((16, 4)) * 0.05 + 0.01).astype(np.float16)
    b = (-8 * s.astype(np.float64) + rng.standard_normal((16, 4)) * 0.01).astype(np.float16)
    want = _exact_qmm_as(x, p.w, s, b, np.float16, F16)
    assert np.array_equal(ref.qmm_t_as(x, p.w, s, b, np.float16), want)
    deq32 = ref.dequantize_as(p.w, s, b, np.float32).astype(np.float64)
    mutant = (x.astype(np.float64) @ deq32.T).astype(np.float16)
    assert not np.array_equal(mutant, want)


# ------------------------------------------------ glue stages and RMSNorm
# Pinned against torch's own functions and closed forms (not restatements).

def test_glue_swiglu_matches_torch_silu():
    rng = np.random.default_rng(3)
    g = rng.standard_normal((7, 33)).astype(np.float32) * 4
    u = rng.standard_normal((7, 33)).astype(np.float32)
    want = (torch.nn.functional.silu(torch.from_numpy(g).double() * 16)
            * torch.from_numpy(u).double() * 16 / 8).numpy()
    assert np.allclose(ref.glue_swiglu(g, u, 16.0, 1.0 / 8), want, rtol=1e-12, atol=1e-12)
    assert np.all(ref.glue_swiglu(np.zeros(3, np.float32), np.ones(3, np.float32), 1, 1) == 0)


def test_glue_gate_add_matches_torch_float64_per_column_gate():
    """fma(gate[j], float(v) * scale, x) with a random per-column gate, scale
    1/16 and a non-square shape, against torch float64 arithmetic done
    independently: v * scale rounded to f32 (the kernel's multiply), then the
    exact product with the gate plus x, rounded once to f32 (the fma)."""
    rng = np.random.default_rng(44)
    m, n = 7, 19
    y = rng.standard_normal((m, n)).astype(np.float32)
    x = rng.standard_normal((m, n)).astype(np.float32)
    gate = rng.standard_normal(n).astype(np.float32)
    scale = 1.0 / 16
    vs = (torch.from_numpy(y) * torch.tensor(np.float32(scale))).double()
    want = (torch.from_numpy(gate).double()[None, :] * vs + torch.from_numpy(x).double()).float()
    got = ref.glue_gate_add(y, x, gate, scale)
    assert got.dtype == np.float32 and got.shape == (m, n)
    assert np.array_equal(got, want.numpy())
    # Mutants: the gate indexed by row instead of column, and the scale dropped.
    row_gate = np.resize(gate, m)[:, None] * (y * np.float32(scale)).astype(np.float64) + x
    assert not np.array_equal(got, row_gate.astype(np.float32))
    no_scale = gate[None, :].astype(np.float64) * y + x
    assert not np.array_equal(got, no_scale.astype(np.float32))


def test_glue_gate_add_and_postscale_closed_forms():
    rng = np.random.default_rng(4)
    y = rng.standard_normal((5, 8)).astype(np.float32)
    x = rng.standard_normal((5, 8)).astype(np.float32)
    assert np.array_equal(ref.glue_gate_add(y, x, np.zeros(8, np.float32), 3.0), x)
    one = ref.glue_gate_add(y, x, np.ones(8, np.float32), 1.0)
    assert np.array_equal(one, (x.astype(np.float64) + y).astype(np.float32))
    assert np.array_equal(ref.glue_postscale(y, 16.0), y * np.float32(16))


def test_rmsnorm_rows_matches_torch():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 300))
    w = rng.standard_normal(300)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (300,), torch.from_numpy(w),
                                        eps=1e-5).numpy()
    assert np.allclose(ref.rmsnorm_rows(x, w), want, rtol=1e-12, atol=1e-12)


def _rne_format(fr: Fraction, mant: int, emin: int, emax: int) -> Fraction | float:
    """Exact rational -> nearest value of a binary format with `mant` significand
    bits (hidden bit included), normal exponents [emin, emax], subnormals,
    ties to even; +-inf past the largest finite value."""
    if fr == 0:
        return Fraction(0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant + 1)
    units = a / ulp
    n = units.numerator // units.denominator
    rem = units - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * ulp
    if v >= Fraction(2) ** (emax + 1):
        return sign * float("inf")
    return sign * v


def test_glue_prescale_matches_exact_double_rounding():
    """(x / s).asType(T): the fp32 quotient of the exact ratio (RNE), then RNE to
    T, checked with rational arithmetic and an independent rounding, and against
    torch's CPU division and conversions."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(1500) * np.exp2(rng.integers(-30, 22, 1500))).astype(np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 16.0, 16 * (1 + 2 ** -11), 16 * (1 + 3 * 2 ** -11),
                                       65504 * 16, 65520 * 16, 2 ** -24 * 16, 2 ** -25 * 16,
                                       3 * 2 ** -26 * 16])])
    for scale in (16.0, 3.0, -0.5, 1e-3):
        s32 = np.float32(scale)
        for dtype, mant, emin, emax in (("f16", 11, -14, 15), ("bf16", 8, -126, 127)):
            got = ref.glue_prescale(x, scale, dtype)
            vals = got.astype(np.float64) if dtype == "f16" else ref.bf16_to_f32(got).astype(np.float64)
            for xi, gi in zip(x.tolist(), vals.tolist()):
                q32 = _rne_format(Fraction(xi) / Fraction(float(s32)), 24, -126, 127)
                want = q32 if isinstance(q32, float) else _rne_format(Fraction(q32), mant, emin, emax)
                assert gi == float(want), (xi, scale, dtype, gi, want)
                if gi == 0:  # a zero keeps the quotient's sign
                    assert np.signbit(gi) == (np.signbit(xi) != np.signbit(s32)), (xi, scale)
            t = torch.from_numpy(x) / torch.tensor(s32)
            tt = t.to(torch.float16 if dtype == "f16" else torch.bfloat16).float().numpy()
            assert np.array_equal(vals.astype(np.float32), tt), (scale, dtype)


def test_glue_prescale_checks_catch_truncation_mutant():
    """A conversion by truncation instead of rounding must fail the exact check:
    1 + 3 * 2^-11 is a tie that rounds to the even 1 + 2^-9 in f16, and
    1 + 2^-8 + 2^-12 rounds up to 1 + 2^-7 in bf16; truncation keeps 1 + 2^-10 / 1."""
    x = np.float32([16 * (1 + 3 * 2 ** -11), 16 * (1 + 2 ** -8 + 2 ** -12)])
    f16 = ref.glue_prescale(x, 16.0, "f16")
    bf16 = ref.bf16_to_f32(ref.glue_prescale(x, 16.0, "bf16"))
    assert float(f16[0]) == float(_rne_format(Fraction(1 + 3 * 2 ** -11), 11, -14, 15)) == 1 + 2 ** -9
    assert float(bf16[1]) == float(_rne_format(Fraction(1 + 2 ** -8 + 2 ** -12), 8, -126, 127)) == 1 + 2 ** -7
    trunc_bf16 = ((x / np.float32(16)).view(np.uint32) >> np.uint32(16)).astype(np.uint16)
    assert float(ref.bf16_to_f32(trunc_bf16)[1]) != float(bf16[1])


def test_glue_postscale_f16_is_the_f16_product():
    """f16(y * f16(s)): against torch's CPU half multiply (an independent
    routine), exact scaling by a power of two, the scale's own f16 rounding
    (1/3 rounds to 0x3555 before the product, checked with rational
    arithmetic) and overflow to inf."""
    rng = np.random.default_rng(21)
    y = (rng.standard_normal(4000) * np.exp2(rng.integers(-20, 12, 4000))).astype(np.float16)
    for scale in (16.0, 1.0 / 3.0, 4.6875, 1e-3, 300.0):
        got = ref.glue_postscale_f16(y, scale)
        assert got.dtype == np.float16
        want = (torch.from_numpy(y) * torch.tensor(scale, dtype=torch.float32).half()).numpy()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), scale
    big = y[np.abs(y) < 2000]
    assert np.array_equal(ref.glue_postscale_f16(big, 16.0), (big.astype(np.float32) * 16).astype(np.float16))
    # 5 * f16(1/3) = 5 * 0x3555 = 1706.25 ulps of [1, 2): 1.666015625; 5 * (1/3) in
    # float32 would round to 1.6669921875
    got5 = float(ref.glue_postscale_f16(np.float16([5.0]), 1.0 / 3.0)[0])
    assert got5 == float(_rne_format(5 * Fraction(float(np.float16(1 / 3))), 11, -14, 15)) == 1.666015625
    # the f32-scale mutant (y * s in float32, then f16) differs at s = 1/3
    mutant = (y.astype(np.float32) * np.float32(1 / 3)).astype(np.float16)
    assert not np.array_equal(ref.glue_postscale_f16(y, 1 / 3), mutant)
    assert np.isinf(ref.glue_postscale_f16(np.float16([60000.0]), 2.0)[0])


def test_dynamic_scale_known_answers():
    """max(amax|x| / target, 1): the amax taken over |x| (a negative element
    decides here), exact quotients for power-of-two targets, the floor at 1,
    the fp32 quotient's rounding, NaN propagation and the empty case."""
    x = np.float32([-300.0, 2.0, 100.0])
    assert ref.dynamic_scale(x, 64.0) == np.float32(4.6875)  # 300 / 64, exact
    assert ref.dynamic_scale(x[1:], 64.0) == np.float32(1.5625)  # 100 / 64
    assert ref.dynamic_scale(np.float32([-10.0, 3.0]), 64.0) == np.float32(1.0)
    assert ref.dynamic_scale(np.float32([]), 64.0) == np.float32(1.0)
    assert np.isnan(ref.dynamic_scale(np.float32([1.0, np.nan, 1000.0]), 64.0))
    assert ref.dynamic_scale(np.float32([np.inf, 1.0]), 64.0) == np.inf
    # a non-dyadic target: the correctly rounded fp32 quotient of the exact ratio
    v = np.float32(1000.0)
    q = ref.dynamic_scale(np.float32([v]), 3.0)
    assert q == np.float32(float(_rne_format(Fraction(1000, 3), 24, -126, 127)))
    # mutants: max instead of abs-max; no floor at 1
    assert np.float32(np.max(x) / 64) != ref.dynamic_scale(x, 64.0)
    assert np.float32(np.max(np.abs(x[:2])) / 1000) != ref.dynamic_scale(x[:2], 1000.0)


def test_cond_sinusoid_known_answers():
    """[cos | sin] of t * 10000^(-i / half): t = 0 gives ones then zeros (a
    swapped-halves mutant fails), t = 1 gives cos / sin of the frequencies
    themselves (closed form 10000^(-i/128) in float64, within a few float32
    ulps of the float operations' rounding), and numpy's float32 functions agree
    within 4 ulps plus what an ulp of a frequency or of the argument t f moves."""
    s0 = ref.cond_sinusoid(np.float32([0.0]), 256)[0]
    assert np.array_equal(s0[:128], np.ones(128, np.float32))
    assert np.array_equal(s0[128:], np.zeros(128, np.float32))
    swapped = np.concatenate([s0[128:], s0[:128]])
    assert not np.array_equal(swapped, s0)
    s1 = ref.cond_sinusoid(np.float32([1.0]), 256)[0].astype(np.float64)
    f = 10000.0 ** (-np.arange(128) / 128.0)
    assert np.max(np.abs(s1[:128] - np.cos(f))) < 4e-7 and np.max(np.abs(s1[128:] - np.sin(f))) < 4e-7
    # a frequency-index mutant (i / (half - 1)) moves them far more
    fm = 10000.0 ** (-np.arange(128) / 127.0)
    assert np.max(np.abs(s1[128:] - np.sin(fm))) > 1e-3
    t = np.float32([0.0, 1.0, 3.5, 250.0, 999.0])
    got = ref.cond_sinusoid(t, 256)
    half = np.float32(128)
    freq = np.exp((-np.log(np.float32(10000)) * np.arange(128, dtype=np.float32)) / half)
    arg = t[:, None] * freq[None, :]
    want = np.concatenate([np.cos(arg), np.sin(arg)], axis=1).astype(np.float32)
    # numpy's float32 exp may differ from the correctly rounded one by an ulp
    # of freq, which t multiplies, and its cos / sin by an ulp of the argument:
    # bound = 4 output ulps + |t| * 2 ulp(freq) + 2 ulp(t f)
    ulp = np.spacing(np.maximum(np.abs(want), np.float32(2 ** -24)))
    slack = (np.abs(t[:, None]) * 2 * np.tile(np.spacing(freq), 2)[None, :]
             + 2 * np.tile(np.spacing(np.abs(arg)), 2))
    assert np.all(np.abs(got - want) <= 4 * ulp + slack)


def test_silu_f32_matches_torch():
    rng = np.random.default_rng(31)
    v = np.concatenate([(rng.standard_normal(5000) * 8).astype(np.float32),
                        np.float32([0.0, -0.0, 1e-30, -90.0, 90.0, -1e4, 1e4])])
    want = torch.nn.functional.silu(torch.from_numpy(v).double()).float().numpy()
    assert np.array_equal(ref.silu_f32(v), want)
    assert ref.silu_f32(np.float32([0.0]))[0] == 0 and ref.silu_f32(np.float32([1e4]))[0] == 1e4


def test_cond_chain_against_torch():
    """The chain's composition against torch float64 on a small model (dim 128,
    sin_dim 64): torch unpacks the codes with its own shifts, dequantizes in
    float32 and runs sinusoid -> matmul -> silu -> matmul -> silu -> matmul."""
    rng = np.random.default_rng(32)
    dim, sin_dim = 128, 64

    def proj(n, k):
        w = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
        s = (np.abs(rng.standard_normal((n, k // 64))) / (4 * np.sqrt(k))).astype(np.float32)
        b = (-8 * s + rng.standard_normal((n, k // 64)) / (40 * np.sqrt(k))).astype(np.float32)
        return w, s, b

    l1, l2, hd = proj(dim, sin_dim), proj(dim, dim), proj(17 * dim, dim)
    t = np.float32([1000.0, 500.0, 37.5])
    temb, heads = ref.cond_chain(t, l1, l2, hd)

    def deq(p):
        w, s, b = (torch.from_numpy(a.astype(np.int64) if a.dtype == np.uint32 else a) for a in p)
        codes = (w[..., None] >> (4 * torch.arange(8))) & 15
        codes = codes.reshape(w.shape[0], -1).float()
        return (codes * s.repeat_interleave(64, 1) + b.repeat_interleave(64, 1)).double()

    x = torch.from_numpy(ref.cond_sinusoid(t, sin_dim)).double()
    silu = torch.nn.functional.silu
    tt = x @ deq(l1).T
    tt = silu(tt.float().double()).float().double() @ deq(l2).T
    want_temb = tt.float()
    want_heads = (silu(want_temb.double()).float().double() @ deq(hd).T).float()
    assert np.allclose(temb, want_temb.numpy(), rtol=1e-6, atol=1e-6)
    assert np.allclose(heads, want_heads.numpy(), rtol=1e-6, atol=1e-6)
    sub = ref.cond_chain(t, l1, l2, hd, head_rows=slice(100, 200))[1]
    assert np.array_equal(sub, heads[:, 100:200])


def test_glue_add_t_matches_torch_half_and_bf16_adds():
    """T(float(r) + float(y)): torch's CPU bf16 and f16 adds (float arithmetic
    rounded to the type) are independent implementations of the same step; a
    mutant that adds in T's precision after rounding each to a coarser type,
    or that drops the residual, fails."""
    rng = np.random.default_rng(33)
    y = (rng.standard_normal(6000) * np.exp2(rng.integers(-12, 12, 6000))).astype(np.float32)
    r = (rng.standard_normal(6000) * np.exp2(rng.integers(-12, 12, 6000))).astype(np.float32)
    yb, rb = torch.from_numpy(y).bfloat16(), torch.from_numpy(r).bfloat16()
    got = ref.glue_add_t(yb.float().numpy(), rb.float().numpy(), "bf16")
    want = (rb + yb).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    yh, rh = torch.from_numpy(y).half(), torch.from_numpy(r).half()
    got16 = ref.glue_add_t(yh.float().numpy(), rh.float().numpy(), "f16")
    assert np.array_equal(got16.view(np.uint16), (rh + yh).numpy().view(np.uint16))
    assert not np.array_equal(got, ref.f32_to_bf16(yb.float().numpy()))


# --------------------------------------------------- f16 and the f64 contraction


def test_c_f16_widening_matches_numpy_on_every_pattern():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = cref.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _f16_neighbourhood() -> np.ndarray:
    """Every finite f16 value, every midpoint between consecutive f16 values
    (the ties), and the f32 values one ulp either side of both, both signs,
    plus the overflow boundary and specials."""
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    mids = (v[:-1] + v[1:]) / 2  # exact in f32: at most 12 significant bits
    base = np.concatenate([v, mids, [65504.0, 65520.0, 65536.0, 2.0 ** -24, 2.0 ** -25,
                                     3 * 2.0 ** -26, 2.0 ** -26, 1e-30, 3e38]]).astype(np.float32)
    up = np.nextafter(base, np.float32(np.inf))
    dn = np.nextafter(base, np.float32(0))
    allv = np.concatenate([base, up, dn])
    return np.concatenate([allv, -allv, np.float32([np.inf, -np.inf, 0.0, -0.0])])


def test_c_f16_narrowing_matches_numpy_on_every_tie_and_neighbour():
    v = _f16_neighbourhood()
    got = cref.f32_to_f16(v)
    want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    rng = np.random.default_rng(45)
    r = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    r = r[np.isfinite(r)]
    assert np.array_equal(cref.f32_to_f16(r), r.astype(np.float16).view(np.uint16))
    nan = cref.f32_to_f16(np.float32([np.nan]))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_c_f16_narrowing_matches_exact_rational_rounding():
    """Independent of numpy: 3000 values of the neighbourhood rounded with
    rational arithmetic (11-bit significand, exponents -14..15, ties to even)."""
    v = _f16_neighbourhood()
    v = v[np.isfinite(v)]
    rng = np.random.default_rng(46)
    pick = v[rng.choice(v.size, 3000, replace=False)]
    got = cref.f32_to_f16(pick).view(np.float16).astype(np.float64)
    for xi, gi in zip(pick.tolist(), got.tolist()):
        want = _rne_format(Fraction(xi), 11, -14, 15)
        assert gi == float(want), (xi, gi, want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_c_dequantize_t_matches_pinned_dequant(dtype):
    """The C T-generic dequant equals the numpy one (pinned above against exact
    rational arithmetic) bit for bit, for bf16 and f16 parameters, including
    the f16 parameter grid of zero, subnormal, negative and huge values."""
    p = synth.make_problem(0, 96, 512, seed=47)
    if dtype == "bf16":
        assert np.array_equal(cref.dequantize_t(p.w, p.scales, p.biases, "bf16"),
                              ref.dequantize(p.w, p.scales, p.biases))
        return
    s16 = ref.bf16_to_f32(p.scales).astype(np.float16)
    b16 = ref.bf16_to_f32(p.biases).astype(np.float16)
    want = ref.dequantize_as(p.w, s16, b16, np.float16).view(np.uint16)
    assert np.array_equal(cref.dequantize_t(p.w, s16, b16, "f16"), want)
    vals = _f16_param_values()
    rng = np.random.default_rng(48)
    n = 64
    s = rng.choice(vals, size=(n, 2)).astype(np.float16)
    b = rng.choice(vals, size=(n, 2)).astype(np.float16)
    w = rng.integers(0, 1 << 32, size=(n, 16), dtype=np.uint64).astype(np.uint32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = ref.dequantize_as(w, s, b, np.float16).view(np.uint16)
    got = cref.dequantize_t(w, s, b, "f16")
    same = (got == want) | (np.isnan(got.view(np.float16)) & np.isnan(want.view(np.float16)))
    assert np.all(same)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_c_qmm_t_f64_matches_pinned_float64_product(dtype):
    """The unrounded double contraction equals the numpy float64 product of the
    pinned dequant (same terms, another summation order: agreement to a few
    ulps of double), and its RNE to T equals the pinned oracle's."""
    p = synth.make_problem(9, 200, 1024, seed=49)
    if dtype == "bf16":
        got = cref.qmm_t_f64(p.x, p.w, p.scales, p.biases, "bf16")
        want = ref.qmm_t_f64(p.x, p.w, p.scales, p.biases)
        assert np.array_equal(ref.f64_to_bf16(got), ref.qmm_t(p.x, p.w, p.scales, p.biases))
    else:
        x16 = ref.bf16_to_f32(p.x).astype(np.float16)
        s16 = ref.bf16_to_f32(p.scales).astype(np.float16)
        b16 = ref.bf16_to_f32(p.biases).astype(np.float16)
        got = cref.qmm_t_f64(x16, p.w, s16, b16, "f16")
        want = x16.astype(np.float64) @ ref.dequantize_as(p.w, s16, b16, np.float16).astype(
            np.float64).T
        assert np.array_equal(got.astype(np.float16), ref.qmm_t_as(x16, p.w, s16, b16, np.float16))
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))
    # A transposed-weight mutant (rows read as K-reversed) must fail.
    rev = ref.pack_codes(ref.unpack_codes(p.w)[:, ::-1].copy())
    bad = cref.qmm_t_f64(p.x if dtype == "bf16" else x16, rev,
                         p.scales if dtype == "bf16" else s16,
                         p.biases if dtype == "bf16" else b16, dtype)
    assert np.max(np.abs(bad - want)) > 1e-3 * np.max(np.abs(want))


# ---------------------------------------------------------------- statistics
def test_error_stats_known_answers():
    """The parity bars' statistics (MAE, normwise max error, floored relative
    error, cosine) on planted errors whose values follow by hand."""
    o = np.array([[1.0, -2.0, 4.0, 0.0]])
    y = o + np.array([[0.5, 0.0, -1.0, 0.0]])
    s = ref.error_stats_values(y, o)
    assert s["mae"] == pytest.approx(1.5 / 4)
    assert s["max_abs"] == pytest.approx(1.0)
    assert s["max_rel_normwise"] == pytest.approx(1.0 / 4.0)
    # floor = max(|o|, 1e-3 rms(o)); the largest d / floor is 0.5 / 1.
    assert s["max_rel_floored"] == pytest.approx(0.5)
    # cosine of (1.5, -2, 3, 0) and (1, -2, 4, 0): 17.5 / (sqrt(15.25) sqrt(21)).
    assert s["cosine"] == pytest.approx(17.5 / (np.sqrt(15.25) * np.sqrt(21.0)), rel=1e-12)
    assert s["bit_exact_frac"] == pytest.approx(0.5)
    # Scaling both by the same factor changes neither normwise nor cosine.
    s2 = ref.error_stats_values(8.0 * y, 8.0 * o)
    assert s2["max_rel_normwise"] == pytest.approx(s["max_rel_normwise"])
    assert s2["cosine"] == pytest.approx(s["cosine"], rel=1e-12)
    assert s2["mae"] == pytest.approx(8.0 * s["mae"])
    # Identical outputs: no error, cosine 1; a sign flip: cosine -1.
    z = ref.error_stats_values(o, o)
    assert z["mae"] == 0 and z["max_rel_normwise"] == 0 and z["cosine"] == pytest.approx(1.0)
    assert ref.error_stats_values(-o, o)["cosine"] == pytest.approx(-1.0)


def test_error_stats_bf16_bits_known_answers():
    """error_stats on bf16 bit patterns decodes them first: one output off by
    one bf16 ulp at 1.0 (2^-7) among four."""
    o_vals = np.array([1.0, 2.0, -0.5, 0.25], np.float32)
    o = ref.f32_to_bf16(o_vals)
    y = o.copy()
    y[0] += 1  # 1.0 -> 1.0078125
    s = ref.error_stats(y, o)
    assert s["mae"] == pytest.approx(2.0 ** -7 / 4)
    assert s["max_rel_normwise"] == pytest.approx(2.0 ** -7 / 2.0)
    assert s["bit_exact_frac"] == pytest.approx(0.75)


def test_error_stats_catch_a_dropped_term():
    """A plausible kernel mistake -- one quantization group's contribution
    dropped -- fails every bar the parity tests apply (MAE <= 1e-3, normwise
    <= 1e-2, cosine >= 0.99999), while the correct product passes them."""
    p = synth.make_problem(8, 64, 256, seed=5)
    good = ref.qmm_t(p.x, p.w, p.scales, p.biases)
    s_ok = ref.error_stats(good, good)
    assert s_ok["mae"] <= 1e-3 and s_ok["max_rel_normwise"] <= 1e-2 and s_ok["cosine"] >= 0.99999
    x_bad = p.x.copy()
    x_bad[:, 64:128] = 0  # bf16 zero bits: the second group never enters the sum
    bad = ref.qmm_t(x_bad, p.w, p.scales, p.biases)
    s = ref.error_stats(bad, good)
    assert s["mae"] > 1e-3 and s["max_rel_normwise"] > 1e-2 and s["cosine"] < 0.99999, s

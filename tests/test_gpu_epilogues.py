"""Fused output stages of the MFMA kernel against qmm + glue.

Known answers: the CPU oracle's qmm (RNE_T of the double-accumulated product
with the bit-exact dequant) followed by the reference's glue arithmetic
(oracle/ref.py glue_*, restating Sources/ImarelloDirect/DirectDiTKernels.swift);
and the library's own unfused qmm output followed by the same glue, which the
fused kernels must match (postscale bit-exactly: same accumulator, same
rounding; the others to one unit in the last place / the stated tolerance).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import synth
from oracle import ref

pytestmark = pytest.mark.gpu

MAE_TOL = 1e-3
NORMWISE_TOL = 1e-2
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)
TORCH = {np.float16: torch.float16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def problem(m, n, k, dtype, seed):
    """bf16: the synthetic generator; f16: the same values cast (bf16 values of
    these magnitudes are exact in f16)."""
    p = synth.make_problem(m, n, k, seed=seed)
    x, w, s, b = synth.to_device(p)
    if dtype == "f16":
        x, s, b = x.half(), s.half(), b.half()
    return p, x, w, s, b


def oracle_qmm(p, x, s, b, dtype, rows=None):
    """float32 values of the T-rounded oracle product x . deq(W[rows])^T."""
    w = p.w if rows is None else p.w[rows]
    if dtype == "bf16":
        sb = p.scales if rows is None else p.scales[rows]
        bb = p.biases if rows is None else p.biases[rows]
        return ref.bf16_to_f32(ref.qmm_t(p.x, w, sb, bb))
    sh = s.cpu().numpy() if rows is None else s.cpu().numpy()[rows]
    bh = b.cpu().numpy() if rows is None else b.cpu().numpy()[rows]
    return ref.qmm_t_as(x.cpu().numpy(), w, sh, bh, np.float16).astype(np.float32)


def to_np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def assert_close(y: np.ndarray, want: np.ndarray, what: str) -> None:
    st = ref.error_stats_values(y.astype(np.float64), want.astype(np.float64))
    note(f"  {what}: mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g} "
         f"bit_exact={st['bit_exact_frac']:.4f} cosine={st['cosine']:.7f}")
    assert st["mae"] <= MAE_TOL and st["max_rel_normwise"] <= NORMWISE_TOL, (what, st)
    assert st["cosine"] >= COSINE_MIN, (what, st)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k", [(300, 512, 768), (17, 96, 256), (1, 64, 512)])
def test_postscale(dtype, m, n, k):
    note(f"qmm_postscale {dtype} M={m} N={n} K={k}")
    p, x, w, s, b = problem(m, n, k, dtype, seed=50)
    y = imq.qmm_postscale(x, w, s, b, 16.0)
    assert y.dtype == torch.float32
    unfused = to_np(imq.qgemm(x, w, s, b)) * np.float32(16.0)
    assert np.array_equal(to_np(y), unfused)
    assert_close(to_np(y), ref.glue_postscale(oracle_qmm(p, x, s, b, dtype), 16.0), "postscale")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("inplace", [False, True])
def test_gate_add(dtype, inplace):
    m, n, k = 260, 384, 1024
    note(f"qmm_gate_add {dtype} M={m} N={n} K={k} inplace={inplace}")
    p, x, w, s, b = problem(m, n, k, dtype, seed=51)
    rng = np.random.default_rng(51)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gate = rng.standard_normal(n).astype(np.float32)
    r_dev = torch.from_numpy(res).cuda()
    g_dev = torch.from_numpy(gate).cuda()
    y = imq.qmm_gate_add(x, w, s, b, r_dev, g_dev, 1.0 / 16, out=r_dev if inplace else None)
    got = to_np(y)
    unfused = ref.glue_gate_add(to_np(imq.qgemm(x, w, s, b)), res, gate, 1.0 / 16)
    assert np.max(np.abs(got - unfused) / np.maximum(np.abs(unfused), 1e-30)) <= 2.0 ** -23
    assert_close(got, ref.glue_gate_add(oracle_qmm(p, x, s, b, dtype), res, gate, 1.0 / 16),
                 "gate_add")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("m,width", [(300, 300), (33, 128), (2, 70)])
def test_swiglu_into_a_pitched_buffer(dtype, m, width):
    """gate and up sections of one projection (N=1024 rows), SwiGLU written into
    columns [40, 40 + width) of a wider buffer; the other columns stay as they were."""
    n, k, gate_row, up_row = 1024, 512, 256, 600
    note(f"qmm_swiglu {dtype} M={m} width={width}")
    p, x, w, s, b = problem(m, n, k, dtype, seed=52)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    buf = torch.full((m, width + 100), 7.0, dtype=tdt, device="cuda")
    out = buf[:, 40:40 + width]
    imq.qmm_swiglu(x, w, s, b, width, gate_row, up_row, in_scale=16.0, out_scale=1.0 / 16, out=out)
    got = to_np(buf)
    assert np.all(got[:, :40] == 7.0) and np.all(got[:, 40 + width:] == 7.0)
    ys = got[:, 40:40 + width]
    full = to_np(imq.qgemm(x, w, s, b))
    unfused = ref.glue_swiglu(full[:, gate_row:gate_row + width], full[:, up_row:up_row + width],
                              16.0, 1.0 / 16)
    want = ref.glue_swiglu(oracle_qmm(p, x, s, b, dtype, np.arange(gate_row, gate_row + width)),
                           oracle_qmm(p, x, s, b, dtype, np.arange(up_row, up_row + width)),
                           16.0, 1.0 / 16)

    def round_t(v):
        t = torch.from_numpy(v.astype(np.float32)).to(tdt).float().numpy()
        return t

    assert_close(ys, round_t(unfused), "swiglu vs unfused")
    assert_close(ys, round_t(want), "swiglu vs oracle")


def test_epilogue_argument_checks():
    p, x, w, s, b = problem(8, 128, 256, "bf16", seed=53)
    with pytest.raises(ValueError):
        imq.qmm_swiglu(x, w, s, b, 100, 0, 64)  # up section past N
    with pytest.raises(NotImplementedError):
        imq.qmm_postscale(x.float(), w, s.float(), b.float(), 1.0)  # f32: no MFMA kernel
    with pytest.raises(ValueError):
        imq.qmm_postscale(x[:, :192], w[:, :24], s[:, :3], b[:, :3], 1.0)  # not contiguous


def _t16_bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("count,offset", [(1, 0), (7, 0), (8, 0), (1000003, 0), (4099, 1)])
@pytest.mark.parametrize("scale", [16.0, 3.0, -0.5])
def test_cast_prescale_bit_exact(dtype, count, offset, scale):
    """cast_prescale equals the oracle's (x / s).asType(T) bit for bit: the vector
    kernel (aligned, count / 8 chunks), the scalar tail and the unaligned path
    (y one element into its buffer), with zeros of both signs, f16 overflow and NaN."""
    note(f"cast_prescale {dtype} count={count} offset={offset} scale={scale}")
    rng = np.random.default_rng(count + offset)
    x = (rng.standard_normal(count) * np.exp2(rng.integers(-30, 22, count))).astype(np.float32)
    specials = np.float32([0.0, -0.0, 65520 * 16, np.nan, 16 * (1 + 3 * 2 ** -11)])
    x[:min(count, 5)] = specials[:min(count, 5)]
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    buf = torch.full((count + offset,), 1.5, dtype=tdt, device="cuda")
    out = buf[offset:]
    imq.cast_prescale(torch.from_numpy(x).cuda(), scale, tdt, out=out)
    got = _t16_bits(out)
    want = ref.glue_prescale(x, scale, dtype)
    want = want.view(np.uint16) if dtype == "f16" else want
    nan = np.isnan(x)
    exp_mask, man_mask = (0x7C00, 0x03FF) if dtype == "f16" else (0x7F80, 0x007F)
    assert np.all((got[nan] & exp_mask) == exp_mask) and np.all((got[nan] & man_mask) != 0)
    assert np.array_equal(got[~nan], want[~nan]), np.flatnonzero(got[~nan] != want[~nan])[:8]
    if offset:
        assert torch.all(buf[:offset] == 1.5).item()


@pytest.mark.parametrize("m,n,k", [(300, 512, 768), (1, 64, 512)])
def test_apply_linear_f16_sandwich(m, n, k):
    """apply_linear (x / 16 to f16, f16 qmm, x 16 to f32) equals cast_prescale +
    qmm_postscale bit for bit and the oracle's sandwich within the tolerance."""
    note(f"apply_linear M={m} N={n} K={k}")
    p, x, w, s, b = problem(m, n, k, "f16", seed=60)
    xf = (x.float() * 24.0).reshape((1, m, k))  # float32 activations, |x| up to ~100
    lin = imq.QuantizedLinear(w, s, b)
    y = imq.apply_linear(lin, xf)
    assert y.dtype == torch.float32 and tuple(y.shape) == (1, m, n)
    unfused = imq.qmm_postscale(imq.cast_prescale(xf, 16.0), w, s, b, 16.0)
    assert np.array_equal(to_np(y), to_np(unfused))
    x16 = ref.glue_prescale(xf.cpu().numpy().reshape(m, k), 16.0, "f16")
    q = ref.qmm_t_as(x16, p.w, s.cpu().numpy(), b.cpu().numpy(), np.float16).astype(np.float32)
    assert_close(to_np(y).reshape(m, n), ref.glue_postscale(q, 16.0), "apply_linear")


@pytest.mark.parametrize("count", [0, 1, 1000, 3_000_001])
def test_dynamic_scale_bit_exact(count):
    """dynamic_scale equals the oracle's max(amax|x| / target, 1) bit for bit: a
    negative element holding the amax, amax below the target (scale 1), a NaN
    (NaN), the empty tensor (1); the large case spans many workgroups."""
    note(f"dynamic_scale count={count}")
    rng = np.random.default_rng(count + 3)
    x = (rng.standard_normal(count) * 40).astype(np.float32)
    if count:
        x[rng.integers(count)] = -713.25
    cases = [(x, 64.0), (x, 3.0), (x * np.float32(1e-3), 64.0)]
    if count:
        xn = x.copy()
        xn[count // 2] = np.nan
        cases.append((xn, 64.0))
    for xi, target in cases:
        got = imq.dynamic_scale(torch.from_numpy(xi).cuda(), target).cpu().numpy()
        want = ref.dynamic_scale(xi, target)
        assert got.shape == (1,) and got.dtype == np.float32
        if np.isnan(want):
            assert np.isnan(got[0])
        else:
            assert got[0].view(np.uint32) == want.view(np.uint32), (target, got[0], want)


@pytest.mark.parametrize("m,n,k", [(300, 512, 768), (1, 64, 512), (4096, 256, 128)])
@pytest.mark.parametrize("mode", ["f16_out", "dynamic", "dynamic_f16_out"])
def test_apply_linear_s4_modes(mode, m, n, k):
    """applyLinearCore's S4 modes (AttentionUtils.swift:166-178,198-230): the f16
    result without the f32 upcast, the per-tensor dynamic scale, and both.  The
    device scale equals the oracle's bit for bit, the prescaled input equals the
    oracle's (x / s).asType(f16) bit for bit, the f16 result equals
    f16(y16 * f16(s)) of the library's own f16 qmm bit for bit, apply_linear equals
    the step-by-step composition bit for bit, and the whole sandwich matches the
    oracle's within the tolerance."""
    note(f"apply_linear {mode} M={m} N={n} K={k}")
    p, x, w, s, b = problem(m, n, k, "f16", seed=61)
    rng = np.random.default_rng(61)
    xf_np = (rng.standard_normal((m, k)) * 90).astype(np.float32)
    xf_np[0, 0] = -1500.0  # amax 1500: dynamic scale 23.4375
    xf = torch.from_numpy(xf_np).cuda()
    lin = imq.QuantizedLinear(w, s, b)
    f16_out = mode.endswith("f16_out")
    target = 64.0 if mode.startswith("dynamic") else None
    y = imq.apply_linear(lin, xf, output_f16=f16_out, dynamic_target=target)
    assert y.dtype == (torch.float16 if f16_out else torch.float32) and tuple(y.shape) == (m, n)
    if target is None:
        sc, sd = np.float32(16.0), None
    else:
        sd = imq.dynamic_scale(xf, target)
        sc = ref.dynamic_scale(xf_np, target)
        assert sd.cpu().numpy()[0] == sc == np.float32(1500.0 / 64)
    x16 = imq.cast_prescale(xf, 16.0, scale_dev=sd)
    x16_want = ref.glue_prescale(xf_np, float(sc), "f16")
    assert np.array_equal(x16.cpu().numpy().view(np.uint16), x16_want.view(np.uint16))
    composed = imq.qmm_postscale(x16, w, s, b, 16.0, scale_dev=sd,
                                 out_dtype=torch.float16 if f16_out else torch.float32)
    assert np.array_equal(to_np(y), to_np(composed))
    y16 = imq.qgemm(x16, w, s, b).cpu().numpy()  # the library's own f16 qmm
    if f16_out:
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint16), ref.glue_postscale_f16(y16, float(sc)).view(np.uint16))
    else:
        assert np.array_equal(to_np(y), ref.glue_postscale(y16.astype(np.float32), float(sc)))
    q = ref.qmm_t_as(x16_want, p.w, s.cpu().numpy(), b.cpu().numpy(), np.float16)
    want = ref.glue_postscale_f16(q, float(sc)) if f16_out else ref.glue_postscale(q.astype(np.float32), float(sc))
    assert_close(to_np(y), want.astype(np.float32), f"apply_linear {mode}")


def test_scale_dev_is_read_when_the_kernel_runs():
    """A graph captured with a device scale replays with the value the tensor
    holds at replay time, for the prescale and both post-scale results; a
    captured dynamic_scale recomputes the amax of what x holds at each replay
    (its accumulator cleared by a kernel, not a memset node)."""
    m, n, k = 64, 256, 512
    p, x, w, s, b = problem(m, n, k, "f16", seed=62)
    xf = x.float() * 40
    sd = torch.full((1,), 2.0, device="cuda")
    x16 = torch.empty((m, k), dtype=torch.float16, device="cuda")
    y32 = torch.empty((m, n), device="cuda")
    y16 = torch.empty((m, n), dtype=torch.float16, device="cuda")
    xv = torch.zeros(5000, device="cuda")
    sd2 = torch.empty(1, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(2):  # warm the launchers outside the capture
            imq.dynamic_scale(xv, 64.0, out=sd2)
            imq.cast_prescale(xf, 1.0, out=x16, scale_dev=sd)
            imq.qmm_postscale(x16, w, s, b, 1.0, out=y32, scale_dev=sd)
            imq.qmm_postscale(x16, w, s, b, 1.0, out=y16, out_dtype=torch.float16, scale_dev=sd)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            imq.dynamic_scale(xv, 64.0, out=sd2)
            imq.cast_prescale(xf, 1.0, out=x16, scale_dev=sd)
            imq.qmm_postscale(x16, w, s, b, 1.0, out=y32, scale_dev=sd)
            imq.qmm_postscale(x16, w, s, b, 1.0, out=y16, out_dtype=torch.float16, scale_dev=sd)
    rng = np.random.default_rng(62)
    for i, val in enumerate((4.0, 23.4375, 2.0)):
        xv_np = (rng.standard_normal(5000) * 10 ** i * 30).astype(np.float32)
        xv.copy_(torch.from_numpy(xv_np))
        sd.fill_(val)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert sd2.cpu().numpy()[0] == ref.dynamic_scale(xv_np, 64.0), i
        e16 = imq.cast_prescale(xf, val)
        assert torch.equal(x16, e16), val
        assert torch.equal(y32, imq.qmm_postscale(e16, w, s, b, val)), val
        assert torch.equal(y16, imq.qmm_postscale(e16, w, s, b, val, out_dtype=torch.float16)), val


def test_s4_argument_checks():
    p, x, w, s, b = problem(8, 128, 256, "f16", seed=63)
    xf = x.float()
    with pytest.raises(ValueError):
        imq.dynamic_scale(x)  # float32 only
    with pytest.raises(imq.ImqInvalid):
        imq.dynamic_scale(xf, 0.0)
    with pytest.raises(ValueError):
        imq.cast_prescale(xf, scale_dev=torch.ones(2, device="cuda"))  # one element
    with pytest.raises(ValueError):
        imq.qmm_postscale(x, w, s, b, 1.0, out_dtype=torch.bfloat16)
    pb, xb, wb, sb, bb = problem(8, 128, 256, "bf16", seed=63)
    with pytest.raises(imq.ImqUnsupported):
        imq.qmm_postscale(xb, wb, sb, bb, 1.0, out_dtype=torch.float16)  # f16 result, bf16 qmm


def test_prescale_argument_checks():
    x = torch.ones(16, device="cuda")
    with pytest.raises(ValueError):
        imq.cast_prescale(x.half())  # x must be float32
    with pytest.raises(imq.ImqInvalid):
        imq.cast_prescale(x, 0.0)  # scale 0
    with pytest.raises(imq.ImqInvalid):
        imq.cast_prescale(x, float("inf"))
    p, xb, w, s, b = problem(8, 128, 256, "bf16", seed=54)
    with pytest.raises(ValueError):
        imq.apply_linear(imq.QuantizedLinear(w, s, b), xb.float())  # bf16 scales


# ------------------------------------- output stages on the register-staged kernel


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_x_embedder_sandwich_k128(dtype):
    """The DiT's x_embedder at 1024^2: latents [4096, 128] fp32 / 16 to T, the qmm
    with K = 128 (not a multiple of 256: the register-staged kernel) and the x16
    post-scale to fp32 (DirectDiTStep.swift:917-941), against the oracle's
    prescale, qmm and postscale; f16 through apply_linear, the operator surface."""
    m, n, k = 4096, 3072, 128
    note(f"x_embedder sandwich {dtype} M={m} N={n} K={k}")
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    plan = imq.qmm_plan(m, n, k, tdt, entry="fused")
    assert plan["kernel"] == "tile_reg" and plan["splits"] == 1, plan
    p, _, w, s, b = problem(1, n, k, dtype, seed=54)
    rng = np.random.default_rng(54)
    lat = rng.standard_normal((m, k)).astype(np.float32)
    lat_d = torch.from_numpy(lat).cuda()
    if dtype == "f16":
        y = imq.apply_linear(imq.QuantizedLinear(w, s, b), lat_d, 16.0)
    else:
        y = imq.qmm_postscale(imq.cast_prescale(lat_d, 16.0, tdt), w, s, b, 16.0)
    got = to_np(y)
    x_t = ref.glue_prescale(lat, 16.0, dtype)
    if dtype == "f16":
        q = ref.qmm_t_as(x_t, p.w, s.cpu().numpy(), b.cpu().numpy(), np.float16).astype(np.float32)
    else:
        q = ref.bf16_to_f32(ref.qmm_t(x_t, p.w, p.scales, p.biases))
    assert_close(got, ref.glue_postscale(q, 16.0), "x_embedder sandwich")
    unfused = to_np(imq.qgemm(imq.cast_prescale(lat_d, 16.0, tdt), w, s, b)) * np.float32(16.0)
    assert np.array_equal(got, unfused)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_gate_add_register_kernel_k192(dtype):
    m, n, k = 300, 384, 192
    note(f"qmm_gate_add (register-staged) {dtype} M={m} N={n} K={k}")
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    assert imq.qmm_plan(m, n, k, tdt, entry="fused")["kernel"] == "tile_reg"
    p, x, w, s, b = problem(m, n, k, dtype, seed=55)
    rng = np.random.default_rng(55)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gate = rng.standard_normal(n).astype(np.float32)
    r_dev = torch.from_numpy(res).cuda()
    y = imq.qmm_gate_add(x, w, s, b, r_dev, torch.from_numpy(gate).cuda(), 0.3, out=r_dev)
    got = to_np(y)
    unfused = ref.glue_gate_add(to_np(imq.qgemm(x, w, s, b)), res, gate, 0.3)
    assert np.array_equal(got, unfused)
    assert_close(got, ref.glue_gate_add(oracle_qmm(p, x, s, b, dtype), res, gate, 0.3),
                 "gate_add k192")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_swiglu_register_kernel_k192_pitched(dtype):
    """A gate/up pair on the register-staged kernel (K = 192), written into
    columns [8, 8 + width) of a wider buffer; a partial last tile of outputs."""
    m, n, k, width, gate_row, up_row = 130, 600, 192, 200, 17, 300
    note(f"qmm_swiglu (register-staged) {dtype} M={m} width={width} K={k}")
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    assert imq.qmm_plan(m, 2 * width, k, tdt, entry="swiglu")["kernel"] == "tile_reg"
    p, x, w, s, b = problem(m, n, k, dtype, seed=56)
    buf = torch.full((m, width + 20), 5.0, dtype=tdt, device="cuda")
    imq.qmm_swiglu(x, w, s, b, width, gate_row, up_row, in_scale=16.0, out_scale=1.0 / 16,
                   out=buf[:, 8:8 + width])
    got = to_np(buf)
    assert np.all(got[:, :8] == 5.0) and np.all(got[:, 8 + width:] == 5.0)
    full = to_np(imq.qgemm(x, w, s, b))
    unfused = ref.glue_swiglu(full[:, gate_row:gate_row + width], full[:, up_row:up_row + width],
                              16.0, 1.0 / 16)
    want = ref.glue_swiglu(oracle_qmm(p, x, s, b, dtype, np.arange(gate_row, gate_row + width)),
                           oracle_qmm(p, x, s, b, dtype, np.arange(up_row, up_row + width)),
                           16.0, 1.0 / 16)

    def round_t(v):
        return torch.from_numpy(v.astype(np.float32)).to(tdt).float().numpy()

    assert_close(got[:, 8:8 + width], round_t(unfused), "swiglu k192 vs unfused")
    assert_close(got[:, 8:8 + width], round_t(want), "swiglu k192 vs oracle")

"""The kernel instances the DiT runs, at its production shapes, against the oracle.

The DiT step's trace runs the tile kernel at 192-, 224- and 256-row tiles
with the plain, gated-residual and SwiGLU output stages (f16), the double
blocks' image and text chains each planned for their share of the CUs.  The
tests here run those shapes through the C entry points (asserting, through
imq_qmm_plan, the tile height each takes) and the whole step at its full
size (5 double + 20 single blocks, 4096 image + 512 text rows, dim 3072,
ff_inner 9216), in f16 and bf16.

Oracle: every op on the path is row-local (RMSNorm per row, qmm per row,
SwiGLU and the gated residual per element), so the CPU oracle follows a few
sampled rows through the full-size problem: RNE_T of the double-accumulated
product with the bit-exact dequant (oracle.cref.qmm_t_f64), then the
reference's glue arithmetic (oracle.ref glue_*).  Bars as in the other GPU
tests: MAE <= 1e-3, normwise max error <= 1e-2, cosine >= 0.99999 per
projection; the step's final fp32 residual within normwise 1e-2, and graph
replays equal to the eager launches bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import synth
from aestrix_amd.step import DitDims, DitStep, random_head, random_projections
from oracle import cref, ref

pytestmark = pytest.mark.gpu

MAE_TOL = 1e-3
NORMWISE_TOL = 1e-2
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)
TDT = {"bf16": torch.bfloat16, "f16": torch.float16}


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def host_bits(t: torch.Tensor) -> np.ndarray:
    """A bf16 / f16 device tensor as uint16 bit patterns on the host."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def t_values(bits: np.ndarray, dtype: str) -> np.ndarray:
    """T bit patterns -> float64 values."""
    if dtype == "bf16":
        return ref.bf16_to_f32(bits).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def round_t(v: np.ndarray, dtype: str) -> np.ndarray:
    """float64 values -> T bit patterns, rounded once (RNE)."""
    if dtype == "bf16":
        return ref.f64_to_bf16(v)
    return np.asarray(v, np.float64).astype(np.float16).view(np.uint16)


def oracle_qmm(x_bits, w, s_bits, b_bits, dtype) -> np.ndarray:
    """float64 values of RNE_T(x . deq_T(W)^T) (T bit patterns in)."""
    return t_values(round_t(cref.qmm_t_f64(x_bits, w, s_bits, b_bits, dtype), dtype), dtype)


def assert_close(y: np.ndarray, want: np.ndarray, what: str) -> None:
    st = ref.error_stats_values(np.asarray(y, np.float64), np.asarray(want, np.float64))
    note(f"  {what}: mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g} "
         f"bit_exact={st['bit_exact_frac']:.4f} cosine={st['cosine']:.7f}")
    assert st["mae"] <= MAE_TOL and st["max_rel_normwise"] <= NORMWISE_TOL, (what, st)
    assert st["cosine"] >= COSINE_MIN, (what, st)


def problem(m, n, k, dtype, seed, x_scale=1.0):
    """Seeded problem on the device in T; the host copies are the device's bytes."""
    p = synth.make_problem(m, n, k, seed=seed)
    x, w, s, b = synth.to_device(p)
    x = x * x_scale  # a power of two: exact
    if dtype == "f16":
        x, s, b = x.half(), s.half(), b.half()
    return p.w, x, w, s, b


def sample_rows(m: int, count: int) -> np.ndarray:
    return np.unique(np.linspace(0, m - 1, count).astype(np.int64))


# --------------------------------------------- fused stages at step tile heights


# (M, N weight rows, K, width, gate_row, up_row, tile rows): the single block's
# to_qkv_mlp_proj MLP half (J = 4608), the double blocks' ff.linear_in over the
# image rows (4096) and ff_context.linear_in over the text rows (512); 1024
# rows of a 9216-row pair take 160-row tiles (7 x 36 = 252 tiles, one round).
SWIGLU = [(4608, 27648, 3072, 9216, 9216, 18432, 224),
          (4096, 18432, 3072, 9216, 0, 9216, 256),
          (512, 18432, 3072, 9216, 0, 9216, 192),
          (1024, 9216, 3072, 4608, 0, 4608, 160)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", SWIGLU, ids=[f"M{c[0]}" for c in SWIGLU])
def test_swiglu_at_production_tile_heights(dtype, case):
    m, n, k, width, gate_row, up_row, tile_rows = case
    note(f"qmm_swiglu {dtype} M={m} N={n} K={k} width={width} gate_row={gate_row} "
         f"up_row={up_row} seed=80")
    plan = imq.qmm_plan(m, 2 * width, k, TDT[dtype], entry="swiglu")
    note(f"  plan {plan}")
    assert plan["kernel"] == "tile" and plan["tile_rows"] == tile_rows and plan["splits"] == 1
    # x / 16 with the reference's in/out scales 16 and 1/16 (the f16 protocol
    # of dd_swiglu_pitched, DirectDiTStep.swift:521-543).
    w_h, x, w, s, b = problem(m, n, k, dtype, seed=80, x_scale=1.0 / 16)
    y = imq.qmm_swiglu(x, w, s, b, width, gate_row, up_row, in_scale=16.0, out_scale=1.0 / 16)
    rows = sample_rows(m, 24)
    got = t_values(host_bits(y)[rows], dtype)
    xb, sb, bb = host_bits(x)[rows], host_bits(s), host_bits(b)
    g = oracle_qmm(xb, w_h[gate_row:gate_row + width], sb[gate_row:gate_row + width],
                   bb[gate_row:gate_row + width], dtype)
    u = oracle_qmm(xb, w_h[up_row:up_row + width], sb[up_row:up_row + width],
                   bb[up_row:up_row + width], dtype)
    want = t_values(round_t(ref.glue_swiglu(g, u, 16.0, 1.0 / 16), dtype), dtype)
    assert np.all(np.isfinite(got))
    assert_close(got, want, f"swiglu M={m} rows={len(rows)}")


# (M, N, K, tile rows): the single block's to_out (K = 12288) over J = 4608
# rows and the double blocks' ff.linear_out (K = 9216) over the image rows;
# 1024 x 9216 at K = 3072 takes 160-row tiles.
GATE_ADD = [(4608, 3072, 12288, 224), (4096, 3072, 9216, 224), (1024, 9216, 3072, 160)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", GATE_ADD, ids=[f"M{c[0]}_K{c[2]}" for c in GATE_ADD])
def test_gate_add_at_production_tile_heights(dtype, case):
    m, n, k, tile_rows = case
    note(f"qmm_gate_add {dtype} M={m} N={n} K={k} seed=81 (in place)")
    plan = imq.qmm_plan(m, n, k, TDT[dtype], entry="fused")
    note(f"  plan {plan}")
    assert plan["kernel"] == "tile" and plan["tile_rows"] == tile_rows and plan["splits"] == 1
    w_h, x, w, s, b = problem(m, n, k, dtype, seed=81, x_scale=1.0 / 16)
    rng = np.random.default_rng(81)
    res = rng.standard_normal((m, n)).astype(np.float32)
    gate = rng.standard_normal(n).astype(np.float32)
    r_dev = torch.from_numpy(res).cuda()
    y = imq.qmm_gate_add(x, w, s, b, r_dev, torch.from_numpy(gate).cuda(), 16.0, out=r_dev)
    torch.cuda.synchronize()
    rows = sample_rows(m, 32)
    got = y.cpu().numpy()[rows]
    v = oracle_qmm(host_bits(x)[rows], w_h, host_bits(s), host_bits(b), dtype)
    want = ref.glue_gate_add(v.astype(np.float32), res[rows], gate, 16.0)
    assert_close(got, want, f"gate_add M={m} K={k} rows={len(rows)}")


# (M, N, K, tile rows, tile columns, splits): the double blocks' Q/K/V over
# image rows and text rows (64 x 128 tiles: 192 of them), the image rows'
# MLP-in width as a plain store (256-row tiles), the 1024-row MLP-in qGEMM
# (160-row tiles: 252 tiles in one round on 256 CUs), and the text encoder's
# q/k/v, o and down at L = 512 (128- and 64-row tiles of 128 columns; down
# split three ways).
PLAIN = [(4096, 3072, 3072, 224, 256, 1), (512, 3072, 3072, 64, 128, 1),
         (4096, 18432, 3072, 256, 256, 1), (1024, 9216, 3072, 160, 256, 1),
         (512, 6144, 2560, 128, 128, 1), (512, 2560, 4096, 64, 128, 1),
         (512, 2560, 9728, 128, 128, 3)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("case", PLAIN, ids=[f"M{c[0]}_N{c[1]}_K{c[2]}" for c in PLAIN])
def test_plain_qmm_at_production_tile_heights(dtype, case):
    m, n, k, tile_rows, tile_cols, splits = case
    note(f"qmm_t {dtype} M={m} N={n} K={k} seed=82")
    plan = imq.qmm_plan(m, n, k, TDT[dtype])
    note(f"  plan {plan}")
    assert plan["kernel"] == "tile" and plan["tile_rows"] == tile_rows
    assert plan["tile_cols"] == tile_cols and plan["splits"] == splits
    w_h, x, w, s, b = problem(m, n, k, dtype, seed=82)
    y = imq.quantized_matmul(x, w, s, b)
    rows = sample_rows(m, 32)
    got = t_values(host_bits(y)[rows], dtype)
    want = oracle_qmm(host_bits(x)[rows], w_h, host_bits(s), host_bits(b), dtype)
    assert_close(got, want, f"qmm_t M={m} N={n} rows={len(rows)}")


# -------------------------------------------------------- the full-size step


def oracle_step_rows(d: DitDims, hp, norm_w, gates, X0, txt_rows, img_rows, dtype):
    """Final fp32 residual rows of the step, following `txt_rows` (of the l_txt
    text rows) and `img_rows` (of the l_img image rows) through every block.
    hp: per projection (w, scale bits, bias bits) on the host.  X0: the
    sampled rows of the initial joint residual, text rows first."""
    dim, ffi = d.dim, d.ff_inner
    nt = len(txt_rows)
    X = X0.astype(np.float32).copy()
    T, I = slice(0, nt), slice(nt, None)

    def rms(Xr):
        return round_t(ref.rmsnorm_rows(Xr, norm_w), dtype)

    def qmm(x_bits, q, rows=None):
        w, s, b = hp[q]
        if rows is not None:
            w, s, b = w[rows], s[rows], b[rows]
        return oracle_qmm(x_bits, w, s, b, dtype)

    def swiglu(x_bits, q, gate_row, up_row):
        g = qmm(x_bits, q, slice(gate_row, gate_row + ffi))
        u = qmm(x_bits, q, slice(up_row, up_row + ffi))
        return round_t(ref.glue_swiglu(g, u, 1.0, 1.0), dtype)

    def gate_add(v, Xr, gate):
        return ref.glue_gate_add(v.astype(np.float32), Xr, gate, 1.0)

    for blk in range(d.n_double):
        base = 12 * blk
        g = gates[4 * blk:4 * blk + 4]
        nX = rms(X)
        v_i = round_t(qmm(nX[I], base + 2), dtype)   # to_v over image rows
        X[I] = gate_add(qmm(v_i, base + 6), X[I], g[0])
        if nt:
            v_t = round_t(qmm(nX[T], base + 5), dtype)   # add_v_proj over text rows
            X[T] = gate_add(qmm(v_t, base + 7), X[T], g[1])
        nX = rms(X)
        X[I] = gate_add(qmm(swiglu(nX[I], base + 8, 0, ffi), base + 9), X[I], g[2])
        if nt:
            X[T] = gate_add(qmm(swiglu(nX[T], base + 10, 0, ffi), base + 11), X[T], g[3])
    for blk in range(d.n_single):
        base = 12 * d.n_double + 2 * blk
        g = gates[4 * d.n_double + blk]
        nX = rms(X)
        sw = swiglu(nX, base, 3 * dim, 3 * dim + ffi)
        # C = [attention half (zeros) | SwiGLU]; the zero half adds exact zeros.
        C = np.zeros((X.shape[0], dim + ffi), np.uint16)
        C[:, dim:] = sw
        X = gate_add(qmm(C, base + 1), X, g)
    return X


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_full_size_step_sampled_rows_and_graph_replays(dtype):
    d = DitDims()
    note(f"dit step {dtype} full size {d} seed=83")
    tdt = TDT[dtype]
    projs = random_projections(d, tdt, seed=83)
    step = DitStep(d, projs)
    try:
        rng = np.random.default_rng(83)
        norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
        gates = (0.5 * rng.standard_normal((4 * d.n_double + d.n_single, d.dim))).astype(np.float32)
        step.set_conditioning(torch.from_numpy(norm_w).cuda(), torch.from_numpy(gates).cuda())
        h = rng.standard_normal((d.l_img, d.dim)).astype(np.float32)
        e = rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)
        h_d, e_d = torch.from_numpy(h).cuda(), torch.from_numpy(e).cuda()
        eager = step.run(h_d, e_d, use_graph=False).cpu().numpy()
        assert step.launches == d.n_double * 14 + d.n_single * 4
        assert np.all(np.isfinite(eager))
        for rep in range(3):  # replays with other device work in between
            torch.randn(1000, device="cuda").sum().item()
            graph = step.run(h_d, e_d, use_graph=True).cpu().numpy()
            assert np.array_equal(graph, eager), f"graph replay {rep} differs from eager"
        note("  graph == eager over 3 replays; oracle on sampled rows ...")
        hp = [(q.w.cpu().numpy().view(np.uint32), host_bits(q.s), host_bits(q.b)) for q in projs]
    finally:
        step.close()
    txt_rows = sample_rows(d.l_txt, 8)
    img_rows = sample_rows(d.l_img, 16)
    X0 = np.concatenate([e[txt_rows], h[img_rows]])
    want = oracle_step_rows(d, hp, norm_w, gates, X0, txt_rows, img_rows, dtype)
    got = np.concatenate([eager[txt_rows], eager[d.l_txt + img_rows]])
    diff = np.abs(got.astype(np.float64) - want)
    normwise = diff.max() / np.abs(want).max()
    mean_rel = diff.mean() / np.abs(want).mean()
    note(f"  {len(txt_rows)} text + {len(img_rows)} image rows: normwise={normwise:.3g} "
         f"mean_rel={mean_rel:.3g}")
    assert normwise <= NORMWISE_TOL, normwise


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_full_size_block_qkv_projections_sampled_rows(dtype):
    """The projections the stand-in step computes but never feeds on (its
    attention stand-in uses V only): every double block's to_q / to_k / to_v
    over the 4096 image rows and add_q / add_k / add_v over the 512 text rows,
    and every single block's Q/K/V rows of to_qkv_mlp_proj over all 4608 rows,
    at full size through the block halves on the stand-in norm of one residual,
    checked on sampled rows against the oracle (MAE, normwise, cosine)."""
    d = DitDims()
    note(f"dit q/k/v projections {dtype} full size {d} seed=86")
    tdt = TDT[dtype]
    projs = random_projections(d, tdt, seed=86)
    step = DitStep(d, projs)
    txt_rows = sample_rows(d.l_txt, 8)
    img_rows = sample_rows(d.l_img, 16)
    rows = np.concatenate([txt_rows, d.l_txt + img_rows])
    try:
        rng = np.random.default_rng(86)
        norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
        step.set_conditioning(torch.from_numpy(norm_w).cuda(), None)
        X = rng.standard_normal((d.joint, d.dim)).astype(np.float32)
        x = torch.from_numpy(X).cuda()
        q, k, v = (torch.empty((d.joint, d.dim), dtype=tdt, device="cuda") for _ in range(3))
        qkv = torch.empty((d.joint, 3 * d.dim), dtype=tdt, device="cuda")
        concat = torch.empty((d.joint, d.dim + d.ff_inner), dtype=tdt, device="cuda")
        got = []
        for b in range(d.n_double):
            step.double_attn_in(b, x, q, k, v)
            got.append([host_bits(t)[rows] for t in (q, k, v)])
        for b in range(d.n_single):
            step.single_attn_in(b, x, qkv, concat)
            got.append([host_bits(qkv)[rows]])
        assert np.array_equal(x.cpu().numpy(), X), "the input halves wrote the residual"
        hp = [(q_.w.cpu().numpy().view(np.uint32), host_bits(q_.s), host_bits(q_.b)) for q_ in projs]
    finally:
        step.close()
    nX = round_t(ref.rmsnorm_rows(X[rows], norm_w), dtype)
    nt = len(txt_rows)
    for b in range(d.n_double):
        for i, name in enumerate("qkv"):
            want_i = oracle_qmm(nX[nt:], *hp[12 * b + i], dtype)
            want_t = oracle_qmm(nX[:nt], *hp[12 * b + 3 + i], dtype)
            assert_close(t_values(got[b][i][nt:], dtype), want_i, f"double {b} to_{name} image rows")
            assert_close(t_values(got[b][i][:nt], dtype), want_t, f"double {b} add_{name} text rows")
    for b in range(d.n_single):
        w, sb, bb = hp[12 * d.n_double + 2 * b]
        want = oracle_qmm(nX, w[:3 * d.dim], sb[:3 * d.dim], bb[:3 * d.dim], dtype)
        assert_close(t_values(got[d.n_double + b][0], dtype), want, f"single {b} Q/K/V rows")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_full_size_denoise_step_sampled_rows(dtype):
    """encodeDenoiseStep at full size: the x_embedder sandwich (K = 128), the 25
    blocks and the head (norm / 16, proj_out N = 128, Euler gate-add with 16 dt)
    as one graph; two graph replays with different dt equal eager runs, and the
    update lat_out - lat_in of sampled image rows matches the oracle (image rows
    never mix with other rows on this path)."""
    d = DitDims()
    channels = 128
    note(f"dit denoise {dtype} full size {d} C={channels} seed=84")
    tdt = TDT[dtype]
    projs = random_projections(d, tdt, seed=84)
    xe, po = random_head(d, channels, tdt, seed=85)
    step = DitStep(d, projs)
    try:
        step.set_head(xe, po)
        rng = np.random.default_rng(84)
        norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
        gates = (0.5 * rng.standard_normal((4 * d.n_double + d.n_single, d.dim))).astype(np.float32)
        step.set_conditioning(torch.from_numpy(norm_w).cuda(), torch.from_numpy(gates).cuda())
        lat = rng.standard_normal((d.l_img, channels)).astype(np.float32)
        e = rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)
        lat_d, e_d = torch.from_numpy(lat).cuda(), torch.from_numpy(e).cuda()
        eager = {dt: step.denoise(lat_d, e_d, dt, use_graph=False).cpu().numpy()
                 for dt in (-0.25, -0.1)}
        assert step.launches == d.n_double * 14 + d.n_single * 4 + 4
        for dt in (-0.1, -0.25):
            torch.randn(1000, device="cuda").sum().item()
            got = step.denoise(lat_d, e_d, dt, use_graph=True).cpu().numpy()
            assert np.array_equal(got, eager[dt]), f"graph replay with dt={dt} differs"
        hp = [(q.w.cpu().numpy().view(np.uint32), host_bits(q.s), host_bits(q.b)) for q in projs]
        xe_h = (xe.w.cpu().numpy().view(np.uint32), host_bits(xe.s), host_bits(xe.b))
        po_h = (po.w.cpu().numpy().view(np.uint32), host_bits(po.s), host_bits(po.b))
    finally:
        step.close()
    img_rows = sample_rows(d.l_img, 16)
    lat16 = ref.glue_prescale(lat[img_rows], 16.0, dtype)
    lat16 = lat16.view(np.uint16) if dtype == "f16" else lat16
    h = ref.glue_postscale(oracle_qmm(lat16, *xe_h, dtype).astype(np.float32), 16.0)
    X = oracle_step_rows(d, hp, norm_w, gates, h, np.arange(0), img_rows, dtype)
    nH = round_t(ref.rmsnorm_rows(X, norm_w) / 16.0, dtype)
    pred = oracle_qmm(nH, *po_h, dtype)
    dt = -0.25
    want = ref.glue_gate_add(pred.astype(np.float32), lat[img_rows], np.ones(channels, np.float32),
                             np.float32(16.0) * np.float32(dt))
    upd = eager[dt][img_rows].astype(np.float64) - lat[img_rows]
    upd_want = want.astype(np.float64) - lat[img_rows]
    normwise = np.abs(upd - upd_want).max() / np.abs(upd_want).max()
    note(f"  {len(img_rows)} image rows: update normwise={normwise:.3g}")
    assert np.all(np.isfinite(eager[dt]))
    assert normwise <= NORMWISE_TOL, normwise


# ---------------------------------------- text-encoder MLP-in at decode sizes


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_swiglu_few_rows_on_the_qgemv(dtype, m):
    """The text encoder's gate and up projections ([9728 x 2560] each, rows
    concatenated) with dq_silu_mul (DirectGlueKernels.swift:77-88) as one
    qmm_swiglu call at decode sizes: the qGEMV's pair mode (one launch streams
    both sections, the gate and up rows of an output read by one lane group).
    Against the oracle on every row."""
    inter, k = 9728, 2560
    note(f"qmm_swiglu (qGEMV pair) {dtype} M={m} width={inter} K={k} seed=86")
    plan = imq.qmm_plan(m, 2 * inter, k, TDT[dtype], entry="swiglu")
    assert plan["kernel"] == "qgemv", plan
    w_h, x, w, s, b = problem(m, 2 * inter, k, dtype, seed=86)
    y = imq.qmm_swiglu(x, w, s, b, inter, 0, inter)
    got = t_values(host_bits(y), dtype)
    xb, sb, bb = host_bits(x), host_bits(s), host_bits(b)
    g = oracle_qmm(xb, w_h[:inter], sb[:inter], bb[:inter], dtype)
    u = oracle_qmm(xb, w_h[inter:], sb[inter:], bb[inter:], dtype)
    want = t_values(round_t(ref.glue_swiglu(g, u, 1.0, 1.0), dtype), dtype)
    assert_close(got, want, f"swiglu qGEMV pair M={m}")

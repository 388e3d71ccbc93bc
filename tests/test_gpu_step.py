"""Whole-step replay (include/imq_step.h) against a CPU restatement.

The oracle runs the same block sequence in numpy with the CPU oracle's qmm
(RNE_T of the double-accumulated product, bit-exact dequant) and the glue
stages of oracle/ref.py, rounding to T wherever the device stores T.  The
step compounds roundings over its blocks, so the bar is on the final fp32
residual: normwise error <= 1e-2 (mean relative error is reported).  Graph
replays must equal the eager launch sequence bit for bit, also when replayed
several times with other device work in between.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from aestrix_amd import _lib
from aestrix_amd.step import DitDims, DitStep, random_head, random_projections
from oracle import ref

pytestmark = pytest.mark.gpu

TINY = DitDims(l_img=64, l_txt=32, dim=256, ff_inner=256, n_double=2, n_single=2)
# Few output tiles and K of 512..1536: every projection splits K, the fused
# gated-residual and SwiGLU stages applied after the partial sums are added.
SPLIT = DitDims(l_img=128, l_txt=64, dim=512, ff_inner=1024, n_double=1, n_single=1)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def to_t(v: np.ndarray, tdt) -> np.ndarray:
    v = np.asarray(v, np.float32)
    if tdt == torch.float16:
        return v.astype(np.float16).astype(np.float32)
    return ref.bf16_to_f32(ref.f32_to_bf16(v))


def qmm_t(x_t: np.ndarray, q, tdt) -> np.ndarray:
    w = q.w.cpu().numpy().view(np.uint32)
    if tdt == torch.float16:
        s = q.s.cpu().numpy()
        b = q.b.cpu().numpy()
        return ref.qmm_t_as(x_t.astype(np.float16), w, s, b, np.float16).astype(np.float32)
    s = q.s.cpu().view(torch.int16).numpy().view(np.uint16)
    b = q.b.cpu().view(torch.int16).numpy().view(np.uint16)
    return ref.bf16_to_f32(ref.qmm_t(ref.f32_to_bf16(x_t), w, s, b))


def sub(q, rows):
    """The projection restricted to weight rows `rows` (a slice)."""
    from aestrix_amd.ops import Q
    return Q(w=q.w[rows], s=q.s[rows], b=q.b[rows], n=rows.stop - rows.start, k=q.k)


def oracle_step(d: DitDims, projs, norm_w, gates, h, e, tdt):
    X = np.concatenate([e, h]).astype(np.float32)
    T, I = slice(0, d.l_txt), slice(d.l_txt, d.joint)
    dim, ffi = d.dim, d.ff_inner

    def rms(X):
        return to_t(ref.rmsnorm_rows(X, norm_w), tdt)

    def swiglu(x_t, q, gate_row, up_row):
        g = qmm_t(x_t, sub(q, slice(gate_row, gate_row + ffi)), tdt)
        u = qmm_t(x_t, sub(q, slice(up_row, up_row + ffi)), tdt)
        return to_t(ref.glue_swiglu(g, u, 1.0, 1.0), tdt)

    for b in range(d.n_double):
        W = projs[12 * b:12 * b + 12]
        g = gates[4 * b:4 * b + 4]
        nX = rms(X)
        V = np.zeros((d.joint, dim), np.float32)
        for q in range(3):
            out_i = qmm_t(nX[I], W[q], tdt)
            out_t = qmm_t(nX[T], W[3 + q], tdt)
            if q == 2:
                V[I], V[T] = out_i, out_t
        X[I] = ref.glue_gate_add(qmm_t(V[I], W[6], tdt), X[I], g[0], 1.0)
        X[T] = ref.glue_gate_add(qmm_t(V[T], W[7], tdt), X[T], g[1], 1.0)
        nX = rms(X)
        sw_i = swiglu(nX[I], W[8], 0, ffi)
        X[I] = ref.glue_gate_add(qmm_t(sw_i, W[9], tdt), X[I], g[2], 1.0)
        sw_t = swiglu(nX[T], W[10], 0, ffi)
        X[T] = ref.glue_gate_add(qmm_t(sw_t, W[11], tdt), X[T], g[3], 1.0)
    for b in range(d.n_single):
        W = projs[12 * d.n_double + 2 * b:12 * d.n_double + 2 * b + 2]
        g = gates[4 * d.n_double + b]
        nX = rms(X)
        C = np.zeros((d.joint, dim + ffi), np.float32)  # attention half stays zero
        C[:, dim:] = swiglu(nX, W[0], 3 * dim, 3 * dim + ffi)
        X = ref.glue_gate_add(qmm_t(C, W[1], tdt), X, g, 1.0)
    return X


@pytest.mark.parametrize("d", [TINY, SPLIT], ids=["tiny", "split_k"])
@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_step_matches_oracle_and_graph_matches_eager(tdt, d):
    note(f"dit step {tdt} {d}")
    projs = random_projections(d, tdt, seed=7)
    step = DitStep(d, projs)
    rng = np.random.default_rng(7)
    norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
    gates = (0.5 * rng.standard_normal((4 * d.n_double + d.n_single, d.dim))).astype(np.float32)
    step.set_conditioning(torch.from_numpy(norm_w).cuda(), torch.from_numpy(gates).cuda())
    h = rng.standard_normal((d.l_img, d.dim)).astype(np.float32)
    e = rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)
    h_d, e_d = torch.from_numpy(h).cuda(), torch.from_numpy(e).cuda()
    eager = step.run(h_d, e_d, use_graph=False).cpu().numpy()
    assert step.launches == d.n_double * 14 + d.n_single * 4
    assert np.array_equal(h_d.cpu().numpy(), h) and np.array_equal(e_d.cpu().numpy(), e)
    for rep in range(3):  # replays with other device work in between
        torch.randn(1000, device="cuda").sum().item()
        graph = step.run(h_d, e_d, use_graph=True).cpu().numpy()
        assert np.array_equal(graph, eager), f"graph replay {rep} differs from eager"
    want = oracle_step(d, projs, norm_w, gates, h, e, tdt)
    diff = np.abs(eager.astype(np.float64) - want)
    normwise = diff.max() / np.abs(want).max()
    mean_rel = diff.mean() / np.abs(want).mean()
    note(f"  normwise={normwise:.3g} mean_rel={mean_rel:.3g}")
    assert np.all(np.isfinite(eager))
    assert normwise <= 1e-2, normwise
    step.close()


def oracle_denoise(d: DitDims, projs, head, norm_w, gates, lat, e, dt, tdt):
    """encodeDenoiseStep on the CPU: x_embedder sandwich (x / 16 to T, qmm, x 16),
    the blocks, the head norm / 16, proj_out and the Euler gate-add (gate ones,
    scale 16 dt)."""
    xe, po = head
    lat16 = ref.glue_prescale(lat, 16.0, "f16" if tdt == torch.float16 else "bf16")
    lat16 = lat16.astype(np.float32) if tdt == torch.float16 else ref.bf16_to_f32(lat16)
    h = ref.glue_postscale(qmm_t(lat16, xe, tdt), 16.0)
    X = oracle_step(d, projs, norm_w, gates, h, e, tdt)
    nH = to_t(ref.rmsnorm_rows(X[d.l_txt:], norm_w) / 16.0, tdt)
    pred = qmm_t(nH, po, tdt)
    return ref.glue_gate_add(pred, lat, np.ones(po.n, np.float32), np.float32(16.0) * np.float32(dt))


@pytest.mark.parametrize("d", [TINY, SPLIT], ids=["tiny", "split_k"])
@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_denoise_step_with_head(tdt, d):
    """imq_dit_step_denoise: the embedder (K = 128: the register-staged kernel
    with the post-scale stage), the blocks and the head.  Graph replays with
    three different dt (read when the graph runs) equal eager runs with the
    same dt; the update lat_out - lat_in matches the CPU restatement."""
    channels = 128
    note(f"dit denoise {tdt} {d} C={channels}")
    projs = random_projections(d, tdt, seed=9)
    head = random_head(d, channels, tdt, seed=10)
    step = DitStep(d, projs)
    step.set_head(*head)
    rng = np.random.default_rng(9)
    norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
    gates = (0.5 * rng.standard_normal((4 * d.n_double + d.n_single, d.dim))).astype(np.float32)
    step.set_conditioning(torch.from_numpy(norm_w).cuda(), torch.from_numpy(gates).cuda())
    lat = rng.standard_normal((d.l_img, channels)).astype(np.float32)
    e = rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)
    lat_d, e_d = torch.from_numpy(lat).cuda(), torch.from_numpy(e).cuda()
    eager = {}
    for dt in (-0.25, -0.125, 0.5):
        eager[dt] = step.denoise(lat_d, e_d, dt, use_graph=False).cpu().numpy()
    assert step.launches == d.n_double * 14 + d.n_single * 4 + 4
    assert np.array_equal(lat_d.cpu().numpy(), lat)
    for dt in (0.5, -0.25, -0.125):
        torch.randn(1000, device="cuda").sum().item()
        got = step.denoise(lat_d, e_d, dt, use_graph=True).cpu().numpy()
        assert np.array_equal(got, eager[dt]), f"graph replay with dt={dt} differs from eager"
    dt = -0.25
    want = oracle_denoise(d, projs, head, norm_w, gates, lat, e, dt, tdt)
    upd, upd_want = eager[dt].astype(np.float64) - lat, want.astype(np.float64) - lat
    normwise = np.abs(upd - upd_want).max() / np.abs(upd_want).max()
    note(f"  update normwise={normwise:.3g}")
    assert np.all(np.isfinite(eager[dt]))
    assert normwise <= 1e-2, normwise
    step.close()


def test_denoise_needs_a_head_and_checks_its_shapes():
    d = TINY
    projs = random_projections(d, torch.float16, seed=11)
    step = DitStep(d, projs)
    lat = torch.zeros((d.l_img, 128), device="cuda")
    e = torch.zeros((d.l_txt, d.dim), device="cuda")
    with pytest.raises(ValueError, match="no head"):
        step.denoise(lat, e, 0.1)
    xe, po = random_head(d, 128, torch.float16, seed=12)
    with pytest.raises(ValueError, match="x_embedder"):
        step.set_head(po, xe)  # swapped
    xe32, _ = random_head(d, 128, torch.bfloat16, seed=12)
    with pytest.raises(ValueError, match="dtypes"):
        step.set_head(xe32, po)
    step.close()


def test_create_rejects_wrong_shapes():
    d = TINY
    projs = random_projections(d, torch.float16, seed=8)
    projs[3], projs[8] = projs[8], projs[3]  # add_q where ff.linear_in belongs
    with pytest.raises(ValueError, match="projection 3"):
        DitStep(d, projs)
    with pytest.raises(ValueError, match="needs"):
        DitStep(d, projs[:-1])

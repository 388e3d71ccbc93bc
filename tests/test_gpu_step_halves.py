"""The DiT block halves (imq_dit_double_attn_in ... imq_dit_head_out) around a
caller's attention core.

* With the plan's stand-ins (nx = None: RMSNorm; the V projection as the
  double blocks' attention output; a zero attention half in the single
  blocks' concat buffer) the halves are imq_dit_step_run / _denoise call for
  call: the same kernels on the same data, so the bar is bit-for-bit
  equality, eager and captured in a graph.
* With a caller's normalized inputs and attention outputs, each half's
  outputs (the double blocks' q, k, v of both row sets, the single blocks' qkv
  and SwiGLU half, and the residual after every gated add) are checked
  against the CPU oracle on the same inputs: MAE <= 1e-3, normwise <= 1e-2
  and cosine >= 0.99999 for the projections (one rounding to T), normwise
  <= 1e-2 for the fp32 residual.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from aestrix_amd.step import DitDims, DitStep, random_head, random_projections
from oracle import ref

from test_gpu_step import qmm_t, sub, to_t

pytestmark = pytest.mark.gpu

TINY = DitDims(l_img=64, l_txt=32, dim=256, ff_inner=256, n_double=2, n_single=2)
SPLIT = DitDims(l_img=128, l_txt=64, dim=512, ff_inner=1024, n_double=1, n_single=1)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def conditioned_step(d: DitDims, tdt, seed: int) -> tuple[DitStep, list]:
    projs = random_projections(d, tdt, seed=seed)
    step = DitStep(d, projs)
    rng = np.random.default_rng(seed)
    norm_w = (1.0 + 0.1 * rng.standard_normal(d.dim)).astype(np.float32)
    gates = (0.5 * rng.standard_normal((4 * d.n_double + d.n_single, d.dim))).astype(np.float32)
    step.set_conditioning(torch.from_numpy(norm_w).cuda(), torch.from_numpy(gates).cuda())
    step.gates_host = gates
    return step, projs


class Buffers:
    """The caller's buffers of the halves (J rows, text rows first)."""

    def __init__(self, d: DitDims, tdt):
        J = d.joint
        self.q = torch.empty((J, d.dim), dtype=tdt, device="cuda")
        self.k = torch.empty_like(self.q)
        self.v = torch.empty_like(self.q)
        self.qkv = torch.empty((J, 3 * d.dim), dtype=tdt, device="cuda")
        self.concat = torch.zeros((J, d.dim + d.ff_inner), dtype=tdt, device="cuda")


def blocks_by_halves(step: DitStep, d: DitDims, x: torch.Tensor, buf: Buffers) -> None:
    """The blocks with the plan's stand-ins: attention = V (double), zeros (single)."""
    for b in range(d.n_double):
        step.double_attn_in(b, x, buf.q, buf.k, buf.v)
        step.double_attn_out(b, buf.v, x)
        step.double_mlp(b, x)
    for b in range(d.n_single):
        step.single_attn_in(b, x, buf.qkv, buf.concat)
        step.single_attn_out(b, buf.concat, x)


@pytest.mark.parametrize("d", [TINY, SPLIT], ids=["tiny", "split_k"])
@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_halves_with_standins_reproduce_step_run(tdt, d):
    note(f"dit halves vs run {tdt} {d}")
    step, _ = conditioned_step(d, tdt, seed=21)
    rng = np.random.default_rng(21)
    h = torch.from_numpy(rng.standard_normal((d.l_img, d.dim)).astype(np.float32)).cuda()
    e = torch.from_numpy(rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)).cuda()
    want = step.run(h, e, use_graph=False)
    buf = Buffers(d, tdt)
    x0 = torch.cat([e, h]).contiguous()
    x = x0.clone()
    blocks_by_halves(step, d, x, buf)
    assert torch.equal(x, want), "halves differ from imq_dit_step_run"
    # The same calls captured into a graph, replayed with other work between.
    xg = x0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        blocks_by_halves(step, d, xg, buf)
    for rep in range(3):
        torch.randn(1000, device="cuda").sum().item()
        xg.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xg, want), f"graph replay {rep} of the halves differs"
    del g
    step.close()


def _random_dims(seed: int) -> list[DitDims]:
    rng = np.random.default_rng(seed)
    return [DitDims(l_img=16 * int(rng.integers(1, 40)), l_txt=16 * int(rng.integers(1, 20)),
                    dim=256 * int(rng.integers(1, 6)), ff_inner=256 * int(rng.integers(1, 9)),
                    n_double=int(rng.integers(1, 3)), n_single=int(rng.integers(1, 3)))
            for _ in range(6)]


@pytest.mark.parametrize("d", _random_dims(41), ids=lambda d: f"img{d.l_img}_txt{d.l_txt}_"
                         f"dim{d.dim}_ff{d.ff_inner}_{d.n_double}x{d.n_single}")
@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_step_at_seeded_random_dims(tdt, d):
    """Seeded random plans (row counts in steps of 16, dim and ff_inner in steps of 256, one or
    two blocks of each kind), so the tile plans, K splits and partial tiles of both chains vary:
    the captured graph gives imq_dit_step_run's eager bits, the halves with the stand-ins give
    them too, and the residual stays finite."""
    note(f"dit step at random dims {tdt} {d}")
    step, _ = conditioned_step(d, tdt, seed=d.l_img + d.dim)
    rng = np.random.default_rng(d.l_txt + d.ff_inner)
    h = torch.from_numpy(rng.standard_normal((d.l_img, d.dim)).astype(np.float32)).cuda()
    e = torch.from_numpy(rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)).cuda()
    want = step.run(h, e, use_graph=False)
    assert torch.isfinite(want).all()
    assert torch.equal(step.run(h, e, use_graph=True), want), "graph differs from eager"
    x = torch.cat([e, h]).contiguous()
    blocks_by_halves(step, d, x, Buffers(d, tdt))
    assert torch.equal(x, want), "halves differ from imq_dit_step_run"
    step.close()


@pytest.mark.parametrize("d", [TINY, SPLIT], ids=["tiny", "split_k"])
@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_denoise_by_halves_reproduces_denoise(tdt, d):
    channels = 128
    note(f"dit denoise halves {tdt} {d}")
    step, _ = conditioned_step(d, tdt, seed=23)
    step.set_head(*random_head(d, channels, tdt, seed=24))
    rng = np.random.default_rng(23)
    lat = torch.from_numpy(rng.standard_normal((d.l_img, channels)).astype(np.float32)).cuda()
    e = torch.from_numpy(rng.standard_normal((d.l_txt, d.dim)).astype(np.float32)).cuda()
    for dt in (-0.25, 0.5):
        want = step.denoise(lat, e, dt, use_graph=False)
        x = torch.empty((d.joint, d.dim), device="cuda")
        x[:d.l_txt] = e
        step.head_embed(lat, x)
        blocks_by_halves(step, d, x, Buffers(d, tdt))
        got = torch.empty_like(lat)
        step.head_out(x, lat, dt, got)
        assert torch.equal(got, want), f"dt={dt}: halves differ from imq_dit_step_denoise"
    step.close()


def check_proj(tag: str, got: torch.Tensor, want: np.ndarray) -> None:
    s = ref.error_stats_values(got.float().cpu().numpy(), np.asarray(want, np.float32))
    note(f"  {tag}: mae={s['mae']:.3g} normwise={s['max_rel_normwise']:.3g} "
         f"cos={s['cosine']:.8f}")
    assert s["mae"] <= 1e-3 and s["max_rel_normwise"] <= 1e-2 and s["cosine"] >= 0.99999, (tag, s)


def check_resid(tag: str, got: torch.Tensor, want: np.ndarray) -> None:
    g = got.cpu().numpy().astype(np.float64)
    normwise = np.abs(g - want).max() / np.abs(want).max()
    note(f"  {tag}: normwise={normwise:.3g}")
    assert np.all(np.isfinite(g)) and normwise <= 1e-2, (tag, normwise)


def modulated(x: torch.Tensor, rng, tdt) -> torch.Tensor:
    """A caller's lnMod stand-in: LayerNorm over each row, then a per-column
    scale and shift, rounded to T (the halves only see the T result)."""
    dim = x.shape[1]
    scale = torch.from_numpy((0.2 * rng.standard_normal(dim)).astype(np.float32)).cuda()
    shift = torch.from_numpy((0.1 * rng.standard_normal(dim)).astype(np.float32)).cuda()
    ln = torch.nn.functional.layer_norm(x, (dim,), eps=1e-6)
    return (ln * (1 + scale) + shift).to(tdt).contiguous()


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16])
def test_halves_with_a_callers_core_match_the_oracle(tdt):
    """Every projection of the double and single blocks (to_q / to_k / to_v,
    add_q / add_k / add_v, to_out / to_add_out, both MLPs, to_qkv_mlp_proj's
    Q/K/V and SwiGLU rows, single to_out) against the oracle, fed the caller's
    normalized inputs and an attention output that is not V."""
    d = SPLIT
    note(f"dit halves with a caller's core {tdt} {d}")
    step, projs = conditioned_step(d, tdt, seed=27)
    gates = step.gates_host
    rng = np.random.default_rng(27)
    T, I = slice(0, d.l_txt), slice(d.l_txt, d.joint)
    dim, ffi = d.dim, d.ff_inner
    x = torch.from_numpy(rng.standard_normal((d.joint, dim)).astype(np.float32)).cuda()
    buf = Buffers(d, tdt)

    def host(t):
        return t.float().cpu().numpy()

    for b in range(d.n_double):
        W = projs[12 * b:12 * b + 12]
        nx = modulated(x, rng, tdt)
        step.double_attn_in(b, None, buf.q, buf.k, buf.v, nx=nx)
        n_h = host(nx)
        for i, (out, name) in enumerate(((buf.q, "q"), (buf.k, "k"), (buf.v, "v"))):
            check_proj(f"double {b} {name} image rows", out[I], qmm_t(n_h[I], W[i], tdt))
            check_proj(f"double {b} {name} text rows", out[T], qmm_t(n_h[T], W[3 + i], tdt))
        # A caller's attention output: anything of q, k, v; here a T mix of all three.
        attn = (0.5 * buf.q.float() - 0.25 * buf.k.float() + buf.v.float()).to(tdt).contiguous()
        a_h = host(attn)
        x_h = host(x)
        want = x_h.astype(np.float64).copy()
        want[I] = ref.glue_gate_add(qmm_t(a_h[I], W[6], tdt), x_h[I], gates[4 * b], 1.0)
        want[T] = ref.glue_gate_add(qmm_t(a_h[T], W[7], tdt), x_h[T], gates[4 * b + 1], 1.0)
        step.double_attn_out(b, attn, x)
        check_resid(f"double {b} attn out", x, want)
        nx2 = modulated(x, rng, tdt)
        n2 = host(nx2)
        x_h = host(x)
        want = x_h.astype(np.float64).copy()
        for rows, wi, wo, gi in ((I, 8, 9, 2), (T, 10, 11, 3)):
            g = qmm_t(n2[rows], sub(W[wi], slice(0, ffi)), tdt)
            u = qmm_t(n2[rows], sub(W[wi], slice(ffi, 2 * ffi)), tdt)
            sw = to_t(ref.glue_swiglu(g, u, 1.0, 1.0), tdt)
            want[rows] = ref.glue_gate_add(qmm_t(sw, W[wo], tdt), x_h[rows], gates[4 * b + gi], 1.0)
        step.double_mlp(b, x, nx=nx2)
        check_resid(f"double {b} mlp", x, want)
    for b in range(d.n_single):
        W = projs[12 * d.n_double + 2 * b:12 * d.n_double + 2 * b + 2]
        nx = modulated(x, rng, tdt)
        step.single_attn_in(b, None, buf.qkv, buf.concat, nx=nx)
        n_h = host(nx)
        check_proj(f"single {b} qkv", buf.qkv, qmm_t(n_h, sub(W[0], slice(0, 3 * dim)), tdt))
        g = qmm_t(n_h, sub(W[0], slice(3 * dim, 3 * dim + ffi)), tdt)
        u = qmm_t(n_h, sub(W[0], slice(3 * dim + ffi, 3 * dim + 2 * ffi)), tdt)
        check_proj(f"single {b} swiglu half", buf.concat[:, dim:],
                   ref.glue_swiglu(g, u, 1.0, 1.0))
        # The caller's attention writes the first dim columns of concat.
        buf.concat[:, :dim] = (buf.qkv[:, :dim].float() * 0.5 + buf.qkv[:, 2 * dim:].float()).to(tdt)
        c_h = host(buf.concat)
        x_h = host(x)
        want = ref.glue_gate_add(qmm_t(c_h, W[1], tdt), x_h, gates[4 * d.n_double + b], 1.0)
        step.single_attn_out(b, buf.concat, x)
        check_resid(f"single {b} attn out", x, want)
    step.close()


def test_halves_check_their_arguments():
    d = TINY
    step, _ = conditioned_step(d, torch.float16, seed=29)
    buf = Buffers(d, torch.float16)
    x = torch.zeros((d.joint, d.dim), device="cuda")
    with pytest.raises(ValueError, match="out of range"):
        step.double_attn_in(d.n_double, x, buf.q, buf.k, buf.v)
    with pytest.raises(ValueError, match="out of range"):
        step.single_attn_out(-1, buf.concat, x)
    with pytest.raises(ValueError, match="neither x nor nx"):
        step.double_attn_in(0, None, buf.q, buf.k, buf.v)
    with pytest.raises(ValueError, match="no head"):
        step.head_embed(torch.zeros((d.l_img, 128), device="cuda"), x)
    step.close()

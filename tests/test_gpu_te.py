"""Text-encoder layer halves (include/imq_te.h) and the fused qmm + dq_add
(imq_qmm_add) against the oracle.

Known answers: the oracle's qmm (RNE_T of the float64 product with the
bit-exact dequant), RMSNorm in float64 rounded to T, and the reference's glue
(oracle/ref.py glue_add_t = dq_add, glue_swiglu at scales 1 = dq_silu_mul).
imq_qmm_add must equal imq_qgemm + dq_add on the device's own product bit for
bit (same accumulator, same rounding).  The halves compound roundings
(RMSNorm, three products, SiLU), yet each output still meets the single
qmm's bars: normwise error <= 1e-2, MAE <= 1e-3 and cosine >= 0.99999 (the
layer output measured at MAE <= 7e-5, cosine >= 0.9999999), on 32 sampled
rows (every op is row-local) at the Qwen3 4B shapes (hidden 2560, q 4096,
k / v 1024, inter 9728)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import synth
from aestrix_amd.ops import Q
from aestrix_amd.te import TextEncoderLayers, random_te_layers
from oracle import ref

pytestmark = pytest.mark.gpu

NORMWISE_TOL = 1e-2
MAE_TOL = 1e-3
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def vals(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def to_t(v: np.ndarray, tdt) -> np.ndarray:
    v = np.asarray(v, np.float32)
    if tdt == torch.float16:
        return v.astype(np.float16).astype(np.float32)
    return ref.bf16_to_f32(ref.f32_to_bf16(v))


def tname(tdt) -> str:
    return "f16" if tdt == torch.float16 else "bf16"


def t_vals(bits_or_f16: np.ndarray, tdt) -> np.ndarray:
    if tdt == torch.float16:
        return np.asarray(bits_or_f16).astype(np.float32)
    return ref.bf16_to_f32(bits_or_f16)


def qmm_t(x_t: np.ndarray, q: Q, tdt, rows=None) -> np.ndarray:
    w = q.w.cpu().numpy().view(np.uint32)
    s, b = q.s.cpu(), q.b.cpu()
    if rows is not None:
        w, s, b = w[rows], s[rows], b[rows]
    if tdt == torch.float16:
        return ref.qmm_t_as(x_t.astype(np.float16), w, s.numpy(), b.numpy(),
                            np.float16).astype(np.float32)
    sb = s.view(torch.int16).numpy().view(np.uint16)
    bb = b.view(torch.int16).numpy().view(np.uint16)
    return ref.bf16_to_f32(ref.qmm_t(ref.f32_to_bf16(x_t), w, sb, bb))


def check(got: np.ndarray, want: np.ndarray, what: str, tol: float = NORMWISE_TOL) -> None:
    d = np.abs(got.astype(np.float64) - want)
    normwise = d.max() / np.abs(want).max()
    st = ref.error_stats_values(got.astype(np.float64), np.asarray(want, np.float64))
    note(f"  {what}: normwise={normwise:.3g} mean_rel={d.mean() / np.abs(want).mean():.3g} "
         f"mae={st['mae']:.3g} cosine={st['cosine']:.8f} equal={np.mean(got == want):.4f}")
    assert np.all(np.isfinite(got))
    assert normwise <= tol, (what, normwise)
    assert st["mae"] <= MAE_TOL and st["cosine"] >= COSINE_MIN, (what, st)


# --------------------------------------------------------------------- RMSNorm


@pytest.mark.parametrize("x_dtype,y_dtype,cols,eps", [
    (torch.float32, torch.float16, 3072, 1e-5), (torch.float32, torch.bfloat16, 3072, 1e-5),
    (torch.bfloat16, torch.bfloat16, 2560, 1e-6), (torch.float16, torch.float16, 2560, 1e-6),
    (torch.float32, torch.bfloat16, 1000, 1e-5), (torch.bfloat16, torch.bfloat16, 1004, 1e-6)])
def test_rmsnorm(x_dtype, y_dtype, cols, eps):
    """imq_rmsnorm against the float64 RMSNorm rounded once to T (cols 1004: the
    T-input kernel's scalar form, the others its 16-byte form): the fp32 sum of
    squares and rsqrt move a value across a rounding boundary rarely, by one
    unit in the last place of T (at most 0.5% of the values here, none by more)."""
    note(f"rmsnorm {x_dtype} -> {y_dtype} cols={cols}")
    g = torch.Generator(device="cuda").manual_seed(cols)
    x = (torch.randn((300, cols), device="cuda", generator=g) * 3).to(x_dtype)
    w = 1.0 + 0.1 * torch.randn(cols, device="cuda", generator=g)
    y = imq.rmsnorm(x, w, eps, out_dtype=y_dtype)
    want = to_t(ref.rmsnorm_rows(vals(x).astype(np.float64), vals(w), eps), y_dtype)
    got = vals(y)
    if y_dtype == torch.float16:
        gi = got.astype(np.float16).view(np.int16).astype(np.int64)
        wi = want.astype(np.float16).view(np.int16).astype(np.int64)
    else:
        gi = ref.f32_to_bf16(got).astype(np.int64)
        wi = ref.f32_to_bf16(want).astype(np.int64)
    ulps = np.abs(gi - wi)
    note(f"  equal={np.mean(ulps == 0):.5f} max_ulps={ulps.max()}")
    assert ulps.max() <= 1 and np.mean(ulps == 0) >= 0.995
    with pytest.raises(imq.ImqUnsupported):  # a 16-bit x of another type than y
        imq.rmsnorm(x.half(), w, eps, out_dtype=torch.bfloat16)


# ------------------------------------------------------------- qmm + dq_add


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(512, 2560, 4096), (30, 2560, 9728), (300, 512, 768),
                                   (7, 256, 192)])
def test_qmm_add(dtype, m, n, k):
    """K = 192: the register-staged kernel's output stage."""
    note(f"qmm_add {dtype} M={m} N={n} K={k}")
    p = synth.make_problem(m, n, k, seed=70)
    x, w, s, b = synth.to_device(p)
    x, s, b = x.to(dtype), s.to(dtype), b.to(dtype)
    resid = (torch.randn((m, n), device="cuda") * 2).to(dtype)
    y = imq.qmm_add(x, w, s, b, resid)
    prod = imq.qgemm(x, w, s, b)
    want_bits = ref.glue_add_t(vals(prod), vals(resid), tname(dtype))
    got = y.cpu()
    got_bits = got.view(torch.int16).numpy().view(np.uint16)
    want_u16 = want_bits.view(np.uint16) if dtype == torch.float16 else want_bits
    assert np.array_equal(got_bits, want_u16), "qmm_add != qgemm + dq_add on the device product"
    q = Q(w=w, s=s, b=b, n=n, k=k)
    want = t_vals(ref.glue_add_t(qmm_t(vals(x), q, dtype), vals(resid), tname(dtype)), dtype)
    check(vals(y), want, "qmm_add vs oracle")
    inplace = resid.clone()
    imq.qmm_add(x, w, s, b, inplace, out=inplace)
    assert torch.equal(inplace, y)


# --------------------------------------------------------------- layer halves


def oracle_attn_in(x: np.ndarray, l, tdt) -> np.ndarray:
    h1 = to_t(ref.rmsnorm_rows(x, vals(l.norm_in), 1e-6), tdt)
    return qmm_t(h1, l.qkv, tdt)


def oracle_attn_out_mlp(x: np.ndarray, attn_o: np.ndarray, l, tdt) -> np.ndarray:
    t = tname(tdt)
    r = t_vals(ref.glue_add_t(qmm_t(attn_o, l.o, tdt), x, t), tdt)
    h2 = to_t(ref.rmsnorm_rows(r, vals(l.norm_post), 1e-6), tdt)
    inter = l.down.k
    g = qmm_t(h2, l.gate_up, tdt, rows=slice(0, inter))
    u = qmm_t(h2, l.gate_up, tdt, rows=slice(inter, 2 * inter))
    m = to_t(ref.glue_swiglu(g, u, 1.0, 1.0), tdt)
    return t_vals(ref.glue_add_t(qmm_t(m, l.down, tdt), r, t), tdt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [512, 30, 17, 16, 8, 4, 3, 2, 1])
def test_layer_halves_match_oracle(dtype, rows):
    note(f"TE layer halves {dtype} rows={rows} (hidden 2560, qkv 6144, inter 9728)")
    layers = random_te_layers(1, dtype=dtype, seed=71)
    te = TextEncoderLayers(layers, max_rows=512)
    l = layers[0]
    g = torch.Generator(device="cuda").manual_seed(71)
    x = torch.randn((rows, 2560), device="cuda", generator=g).to(dtype)
    attn_o = torch.randn((rows, 4096), device="cuda", generator=g).to(dtype)
    qkv = te.attn_in(0, x)
    y = te.attn_out_mlp(0, x, attn_o)
    torch.cuda.synchronize()
    sample = np.sort(np.random.default_rng(rows).choice(rows, min(rows, 32), replace=False))
    xs, ao = vals(x)[sample], vals(attn_o)[sample]
    check(vals(qkv)[sample], oracle_attn_in(xs, l, dtype), "qkv")
    check(vals(y)[sample], oracle_attn_out_mlp(xs, ao, l, dtype), "layer output")
    # in place (out = x) gives the same result
    x2 = x.clone()
    te.attn_out_mlp(0, x2, attn_o, out=x2)
    assert torch.equal(x2, y)
    te.close()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 2])
def test_layer_halves_at_one_and_two_rows_equal_the_unfused_ops(dtype, rows):
    """At 1-2 rows the q/k/v and gate/up qGEMVs normalize their input in the
    x staging instead of after a separate RMSNorm launch: the halves equal, bit
    for bit, the same products on the RMSNorm kernel's output (imq.rmsnorm,
    imq.qgemv, imq.qmm_swiglu on the qGEMV; the residual adds T(float(a) +
    float(b)) in torch's fp32 and round-to-nearest-even)."""
    note(f"TE halves at {rows} rows {dtype}: fused norm == rmsnorm + products")
    layers = random_te_layers(1, dtype=dtype, seed=74)
    te = TextEncoderLayers(layers, max_rows=16)
    l = layers[0]
    g = torch.Generator(device="cuda").manual_seed(74 + rows)
    x = torch.randn((rows, 2560), device="cuda", generator=g).to(dtype)
    attn_o = torch.randn((rows, 4096), device="cuda", generator=g).to(dtype)
    qkv = te.attn_in(0, x)
    y = te.attn_out_mlp(0, x, attn_o)
    h1 = imq.rmsnorm(x, l.norm_in, 1e-6)
    assert torch.equal(qkv, imq.qgemv(h1, l.qkv.w, l.qkv.s, l.qkv.b)), "attn_in"
    r = (x.float() + imq.qgemv(attn_o, l.o.w, l.o.s, l.o.b).float()).to(dtype)
    h2 = imq.rmsnorm(r, l.norm_post, 1e-6)
    inter = l.down.k
    m = imq.qmm_swiglu(h2, l.gate_up.w, l.gate_up.s, l.gate_up.b, inter, 0, inter)
    want = (r.float() + imq.qgemv(m, l.down.w, l.down.s, l.down.b).float()).to(dtype)
    assert torch.equal(y, want), "attn_out_mlp"
    te.close()


def test_layer_halves_under_graph_capture():
    """Both halves allocate nothing per call: a captured pair of calls over two
    layers replays bit-equal to eager, with other device work in between."""
    layers = random_te_layers(2, dtype=torch.bfloat16, seed=72)
    te = TextEncoderLayers(layers, max_rows=64)
    g = torch.Generator(device="cuda").manual_seed(72)
    x = torch.randn((48, 2560), device="cuda", generator=g).bfloat16()
    attn = torch.randn((48, 4096), device="cuda", generator=g).bfloat16()
    qkv = torch.empty((48, 6144), dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(x)
    y = torch.empty_like(x)

    def layer_pair():
        te.attn_in(0, x, qkv)
        te.attn_out_mlp(0, x, attn, h)
        te.attn_in(1, h, qkv)
        te.attn_out_mlp(1, h, attn, y)

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        layer_pair()
        s.synchronize()
        want_qkv, want_y = qkv.clone(), y.clone()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            layer_pair()
    for rep in range(3):
        qkv.zero_()
        y.zero_()
        torch.randn(1000, device="cuda").sum().item()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(qkv, want_qkv) and torch.equal(y, want_y), rep
    te.close()


def test_loaded_layers_with_reference_keys(tmp_path):
    """load_te_layers reads DirectTEForward's names (layers.<i>.self_attn.q_proj,
    ..., input_layernorm.weight; DirectTEForward.swift:97-138) and concatenates
    q/k/v and gate/up; the plan over loaded layers equals the one over the same
    tensors built directly, bit for bit."""
    from safetensors.torch import save_file

    from aestrix_amd.te import load_te_layers
    from aestrix_amd.weights import SafetensorsSet
    dims = dict(hidden=256, nq=256, nkv=64, inter=512)
    layers = random_te_layers(2, dtype=torch.bfloat16, seed=73, **dims)
    tensors = {}

    def put(prefix, w, s, b):
        tensors[f"{prefix}.weight"] = w.cpu().contiguous().view(torch.uint32)
        tensors[f"{prefix}.scales"] = s.cpu().contiguous()
        tensors[f"{prefix}.biases"] = b.cpu().contiguous()

    for i, l in enumerate(layers):
        p = f"layers.{i}"
        cuts = {"q": (0, 256), "k": (256, 320), "v": (320, 384)}
        for nm, (a, z) in cuts.items():
            put(f"{p}.self_attn.{nm}_proj", l.qkv.w[a:z], l.qkv.s[a:z], l.qkv.b[a:z])
        put(f"{p}.self_attn.o_proj", l.o.w, l.o.s, l.o.b)
        put(f"{p}.mlp.gate_proj", l.gate_up.w[:512], l.gate_up.s[:512], l.gate_up.b[:512])
        put(f"{p}.mlp.up_proj", l.gate_up.w[512:], l.gate_up.s[512:], l.gate_up.b[512:])
        put(f"{p}.mlp.down_proj", l.down.w, l.down.s, l.down.b)
        # the file holds bf16 norm weights; the direct plan gets the same values
        l.norm_in = l.norm_in.bfloat16().float()
        l.norm_post = l.norm_post.bfloat16().float()
        tensors[f"{p}.input_layernorm.weight"] = l.norm_in.bfloat16().cpu()
        tensors[f"{p}.post_attention_layernorm.weight"] = l.norm_post.bfloat16().cpu()
    save_file(tensors, str(tmp_path / "0.safetensors"))
    with SafetensorsSet.open_dir(str(tmp_path)) as st:
        loaded = load_te_layers(st, 2)
    a, b = TextEncoderLayers(loaded, max_rows=40), TextEncoderLayers(layers, max_rows=40)
    g = torch.Generator(device="cuda").manual_seed(73)
    x = torch.randn((40, 256), device="cuda", generator=g).bfloat16()
    attn = torch.randn((40, 256), device="cuda", generator=g).bfloat16()
    for i in range(2):
        assert torch.equal(a.attn_in(i, x), b.attn_in(i, x))
        assert torch.equal(a.attn_out_mlp(i, x, attn), b.attn_out_mlp(i, x, attn))
    a.close()
    b.close()


def test_argument_checks():
    layers = random_te_layers(1, hidden=256, nq=256, nkv=64, inter=512, seed=74)
    te = TextEncoderLayers(layers, max_rows=16)
    x = torch.zeros((16, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(imq.ImqInvalid, match="layer"):
        te.attn_in(1, x)
    with pytest.raises(imq.ImqInvalid, match="rows"):
        te.attn_in(0, torch.zeros((17, 256), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        te.attn_in(0, x.half())
    te.close()
    bad = random_te_layers(1, hidden=256, nq=256, nkv=64, inter=512, seed=75)
    bad[0].o, bad[0].down = bad[0].down, bad[0].o  # swapped
    with pytest.raises(imq.ImqInvalid, match="do not form a layer"):
        TextEncoderLayers(bad, max_rows=16)

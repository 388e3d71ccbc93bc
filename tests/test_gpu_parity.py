"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (stated here, applied below):
* dequantize: bit-exact against RNE_bf16(fl32(fl32(s*q) + b)).
* qGEMV / qGEMM: against oracle = RNE_bf16(x . deq(W)^T accumulated in double)
  with the bit-exact bf16 dequant: mean |y - oracle| <= MAE_TOL,
  max |y - oracle| / max |oracle| <= NORMWISE_TOL, and the reference's own
  qmm criterion, cosine(y, oracle) >= COSINE_MIN (DirectQmmSpike.swift:141-153).
* one-hot activations make y a column of deq(W): that must be bit-exact in
  both matmul kernels (it pins their fused in-register dequantization).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import _lib, ops, synth
from oracle import cref, ref

pytestmark = pytest.mark.gpu

MAE_TOL = 1e-3
NORMWISE_TOL = 1e-2
COSINE_MIN = 0.99999  # the reference's qmm parity bar (DirectQmmSpike.swift:141-153)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def to_dev_words(w: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).cuda()


def to_dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return synth.bf16_bits(t)


def assert_close(y_bits: np.ndarray, oracle_bits: np.ndarray, what: str) -> dict:
    st = ref.error_stats(y_bits, oracle_bits)
    note(f"  {what}: mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g} "
         f"bit_exact={st['bit_exact_frac']:.4f} cosine={st['cosine']:.7f}")
    assert st["mae"] <= MAE_TOL, (what, st)
    assert st["max_rel_normwise"] <= NORMWISE_TOL, (what, st)
    assert st["cosine"] >= COSINE_MIN, (what, st)
    return st


# ------------------------------------------------------------------ dequant


def test_dequant_golden_bit_exact():
    d = np.load(GOLDEN)
    for tag in ("deq", "kat"):
        note(f"dequant golden {tag}")
        out = imq.dequantize(to_dev_words(d[f"{tag}_w"]), to_dev_bf16(d[f"{tag}_s"]),
                             to_dev_bf16(d[f"{tag}_b"]))
        assert np.array_equal(bits(out), d[f"{tag}_out"])


def test_dequant_exact_rational_grid():
    import test_oracle as t

    note("dequant exact-rational (scale, bias) grid")
    _, _, w, s, b = t._grid_problem()
    out = imq.dequantize(to_dev_words(w), to_dev_bf16(s), to_dev_bf16(b))
    assert np.array_equal(bits(out), t.exact_grid())


@pytest.mark.parametrize("n,k", [(27648, 3072), (3072, 12288), (1, 64), (7, 4160)])
def test_dequant_block_shapes_bit_exact(n, k):
    note(f"dequant N={n} K={k} seed=11")
    p = synth.make_problem(0, n, k, seed=11)
    out = imq.dequantize(to_dev_words(p.w), to_dev_bf16(p.scales), to_dev_bf16(p.biases))
    got = bits(out)
    want = cref.dequantize(p.w, p.scales, p.biases)
    assert np.array_equal(got, want)


def test_dequant_f16_bit_exact():
    note("dequant f16 N=96 K=512")
    p = synth.make_problem(0, 96, 512, seed=12)
    s16 = ref.bf16_to_f32(p.scales).astype(np.float16)
    b16 = ref.bf16_to_f32(p.biases).astype(np.float16)
    q = ref.unpack_codes(p.w).astype(np.float32)
    sf = np.repeat(s16.astype(np.float32), 64, axis=1)
    bf = np.repeat(b16.astype(np.float32), 64, axis=1)
    want = (sf * q + bf).astype(np.float16)
    out = imq.dequantize(to_dev_words(p.w), torch.from_numpy(s16).cuda(),
                         torch.from_numpy(b16).cuda())
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16))


# ------------------------------------------------------------ quantized matmul


def test_qmm_golden_within_tolerance():
    d = np.load(GOLDEN)
    for i, (m, n, k, seed) in enumerate(d["qmm_cases"]):
        note(f"qmm golden case {i}: M={m} N={n} K={k} seed={seed}")
        x, w, s, b = (to_dev_bf16(d[f"qmm{i}_x"]), to_dev_words(d[f"qmm{i}_w"]),
                      to_dev_bf16(d[f"qmm{i}_s"]), to_dev_bf16(d[f"qmm{i}_b"]))
        for name, fn in (("qmm_t", imq.quantized_matmul), ("qgemm", imq.qgemm)):
            assert_close(bits(fn(x, w, s, b)), d[f"qmm{i}_y"], f"{name} case {i}")
        if m <= 16:
            assert_close(bits(imq.qgemv(x, w, s, b)), d[f"qmm{i}_y"], f"qgemv case {i}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("n,k", [(9728, 2560), (2560, 9728), (100, 64), (33, 4160), (1000, 768)])
def test_qgemv_shapes(m, n, k):
    note(f"qgemv M={m} N={n} K={k} seed=13")
    p = synth.make_problem(m, n, k, seed=13)
    x, w, s, b = synth.to_device(p)
    got = bits(imq.qgemv(x, w, s, b))
    want = cref.qmm_t(p.x, p.w, p.scales, p.biases)
    assert_close(got, want, f"qgemv M={m} N={n} K={k}")


@pytest.mark.parametrize("m,n,k", [(17, 32, 64), (64, 96, 128), (128, 256, 320), (129, 200, 192),
                                   (300, 257, 3072), (1, 512, 256), (255, 1000, 640)])
def test_qgemm_shapes(m, n, k):
    note(f"qgemm M={m} N={n} K={k} seed=14")
    p = synth.make_problem(m, n, k, seed=14)
    x, w, s, b = synth.to_device(p)
    got = bits(imq.qgemm(x, w, s, b))
    want = cref.qmm_t(p.x, p.w, p.scales, p.biases)
    assert_close(got, want, f"qgemm M={m} N={n} K={k}")


def _sampled_rows_check(m, n, k, seed, rows=48):
    note(f"qmm_t M={m} N={n} K={k} seed={seed} (oracle on {rows} sampled rows)")
    p = synth.make_problem(m, n, k, seed=seed)
    x, w, s, b = synth.to_device(p)
    y = imq.quantized_matmul(x, w, s, b)
    idx = np.unique(np.linspace(0, m - 1, rows).astype(np.int64))
    got = bits(y)[idx]
    want = cref.qmm_t(p.x[idx], p.w, p.scales, p.biases)
    return assert_close(got, want, f"qmm_t M={m} N={n} K={k} rows={len(idx)}")


def test_qmm_pr1_shape_sampled_rows():
    _sampled_rows_check(1024, 9216, 3072, seed=0)


def test_qmm_target_shape_sampled_rows():
    _sampled_rows_check(4608, 18432, 3072, seed=0, rows=32)


def test_qmm_single_block_shapes_sampled_rows():
    _sampled_rows_check(4608, 27648, 3072, seed=1, rows=24)
    _sampled_rows_check(4608, 3072, 9216, seed=2, rows=48)


@pytest.mark.parametrize("m,n,k", [(256, 2560, 768), (384, 6144, 1280), (192, 3072, 3328),
                                   (64, 4096, 3840), (512, 2560, 9728)])
def test_tile_kernel_two_step_tail_is_deterministic(m, n, k):
    """Tiles of up to 128 rows issue each K-step's loads two steps ahead; a split range of
    4 i + 2 steps ends in two steps that issue no loads, the last one waiting for all of them
    (the activation stage it reads was loaded by the loop's last step).  These plans end that
    way, unsplit and split (the text encoder's down projection at L = 512 among them): twelve
    calls back to back give the same bits, within the oracle bar on sampled rows."""
    plan = imq.qmm_plan(m, n, k)
    assert plan["kernel"] == "tile" and plan["tile_rows"] <= 128, plan
    steps, sp = k // 128, plan["splits"]
    sps = ((steps + sp - 1) // sp + 1) // 2 * 2
    assert sps % 4 == 2 or (steps - (sp - 1) * sps) % 4 == 2, (plan, steps)
    note(f"two-step tail M={m} N={n} K={k} plan {plan}")
    p = synth.make_problem(m, n, k, seed=31)
    x, w, s, b = synth.to_device(p)
    ys = [imq.quantized_matmul(x, w, s, b) for _ in range(12)]
    first = bits(ys[0])
    for i, y in enumerate(ys[1:], 1):
        assert np.array_equal(bits(y), first), f"call {i} differs"
    idx = np.unique(np.linspace(0, m - 1, 32).astype(np.int64))
    assert_close(first[idx], cref.qmm_t(p.x[idx], p.w, p.scales, p.biases),
                 f"two-step tail M={m} N={n} K={k}")


@pytest.mark.parametrize("fn_name,m,k", [("qgemm", 128, 128), ("qgemm", 40, 3072),
                                         ("qgemv", 16, 3072), ("qgemv", 1, 2560)])
def test_one_hot_rows_reproduce_dequant_bit_exact(fn_name, m, k):
    """x rows are one-hot, so y[i, :] = deq(W)[:, k_i] exactly (products with
    1.0 and 0.0 and their fp32 sums are exact)."""
    n = 320
    note(f"{fn_name} one-hot M={m} N={n} K={k}")
    p = synth.make_problem(0, n, k, seed=15)
    rng = np.random.default_rng(15)
    cols = np.arange(m) if m == k else rng.choice(k, size=m, replace=False)
    xh = np.zeros((m, k), dtype=np.uint16)
    xh[np.arange(m), cols] = 0x3F80
    x, w, s, b = to_dev_bf16(xh), to_dev_words(p.w), to_dev_bf16(p.scales), to_dev_bf16(p.biases)
    y = bits(getattr(imq, fn_name)(x, w, s, b))
    deq_gpu = bits(imq.dequantize(w, s, b))
    assert np.array_equal(y, deq_gpu[:, cols].T)


def test_dispatcher_routes_by_m():
    """M <= 2 is the qGEMV kernel bit for bit; above, the matrix-core kernels
    (3 <= M <= 16 the weight-streaming one, then the tiled one, whose K may be
    split by the dispatcher: other fp32 summation orders).  imq_qmm_plan names
    the same kernels."""
    p = synth.make_problem(17, 384, 512, seed=16)
    x, w, s, b = synth.to_device(p)
    for m in (1, 2):
        note(f"dispatcher M={m}")
        assert imq.qmm_plan(m, 384, 512)["kernel"] == "qgemv"
        assert np.array_equal(bits(imq.quantized_matmul(x[:m], w, s, b)),
                              bits(imq.qgemv(x[:m], w, s, b)))
    for m in (3, 4, 5, 16, 17):
        assert imq.qmm_plan(m, 384, 512)["kernel"] == ("few_row" if m <= 16 else "tile")
        note(f"dispatcher M={m}")
        y = bits(imq.quantized_matmul(x[:m], w, s, b))
        assert_close(y, cref.qmm_t(p.x[:m], p.w, p.scales, p.biases), f"dispatcher M={m}")


@pytest.mark.parametrize("m,n,k", [(17, 384, 512), (40, 1000, 2560), (24, 1001, 1024),
                                   (96, 512, 4096), (300, 512, 768), (512, 2560, 9728)])
def test_split_k_dispatcher(m, n, k):
    """Shapes with too few output tiles for the chip: the dispatcher splits K
    (and takes 32- or 64-row tiles); N = 1001 takes the reduction's
    single-element path.  Oracle within tolerance, the same bits on
    a second call (deterministic order), and one-hot rows are single weights
    even when summed over splits."""
    note(f"split-K dispatcher M={m} N={n} K={k}")
    p = synth.make_problem(m, n, k, seed=21)
    x, w, s, b = synth.to_device(p)
    y1 = bits(imq.quantized_matmul(x, w, s, b))
    y2 = bits(imq.quantized_matmul(x, w, s, b))
    assert np.array_equal(y1, y2)
    if m * n * k <= 512 * 2560 * 9728 // 8:
        assert_close(y1, cref.qmm_t(p.x, p.w, p.scales, p.biases), "split-K")
    rng = np.random.default_rng(22)
    cols = rng.choice(k, size=m, replace=m > k)
    xh = np.zeros((m, k), dtype=np.uint16)
    xh[np.arange(m), cols] = 0x3F80
    yo = bits(imq.quantized_matmul(to_dev_bf16(xh), w, s, b))
    assert np.array_equal(yo, bits(imq.dequantize(w, s, b))[:, cols].T)


@pytest.mark.parametrize("m,n,k,splits", [(16, 2560, 9728, 10), (12, 2560, 9728, 10),
                                          (12, 1000, 4608, 9), (8, 2560, 9728, 10),
                                          (16, 1024, 9728, 10), (13, 1030, 4608, 9),
                                          (6, 2560, 9728, 10), (16, 2560, 4096, 4),
                                          (16, 19456, 2560, 5), (16, 4096, 9728, 10),
                                          (5, 2560, 9728, 1), (4, 2560, 9728, 1),
                                          (16, 9728, 2560, 5), (16, 6144, 2560, 1),
                                          (12, 12288, 2560, 5), (13, 2560, 4096, 1),
                                          (12, 2560, 2560, 1), (12, 1024, 2560, 1),
                                          (3, 2560, 9728, 1)])
def test_few_row_split_plan(m, n, k, splits):
    """imq_qmm_plan reports the few-row K split and its workspace: taken from
    M = 6 where x does not fit LDS ([2560 x 9728], [1000 x 4608], [2560 x
    4096] at M = 16), where the multi-tile kernel would need two rounds of the
    CUs ([19456 x 2560] M = 16) or streams 10 MiB of weights or more
    ([9728 x 2560] M = 16, [12288 x 2560] M = 12); not at M <= 5, nor where the
    multi-tile kernel fits one round below that ([6144 x 2560], [2560 x 4096]
    at M = 13, [2560 x 2560] and [1024 x 2560] at M = 12).  Splits: two 512-k
    pieces each from K = 8192, and from K = 4096 where that leaves 160
    workgroups of 64 rows ([2560 x 4096]; not [1000 x 4608]), else one."""
    plan = imq.qmm_plan(m, n, k, torch.bfloat16)
    assert plan["kernel"] == "few_row", plan
    assert plan["splits"] == splits, plan
    assert plan["workspace_bytes"] == (splits * m * n * 4 if splits > 1 else 0), plan


@pytest.mark.parametrize("m,n,k,splits", [(17, 2560, 9728, 10), (30, 2560, 9728, 10),
                                          (32, 2560, 9728, 10), (30, 2560, 4096, 4),
                                          (24, 1024, 2560, 5), (24, 1030, 4608, 9),
                                          (30, 9728, 2560, 5), (30, 2560, 1024, 2),
                                          (33, 2560, 9728, 0), (20, 2560, 2560, 5),
                                          (30, 3072, 3072, 6), (24, 2560, 3840, 0),
                                          (20, 17, 1024, 2), (30, 6144, 2560, 5),
                                          (17, 6144, 2560, 5), (30, 4096, 2560, 5),
                                          (20, 9728, 2560, 5), (30, 19456, 2560, 5)])
def test_few_row_split_past_16_rows_plan(m, n, k, splits):
    """17 to 32 rows take the few-row K split (two token groups per weight
    fragment) wherever K % 512 == 0 with at least two 512-k pieces, at any
    count of row tiles; pieces per split as for 16 rows and fewer.
    The others here (splits 0) run the tile kernel: 33 rows, K = 3840."""
    plan = imq.qmm_plan(m, n, k, torch.bfloat16)
    if splits:
        assert plan["kernel"] == "few_row" and plan["splits"] == splits, plan
        assert plan["workspace_bytes"] == splits * m * n * 4, plan
    else:
        assert plan["kernel"] == "tile", plan


@pytest.mark.gpu
def test_few_row_split_repeated_and_replayed():
    """The few-row K split (partial sums in the stream's workspace, added by a
    second kernel) on four shapes with different tile groups and splits,
    alternating on one stream many times, then inside a captured graph
    replayed several times with the zeroed outputs and eager calls in between:
    every result equals the first call's bits."""
    shapes = [(16, 2560, 9728), (12, 1000, 4608), (8, 2560, 9728), (13, 1030, 4608),
              (30, 2560, 9728), (25, 1030, 4608)]
    probs = []
    for i, (m, n, k) in enumerate(shapes):
        assert imq.qmm_plan(m, n, k, torch.bfloat16)["splits"] > 1
        p = synth.make_problem(m, n, k, seed=40 + i)
        x, w, s_, b = synth.to_device(p)
        probs.append((x, w, s_, b, imq.quantized_matmul(x, w, s_, b)))
    torch.cuda.synchronize()
    want = [bits(y) for *_, y in probs]
    for rep in range(6):
        for i, (x, w, s_, b, _) in enumerate(probs):
            y = imq.quantized_matmul(x, w, s_, b)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y), want[i]), f"eager call {rep} of shape {shapes[i]}"
    stream = torch.cuda.Stream()
    outs = [torch.empty_like(y) for *_, y in probs]
    with torch.cuda.stream(stream):
        for i, (x, w, s_, b, _) in enumerate(probs):  # the stream's workspace, outside capture
            imq.quantized_matmul(x, w, s_, b, out=outs[i])
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i, (x, w, s_, b, _) in enumerate(probs):
            imq.quantized_matmul(x, w, s_, b, out=outs[i])
    for rep in range(4):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert np.array_equal(bits(o), want[i]), f"replay {rep} of shape {shapes[i]}"
        x, w, s_, b, _ = probs[0]
        assert np.array_equal(bits(imq.quantized_matmul(x, w, s_, b)), want[0])
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("m,n,k", [(4, 384, 512), (5, 384, 512), (16, 1001, 1024), (13, 17, 128),
                                   (8, 9728, 2560), (4, 2560, 9728), (5, 2560, 9728),
                                   (6, 2560, 9728), (8, 2560, 9728), (16, 2560, 9728),
                                   (9, 384, 192), (12, 9728, 2560), (16, 9728, 2560),
                                   (14, 3000, 4096), (12, 1000, 4608), (13, 1030, 4608),
                                   (3, 1001, 1024), (7, 1030, 2560), (8, 17, 512),
                                   (17, 2560, 9728), (30, 2560, 4096), (32, 2560, 9728),
                                   (24, 1030, 4608), (30, 1000, 4608), (20, 520, 9728),
                                   (29, 19400, 2560), (20, 2100, 4608), (7, 4100, 9728)])
def test_few_row_matrix_core_dispatch(dtype, m, n, k):
    """3 <= M <= 16 through the dispatcher.  The 16-row weight-streaming kernel
    stages x in LDS when M K 2, rounded up to whole wave instructions, fits
    96 KiB: M = 4 and 5 at K = 9728 (80 and exactly 96 KiB) take that path,
    M = 6 and 16 there (128 KiB and more) load x per chunk into registers.
    With x in LDS, M <= 8 and K % 512 == 0 its 8-row-load form runs (B
    columns = token and K half): 384 x 512 at M = 4, 5, [9728 x 2560] at M = 8,
    [2560 x 9728] at M = 4, 5, 1001 x 1024 at M = 3 and 17 x 512 at M = 8
    (partial row tiles; K = 512 is one span per wave pair), 1030 x 2560 at
    M = 7 (N % 4 != 0: single-element stores).
    12 <= M <= 16 with K <= 4096 (K % 512 == 0) take the multi-tile kernel
    with x in LDS where it fits one round of the CUs on less than 10 MiB of
    weights: 3000 x 4096 at M = 14 (a partial last tile), 1001 x 1024 at M =
    16.  N = 1001 and 17 end in a partial row block and take the
    single-element stores; K = 128 is one chunk; K % 128 != 0 (K = 192) runs
    the tiled kernel.  From M = 6 where x does not fit LDS, and from 12 rows
    where the multi-tile kernel would stream 10 MiB or more ([9728 x 2560] at
    M = 12 and 16), K is split (the rows-per-wave kernel; fp32 partial sums
    added in order by a second kernel): [2560 x 9728] at M = 6, 8 and 16, 1000
    x 4608 at M = 12, 1030 x 4608 at M = 13 (N % 4 != 0: the single-element
    partial stores and reduction), 4100 x 9728 at M = 7 (a partial last
    workgroup of 64 rows).  17 to 32 rows run only that split, with two token
    groups: [2560 x 9728] at M = 17 (the second group one token) and 32, 2560
    x 4096 at M = 30, 1030 x 4608 at M = 24, 1000 x 4608 at M = 30, 520 x 9728
    at M = 20 (a partial last row tile), 19400 x 2560 at M = 29 (two tiles per
    wave, the last tile partial), 2100 x 4608 at M = 20 (two 512-k pieces per
    split, the last split one: its second chunk block clamped).  Oracle
    within tolerance, the same bits on a second call, and one-hot rows
    reproduce the dequantized weights bit for bit (a one-hot row has one
    nonzero product in one split)."""
    note(f"few-row dispatch {dtype} M={m} N={n} K={k}")
    p = synth.make_problem(m, n, k, seed=23)
    x, w, s, b = synth.to_device(p)
    if dtype == "f16":
        x, s, b = x.half(), s.half(), b.half()
    y1 = imq.quantized_matmul(x, w, s, b)
    y2 = imq.quantized_matmul(x, w, s, b)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    if dtype == "bf16":
        assert_close(bits(y1), cref.qmm_t(p.x, p.w, p.scales, p.biases), "few-row")
    else:
        want = ref.qmm_t_as(x.cpu().numpy(), p.w, s.cpu().numpy(), b.cpu().numpy(), np.float16)
        st = ref.error_stats_values(y1.float().cpu().numpy(), want.astype(np.float32))
        note(f"  f16: mae={st['mae']:.3g} normwise={st['max_rel_normwise']:.3g}")
        assert st["mae"] <= MAE_TOL and st["max_rel_normwise"] <= NORMWISE_TOL, st
        assert st["cosine"] >= COSINE_MIN, st
    rng = np.random.default_rng(24)
    cols = rng.choice(k, size=m, replace=False)
    xh = np.zeros((m, k), dtype=np.uint16)
    xh[np.arange(m), cols] = 0x3F80 if dtype == "bf16" else 0x3C00
    xo = torch.from_numpy(xh.view(np.int16)).cuda().view(x.dtype)
    yo = imq.quantized_matmul(xo, w, s, b)
    deq = imq.dequantize(w, s, b)
    torch.cuda.synchronize()
    assert torch.equal(yo, deq[:, torch.from_numpy(cols).cuda()].T.contiguous())


def test_split_k_dispatcher_under_graph_capture():
    """A split-K call captured in a graph on a stream whose workspace exists
    replays to the eager bits, with other device work and synchronizations
    between replays, also after a larger call outgrew that workspace; captured
    on a stream that never ran it (no workspace, none grown under capture) it
    runs unsplit, within tolerance of the oracle."""
    m, n, k = 40, 1000, 2560
    note(f"split-K dispatcher under graph capture M={m} N={n} K={k}")
    p = synth.make_problem(m, n, k, seed=25)
    x, w, s, b = synth.to_device(p)
    side = torch.cuda.Stream()
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        imq.quantized_matmul(x, w, s, b, out=y)  # grows this stream's workspace
    side.synchronize()
    eager = bits(y)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        imq.quantized_matmul(x, w, s, b, out=y)
    for rep in range(3):
        y.zero_()
        torch.randn(1000, device="cuda").sum().item()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(y), eager), f"replay {rep}"
    # A larger split call on the same stream outgrows its workspace; the
    # graph still addresses the old one, which must stay allocated.
    pb = synth.make_problem(512, 2560, 9728, seed=26)
    xb, wb, sb, bb = synth.to_device(pb)
    with torch.cuda.stream(side):
        imq.quantized_matmul(xb, wb, sb, bb)
    side.synchronize()
    y.zero_()
    g.replay()
    torch.cuda.synchronize()
    assert np.array_equal(bits(y), eager), "replay after the workspace grew"
    fresh = torch.cuda.Stream()
    y2 = torch.empty_like(y)
    g2 = torch.cuda.CUDAGraph()
    fresh.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g2, stream=fresh):
        imq.quantized_matmul(x, w, s, b, out=y2)
    want = cref.qmm_t(p.x, p.w, p.scales, p.biases)
    for rep in range(2):
        y2.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert_close(bits(y2), want, f"unsplit capture, replay {rep}")


def test_weights_of_4_gib_take_the_64_bit_path():
    """Packed weights of 4 GiB are past the qGEMV kernel's 32-bit offsets: the
    dispatcher runs M=1 on the MFMA path's register-staged kernel, imq_qgemv
    refuses.  Every word is 0x76543210 (codes 0..7 in k order) with one scale
    and bias, so a one-hot x row picks the weight of code k % 8 in every row."""
    n, k = 262144, 32768  # n * k / 2 = 4 GiB
    note(f"4 GiB weights N={n} K={k} M=1")
    w = torch.full((n, k // 8), 0x76543210, dtype=torch.int32, device="cuda")
    s_bits, b_bits = 0x3C23, 0xBD23  # bf16 0.00995..., -0.0398...
    def as_i16(v):
        return int(np.array([v], np.uint16).view(np.int16)[0])

    s = torch.full((n, k // 64), as_i16(s_bits), dtype=torch.int16, device="cuda")
    b = torch.full((n, k // 64), as_i16(b_bits), dtype=torch.int16, device="cuda")
    s, b = s.view(torch.bfloat16), b.view(torch.bfloat16)
    col = 12345
    x = torch.zeros((1, k), dtype=torch.bfloat16, device="cuda")
    x[0, col] = 1.0
    y = bits(imq.quantized_matmul(x, w, s, b))
    q = col % 8
    sv = ref.bf16_to_f32(np.array([s_bits], np.uint16))[0]
    bv = ref.bf16_to_f32(np.array([b_bits], np.uint16))[0]
    want = ref.f32_to_bf16(np.array([np.float32(sv * np.float32(q)) + bv], np.float32))[0]
    assert np.all(y == want), (np.unique(y), want)
    with pytest.raises(_lib.ImqUnsupported):
        imq.qgemv(x, w, s, b)
    del w, s, b
    torch.cuda.empty_cache()


def test_small_tiles_plain_qgemm():
    """imq_qgemm at M <= 64 runs 32- and 64-row tiles (no split)."""
    for m in (17, 33, 64):
        note(f"qgemm small tiles M={m}")
        p = synth.make_problem(m, 768, 1024, seed=23 + m)
        x, w, s, b = synth.to_device(p)
        assert_close(bits(imq.qgemm(x, w, s, b)), cref.qmm_t(p.x, p.w, p.scales, p.biases),
                     f"qgemm M={m}")


# ----------------------------------------------------------- host interface


def test_row_offsets_like_direct_engine():
    note("qmm with row offsets (row halves)")
    p = synth.make_problem(64, 256, 384, seed=17)
    x, w, s, b = synth.to_device(p)
    q = imq.Q(w=w, s=s, b=b, n=256, k=384)
    y = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    imq.qmm(q, x, 0, y, 0, 32)
    imq.qmm(q, x, 32, y, 32, 32)
    want = cref.qmm_t(p.x, p.w, p.scales, p.biases)
    assert_close(bits(y), want, "row halves")


def test_quantized_linear_batched_input():
    note("QuantizedLinear on [2, 40, K]")
    p = synth.make_problem(80, 192, 256, seed=18)
    x, w, s, b = synth.to_device(p)
    lin = imq.QuantizedLinear(w, s, b)
    assert lin.in_features == 256 and lin.out_features == 192
    y = lin(x.view(2, 40, 256))
    assert tuple(y.shape) == (2, 40, 192)
    assert_close(bits(y).reshape(80, 192), cref.qmm_t(p.x, p.w, p.scales, p.biases), "3-D input")
    assert np.array_equal(bits(lin.dequantized()), cref.dequantize(p.w, p.scales, p.biases))


def test_runs_on_a_side_stream():
    note("qgemm on a non-default torch stream")
    p = synth.make_problem(200, 320, 512, seed=19)
    x, w, s, b = synth.to_device(p)
    base = bits(imq.qgemm(x, w, s, b))
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        y = imq.qgemm(x, w, s, b)
    st.synchronize()
    assert np.array_equal(bits(y), base)


def test_one_context_from_several_threads():
    """Four host threads share the device's context, each on its own stream,
    with split-K shapes (each stream's workspace is created and grown while the
    others run): every result equals the single-threaded one."""
    import threading

    note("one context, four threads, four streams")
    shapes = [(40, 1000, 2560), (96, 512, 4096), (300, 512, 768), (17, 384, 512)]
    probs = [synth.make_problem(m, n, k, seed=40 + i) for i, (m, n, k) in enumerate(shapes)]
    devs = [synth.to_device(p) for p in probs]
    want = [bits(imq.quantized_matmul(*d)) for d in devs]
    got = [[None] * 5 for _ in devs]
    errors = []

    def worker(i):
        try:
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                for r in range(5):
                    got[i][r] = imq.quantized_matmul(*devs[i])
            st.synchronize()
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(devs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for i, ys in enumerate(got):
        for r, y in enumerate(ys):
            assert np.array_equal(bits(y), want[i]), (shapes[i], r)


def test_argument_errors_are_reported():
    p = synth.make_problem(4, 64, 128, seed=20)
    x, w, s, b = synth.to_device(p)
    note("error paths")
    with pytest.raises(NotImplementedError):
        imq.quantized_matmul(x, w, s, b, group_size=32)
    with pytest.raises(NotImplementedError):
        imq.quantized_matmul(x, w, s, b, bits=8)
    with pytest.raises(NotImplementedError):
        imq.quantized_matmul(x.double(), w, s.double(), b.double())  # no f64 element type
    with pytest.raises(NotImplementedError):
        imq.quantized_matmul(x, w, s, b, transpose=False)
    with pytest.raises(ValueError):
        imq.qgemv(torch.cat([x] * 5), w, s, b)  # M = 20 > 16
    with pytest.raises(ValueError):
        imq.quantized_matmul(x[:, :64], w, s, b)  # K mismatch
    L = _lib.load()
    ctx = ops.context()
    y = torch.empty((4, 64), dtype=torch.bfloat16, device="cuda")
    vp = ctypes.c_void_p
    args = [vp(w.data_ptr()), vp(s.data_ptr()), vp(b.data_ptr()), vp(x.data_ptr()),
            vp(y.data_ptr())]
    st = L.imq_qmm_t(ctx, *args, 100, 64, 4, 64, 4, 0, None)  # K % 64 != 0
    assert st == _lib.IMQ_EINVAL and b"multiple of the group size" in L.imq_last_error(ctx)
    bad = list(args)
    bad[3] = vp(x.data_ptr() + 2)  # misaligned x
    assert L.imq_qmm_t(ctx, *bad, 128, 64, 4, 64, 4, 0, None) == _lib.IMQ_EINVAL
    bad = list(args)
    bad[0] = vp(0)
    assert L.imq_qmm_t(ctx, *bad, 128, 64, 4, 64, 4, 0, None) == _lib.IMQ_EINVAL
    assert L.imq_qmm_t(ctx, *args, 128, 64, 0, 64, 4, 0, None) == _lib.IMQ_EINVAL
    assert L.imq_qmm_t(ctx, *args, 128, 64, 4, 64, 8, 0, None) == _lib.IMQ_EUNSUPPORTED
    assert L.imq_qmm_t(ctx, *args, 128, 64, 4, 32, 4, 0, None) == _lib.IMQ_EUNSUPPORTED
    assert L.imq_qgemv(ctx, *args, 128, 64, 17, 64, 4, 0, None) == _lib.IMQ_EINVAL
    assert L.imq_dequantize(ctx, args[0], args[1], args[2], args[4], 128, 64, 64, 4, 7,
                            None) == _lib.IMQ_EUNSUPPORTED  # no such dtype
    out = ctypes.c_void_p()
    assert L.imq_create(10_000, ctypes.byref(out)) == _lib.IMQ_EINVAL


def test_plain_c_caller_on_the_device():
    """tests/c/abi_check.c, a C11 program linked against libimq.so: dequant
    against the closed form, one-hot qmm_t in both regimes, error statuses."""
    import subprocess

    from aestrix_amd import build

    note("plain C11 caller of the ABI")
    assert os.path.exists(build.ABI_CHECK), "abi_check is not built (python -m aestrix_amd.build)"
    r = subprocess.run([build.ABI_CHECK], capture_output=True, text=True, timeout=90)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checks passed" in r.stdout


def test_pure_c_abi_memory_stream_and_kernel():
    """Everything through the C ABI: imq_malloc / memcpy (h2d, d2d, d2h) / stream /
    dequant / qmm."""
    note("pure C-ABI round trip")
    L = _lib.load()
    ctx = ops.context()
    p = synth.make_problem(3, 128, 256, seed=21)
    stream = ctypes.c_void_p()
    _lib.check(L.imq_stream_create(ctx, ctypes.byref(stream)), ctx)
    bufs = {}
    host = {"w": p.w, "s": p.scales, "b": p.biases, "x": p.x}
    for name, a in host.items():
        ptr = ctypes.c_void_p()
        _lib.check(L.imq_malloc(ctx, a.nbytes, ctypes.byref(ptr)), ctx)
        _lib.check(L.imq_memcpy_h2d(ctx, ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                                    stream), ctx)
        bufs[name] = ptr
    deq = ctypes.c_void_p()
    y = ctypes.c_void_p()
    _lib.check(L.imq_malloc(ctx, 128 * 256 * 2, ctypes.byref(deq)), ctx)
    _lib.check(L.imq_malloc(ctx, 3 * 128 * 2, ctypes.byref(y)), ctx)
    _lib.check(L.imq_dequantize(ctx, bufs["w"], bufs["s"], bufs["b"], deq, 256, 128, 64, 4,
                                _lib.IMQ_BF16, stream), ctx)
    # x through a device-to-device copy into a second buffer.
    x2 = ctypes.c_void_p()
    _lib.check(L.imq_malloc(ctx, p.x.nbytes, ctypes.byref(x2)), ctx)
    _lib.check(L.imq_memcpy_d2d(ctx, x2, bufs["x"], p.x.nbytes, stream), ctx)
    bufs["x2"] = x2
    _lib.check(L.imq_qmm_t(ctx, bufs["w"], bufs["s"], bufs["b"], bufs["x2"], y, 256, 128, 3, 64,
                           4, _lib.IMQ_BF16, stream), ctx)
    deq_h = np.empty((128, 256), dtype=np.uint16)
    y_h = np.empty((3, 128), dtype=np.uint16)
    _lib.check(L.imq_memcpy_d2h(ctx, deq_h.ctypes.data_as(ctypes.c_void_p), deq, deq_h.nbytes,
                                stream), ctx)
    _lib.check(L.imq_memcpy_d2h(ctx, y_h.ctypes.data_as(ctypes.c_void_p), y, y_h.nbytes,
                                stream), ctx)
    _lib.check(L.imq_stream_sync(ctx, stream), ctx)
    for ptr in list(bufs.values()) + [deq, y]:
        _lib.check(L.imq_free(ctx, ptr), ctx)
    _lib.check(L.imq_stream_destroy(ctx, stream), ctx)
    assert np.array_equal(deq_h, cref.dequantize(p.w, p.scales, p.biases))
    assert_close(y_h, cref.qmm_t(p.x, p.w, p.scales, p.biases), "pure C ABI qmm")

"""imq_qmm_t_noalloc (the dispatcher with its split-K partial sums in the
library's static scratch) against imq_qmm_t, through the C ABI.

Both run the same plan and kernels, so the bar is bit-for-bit equality.  Each
case makes two calls in a row on one stream, the second with a smaller input,
so the second call runs on scratch the first one filled.  A shape whose plan
needs more scratch than the library holds is refused, and the entry point
captured in a HIP graph replays to the eager bits.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import aestrix_amd as imq
from aestrix_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 64 << 20


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def noalloc(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, b: torch.Tensor,
            y: torch.Tensor) -> None:
    """One imq_qmm_t_noalloc call on torch's current stream (raises on a status)."""
    n, k = w.shape[0], w.shape[1] * 8
    m = x.shape[0]
    ctx = ops.context(x.device)
    st = _lib.load().imq_qmm_t_noalloc(
        ctx, ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(s.data_ptr()),
        ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(x.data_ptr()),
        ctypes.c_void_p(y.data_ptr()), k, n, m, 64, 4, ops._DTYPES[x.dtype],
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(st, ctx)


def problem(m, n, k, seed, dtype):
    p = synth.make_problem(m, n, k, seed=seed)
    x, w, s, b = synth.to_device(p)
    if dtype == "f16":
        x, s, b = x.half(), s.half(), b.half()
    return x, w, s, b


def split_bytes(m, n, k):
    """Split-K workspace bytes of imq_qmm_t's plan for this shape (imq_qmm_plan)."""
    return imq.qmm_plan(m, n, k)["workspace_bytes"]


# (first, second): the second call's input is smaller.
PAIRS = [
    ((512, 2560, 9728), (32, 9728, 2560)),     # split-K plans, 3 then 5 splits
    ((2048, 2560, 9728), (128, 3072, 12288)),  # 60 MiB of scratch, then 15 MiB
    ((1024, 3072, 9216), (8, 9728, 2560)),     # split-K, then the few-row kernel
    ((40, 1000, 2560), (1, 2560, 9728)),       # split-K, then the qGEMV
    ((4608, 3072, 3072), (64, 3072, 3072)),    # unsplit tiles, then split-K (128-column tiles)
    ((16, 2560, 9728), (12, 1000, 4608)),      # the few-row kernel's K split: 10, then 9 splits
]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("first,second", PAIRS, ids=[f"{a[0]}x{a[1]}x{a[2]}-{b[0]}x{b[1]}x{b[2]}"
                                                    for a, b in PAIRS])
def test_noalloc_matches_qmm_t_on_two_calls(dtype, first, second):
    outs = []
    for i, (m, n, k) in enumerate((first, second)):
        note(f"noalloc {dtype} call {i}: M={m} N={n} K={k} (split-K scratch "
             f"{split_bytes(m, n, k)} bytes)")
        x, w, s, b = problem(m, n, k, seed=60 + i, dtype=dtype)
        y_na = torch.full((m, n), 3.0, dtype=x.dtype, device="cuda")
        noalloc(x, w, s, b, y_na)
        outs.append((x, w, s, b, y_na))
    torch.cuda.synchronize()
    for i, (x, w, s, b, y_na) in enumerate(outs):
        want = imq.quantized_matmul(x, w, s, b)
        torch.cuda.synchronize()
        assert torch.equal(y_na, want), f"call {i}: imq_qmm_t_noalloc differs from imq_qmm_t"


def test_noalloc_refuses_a_plan_past_the_static_scratch():
    # 224-row tiles, K split three ways: 3 x 1536 x 6144 fp32 partial sums (108 MiB).
    m, n, k = 1536, 6144, 32768
    need = split_bytes(m, n, k)
    note(f"noalloc M={m} N={n} K={k}: plan needs {need} bytes")
    assert need > STATIC_SCRATCH_BYTES
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    s = torch.zeros((n, k // 64), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.ImqInvalid, match="static scratch"):
        noalloc(x, w, s, s, y)


def test_noalloc_refuses_a_few_row_split_past_the_static_scratch():
    """At 16 rows the few-row kernel splits K when x does not fit LDS; with
    enough weight rows its partial sums outgrow the static scratch.  imq_qmm_t
    runs that split plan; the allocation-free entry point refuses the call
    rather than run a different plan (different bits)."""
    m, k = 16, 8192
    for n in (131072, 262144, 524288):
        plan = imq.qmm_plan(m, n, k)
        note(f"few-row plan M={m} N={n} K={k}: {plan}")
        if plan["kernel"] == "few_row" and plan["workspace_bytes"] > STATIC_SCRATCH_BYTES:
            break
    else:
        pytest.fail("no few-row split plan past the static scratch among the shapes tried")
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((n, k // 8), dtype=torch.int32, device="cuda")
    s = torch.zeros((n, k // 64), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.ImqInvalid, match="static scratch"):
        noalloc(x, w, s, s, y)
    del x, w, s, y
    torch.cuda.empty_cache()


def test_noalloc_calls_on_two_streams_are_ordered():
    """Eager calls on different streams share the one scratch; the library
    orders them on the GPU, so back-to-back calls on two streams (no host sync
    between) both return imq_qmm_t's bits."""
    # Split-K tile plans and few-row K splits (the shapes of the pairs above).
    shapes = [(512, 2560, 9728), (40, 1000, 2560), (16, 2560, 9728), (32, 9728, 2560)]
    probs = [problem(m, n, k, seed=80 + i, dtype="bf16") for i, (m, n, k) in enumerate(shapes)]
    for m, n, k in shapes:
        assert split_bytes(m, n, k) > 0, (m, n, k)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    ys = []
    for rep in range(3):
        for i, ((m, n, k), (x, w, s, b)) in enumerate(zip(shapes, probs)):
            y = torch.full((m, n), 5.0, dtype=torch.bfloat16, device="cuda")
            streams[i % 2].wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(streams[i % 2]):
                noalloc(x, w, s, b, y)
            ys.append((i, y))
    torch.cuda.synchronize()
    for i, y in ys:
        x, w, s, b = probs[i]
        assert torch.equal(y, imq.quantized_matmul(x, w, s, b)), f"shape {shapes[i]}"


def test_noalloc_under_graph_capture():
    """Captured on a fresh stream (where imq_qmm_t would have no workspace and
    would run unsplit), the entry point keeps its split plan; replays with
    other device work in between reproduce the eager bits."""
    m, n, k = 40, 1000, 2560
    note(f"noalloc graph capture M={m} N={n} K={k}")
    assert split_bytes(m, n, k) > 0
    x, w, s, b = problem(m, n, k, seed=70, dtype="bf16")
    eager = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    noalloc(x, w, s, b, eager)
    torch.cuda.synchronize()
    assert torch.equal(eager, imq.quantized_matmul(x, w, s, b))
    y = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        noalloc(x, w, s, b, y)
    for rep in range(3):
        y.fill_(7.0)
        torch.randn(1000, device="cuda").sum().item()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep}"

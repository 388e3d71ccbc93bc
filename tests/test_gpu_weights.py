"""GPU side of the packed-tensor loader: staged uploads, scale-dtype
conversion, resident projections feeding the matmul kernels.

Known answers: the bytes the `safetensors` package wrote; torch's own
bf16 -> f16 / f32 conversions (round to nearest even, exact widening); the CPU
oracle for the matmul on loaded weights (MAE <= 1e-3, normwise <= 1e-2).
"""

from __future__ import annotations

import ctypes
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import aestrix_amd as imq
from aestrix_amd import _lib, ops, synth, weights
from aestrix_amd.weights import SafetensorsSet, WeightsError
from oracle import ref

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def note(msg: str) -> None:
    print(msg, flush=True)


def packed(n: int, k: int, seed: int, p: synth.Problem | None = None) -> dict[str, torch.Tensor]:
    p = p if p is not None else synth.make_problem(0, n, k, seed=seed)
    return {
        "weight": torch.from_numpy(p.w.view(np.int32)).view(torch.uint32),
        "scales": torch.from_numpy(p.scales.view(np.int16)).view(torch.bfloat16),
        "biases": torch.from_numpy(p.biases.view(np.int16)).view(torch.bfloat16),
    }


def test_upload_raw_and_converted(tmp_path):
    note("loader: raw and converted uploads")
    g = torch.Generator().manual_seed(0)
    src = {
        "a.bf16": (torch.randn((300, 7), generator=g) * 1e3).to(torch.bfloat16),
        "a.f16": torch.randn((5, 9), generator=g).to(torch.float16),
        "a.f32": torch.randn((17,), generator=g),
        "a.u32": torch.randint(0, 2 ** 31, (33, 4), generator=g).to(torch.int32).view(torch.uint32),
    }
    src["a.bf16"][0, :4] = torch.tensor([1e-6, 70000.0, -1e-8, 65520.0]).to(torch.bfloat16)
    save_file(src, str(tmp_path / "0.safetensors"))
    with SafetensorsSet.open_dir(tmp_path) as st:
        b = src["a.bf16"].cuda()
        assert torch.equal(st.upload("a.bf16"), b)
        assert torch.equal(st.upload("a.bf16", torch.float16).view(torch.int16),
                           b.to(torch.float16).view(torch.int16))
        assert torch.equal(st.upload("a.bf16", torch.float32), b.float())
        assert torch.equal(st.upload("a.f16", torch.float32), src["a.f16"].cuda().float())
        assert torch.equal(st.upload("a.f32"), src["a.f32"].cuda())
        assert torch.equal(st.upload("a.u32"), src["a.u32"].view(torch.int32).cuda())
        with pytest.raises(NotImplementedError):
            st.upload("a.f32", torch.float16)  # no narrowing


def test_converted_upload_split_over_copy_threads(tmp_path):
    """Conversions of tensors large enough that each staging chunk is filled
    by several host threads (ragged element counts, chunk and part seams)."""
    note("loader: converted uploads over the copy threads")
    g = torch.Generator().manual_seed(3)
    src = {"big.bf16": (torch.randn((9 * 2 ** 20 + 77,), generator=g) * 50).to(torch.bfloat16),
           "big.f16": torch.randn((3 * 2 ** 20 + 5,), generator=g).to(torch.float16)}
    save_file(src, str(tmp_path / "0.safetensors"))
    with SafetensorsSet.open_dir(tmp_path) as st:
        b = src["big.bf16"].cuda()
        assert torch.equal(st.upload("big.bf16"), b)
        assert torch.equal(st.upload("big.bf16", torch.float32), b.float())
        assert torch.equal(st.upload("big.bf16", torch.float16).view(torch.int16),
                           b.to(torch.float16).view(torch.int16))
        assert torch.equal(st.upload("big.f16", torch.float32), src["big.f16"].cuda().float())


def test_upload_many_staging_chunks():
    """160 MiB through the two 32 MiB pinned buffers, with a ragged tail."""
    note("loader: imq_upload 160 MiB")
    L = _lib.load()
    ctx = ops.context()
    n = 160 * 2 ** 20 + 12345
    host = np.random.default_rng(1).integers(0, 255, n, dtype=np.uint8)
    dev = torch.empty(n, dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream()
    rc = L.imq_upload(ctx, ctypes.c_void_p(dev.data_ptr()), host.ctypes.data_as(ctypes.c_void_p),
                      n, ctypes.c_void_p(st.cuda_stream))
    _lib.check(rc, ctx)
    host[:] = 0  # the source may be reused as soon as the call returns
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy(),
                          np.random.default_rng(1).integers(0, 255, n, dtype=np.uint8))


@pytest.mark.parametrize("scales", [torch.bfloat16, torch.float16, torch.float32])
def test_loaded_projection_feeds_the_matmul(tmp_path, scales):
    n, k, m = 384, 1024, 24
    note(f"loader: load_qlinear scales={scales} N={n} K={k} M={m}")
    p = synth.make_problem(m, n, k, seed=40)
    t = packed(n, k, seed=40, p=p)
    save_file({f"layer.{key}": v for key, v in t.items()}, str(tmp_path / "0.safetensors"))
    with SafetensorsSet.open_dir(tmp_path) as st:
        q = weights.load_qlinear(st, "layer", scales, n=n, k=k)
    assert q.n == n and q.k == k and q.s.dtype == scales
    assert np.array_equal(q.w.cpu().numpy().view(np.uint32), p.w)
    x_bf16 = synth.to_device(p)[0]
    x = x_bf16.to(scales)  # bf16 activations are exact in f16 / f32 for this generator
    y = imq.quantized_matmul(x, q.w, q.s, q.b).cpu()
    s_np = q.s.cpu().float().numpy().astype(np.float16 if scales == torch.float16 else np.float32)
    b_np = q.b.cpu().float().numpy().astype(s_np.dtype)
    if scales == torch.bfloat16:
        want = ref.qmm_t(p.x, p.w, p.scales, p.biases)
        st_ = ref.error_stats(synth.bf16_bits(y), want)
    else:
        want = ref.qmm_t_as(x.cpu().numpy(), p.w, s_np, b_np, s_np.dtype)
        st_ = ref.error_stats_values(y.numpy(), want)
    note(f"  mae={st_['mae']:.3g} normwise={st_['max_rel_normwise']:.3g}")
    assert st_["mae"] <= 1e-3 and st_["max_rel_normwise"] <= 1e-2


def test_c_abi_load_qlinear_round_trip(tmp_path):
    """imq_load_qlinear (one allocation, f16 scales) read back through imq_memcpy_d2h."""
    note("loader: imq_load_qlinear C path")
    n, k = 96, 512
    t = packed(n, k, seed=41)
    save_file({f"x.{key}": v for key, v in t.items()}, str(tmp_path / "0.safetensors"))
    L = _lib.load()
    ctx = ops.context()
    with SafetensorsSet.open_dir(tmp_path) as st:
        q = _lib.QWeight()
        _lib.check(L.imq_load_qlinear(ctx, st.handle, b"x", _lib.IMQ_F16, ctypes.byref(q), None),
                   ctx)
        assert (q.n, q.k, q.dtype) == (n, k, _lib.IMQ_F16)
        _lib.check(L.imq_stream_sync(ctx, None), ctx)
        w = np.empty((n, k // 8), np.uint32)
        s = np.empty((n, k // 64), np.float16)
        _lib.check(L.imq_memcpy_d2h(ctx, w.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(q.w),
                                    w.nbytes, None), ctx)
        _lib.check(L.imq_memcpy_d2h(ctx, s.ctypes.data_as(ctypes.c_void_p),
                                    ctypes.c_void_p(q.scales), s.nbytes, None), ctx)
        assert np.array_equal(w, t["weight"].view(torch.int32).numpy().view(np.uint32))
        assert np.array_equal(s, t["scales"].float().numpy().astype(np.float16))
        _lib.check(L.imq_qweight_free(ctx, ctypes.byref(q)), ctx)
        assert q.base is None
        bad = _lib.QWeight()
        assert L.imq_load_qlinear(ctx, st.handle, b"y", _lib.IMQ_F16, ctypes.byref(bad),
                                  None) == _lib.IMQ_EINVAL
        assert b"missing tensor y.weight" in L.imq_last_error(ctx)


def test_dit_key_map_over_two_shards(tmp_path):
    """load_dit_blocks / load_dit_head over a two-shard pack with an index, at
    reduced widths (the key map is the reference's; only the sizes shrink)."""
    note("loader: DiT key map, reduced widths")
    dims = dict(dim=128, ff_inner=192, ff_wide=384, proj_width=512, concat_width=320)
    shard = [{}, {}]
    seed = 100
    for i in range(2):
        for name, n, k in weights.dit_double_linears(128, 192, 384):
            for key, v in packed(n, k, seed).items():
                shard[i % 2][f"transformer_blocks.{i}.{name}.{key}"] = v
            seed += 1
    for i in range(3):
        for name, n, k in weights.dit_single_linears(128, 512, 320):
            for key, v in packed(n, k, seed).items():
                shard[(i + 1) % 2][f"single_transformer_blocks.{i}.{name}.{key}"] = v
            seed += 1
    for name, n, k in (("x_embedder", 128, 128), ("proj_out", 128, 128)):
        for key, v in packed(n, k, seed).items():
            shard[0][f"{name}.{key}"] = v
        seed += 1
    wm = {}
    for j, sh in enumerate(shard):
        fn = f"model-0000{j + 1}-of-00002.safetensors"
        save_file(sh, str(tmp_path / fn))
        wm.update({key: fn for key in sh})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    with SafetensorsSet.open_dir(tmp_path) as st:
        blocks = weights.load_dit_blocks(st, n_double=2, n_single=3, dims=dims)
        head = weights.load_dit_head(st)
        assert len(blocks) == 2 * 12 + 3 * 2 and set(head) == {"x_embedder", "proj_out"}
        q = blocks["single_transformer_blocks.2.attn.to_out"]
        assert (q.n, q.k, q.s.dtype) == (128, 320, torch.float16)
        assert np.array_equal(q.s.cpu().numpy(),
                              shard[1]["single_transformer_blocks.2.attn.to_out.scales"]
                              .float().numpy().astype(np.float16))
        with pytest.raises(WeightsError, match="expected N=3072"):
            weights.load_dit_blocks(st, n_double=1, n_single=0)  # full-size map on a small pack


def test_concatenated_projections_c_abi_and_python(tmp_path):
    """imq_load_qlinear_cat / load_qlinear_cat: q, k, v (K shared, N 96 + 32 +
    32) as one projection whose rows are theirs in order, scales converted to
    f16; byte-equal to the parts loaded one by one.  A K mismatch is refused."""
    note("loader: concatenated projections (C and Python)")
    k = 512
    parts = {"q": packed(96, k, seed=51), "k": packed(32, k, seed=52), "v": packed(32, k, seed=53),
             "odd": packed(32, 256, seed=54)}
    save_file({f"l.{p}.{key}": v for p, t in parts.items() for key, v in t.items()},
              str(tmp_path / "0.safetensors"))
    L = _lib.load()
    ctx = ops.context()
    with SafetensorsSet.open_dir(tmp_path) as st:
        names = (ctypes.c_char_p * 3)(b"l.q", b"l.k", b"l.v")
        q = _lib.QWeight()
        _lib.check(L.imq_load_qlinear_cat(ctx, st.handle, names, 3, _lib.IMQ_F16,
                                          ctypes.byref(q), None), ctx)
        assert (q.n, q.k, q.dtype) == (160, k, _lib.IMQ_F16)
        _lib.check(L.imq_stream_sync(ctx, None), ctx)
        w = np.empty((160, k // 8), np.uint32)
        s = np.empty((160, k // 64), np.float16)
        b = np.empty((160, k // 64), np.float16)
        for dst, src in ((w, q.w), (s, q.scales), (b, q.biases)):
            _lib.check(L.imq_memcpy_d2h(ctx, dst.ctypes.data_as(ctypes.c_void_p),
                                        ctypes.c_void_p(src), dst.nbytes, None), ctx)
        want_w = np.concatenate([parts[p]["weight"].view(torch.int32).numpy().view(np.uint32)
                                 for p in ("q", "k", "v")])
        want_s = np.concatenate([parts[p]["scales"].float().numpy().astype(np.float16)
                                 for p in ("q", "k", "v")])
        want_b = np.concatenate([parts[p]["biases"].float().numpy().astype(np.float16)
                                 for p in ("q", "k", "v")])
        assert np.array_equal(w, want_w) and np.array_equal(s, want_s) and np.array_equal(b, want_b)
        _lib.check(L.imq_qweight_free(ctx, ctypes.byref(q)), ctx)
        bad_names = (ctypes.c_char_p * 2)(b"l.q", b"l.odd")
        bad = _lib.QWeight()
        assert L.imq_load_qlinear_cat(ctx, st.handle, bad_names, 2, _lib.IMQ_F16,
                                      ctypes.byref(bad), None) == _lib.IMQ_EINVAL
        assert b"K=" in L.imq_last_error(ctx)
        cat = weights.load_qlinear_cat(st, ["l.q", "l.k", "l.v"], torch.float16)
        torch.cuda.synchronize()
        assert cat.n == 160 and cat.k == k
        assert np.array_equal(cat.w.cpu().numpy().view(np.uint32), want_w)
        assert np.array_equal(cat.s.cpu().numpy(), want_s)
        assert np.array_equal(cat.b.cpu().numpy(), want_b)
        with pytest.raises(weights.WeightsError, match="disagree on K"):
            weights.load_qlinear_cat(st, ["l.q", "l.odd"])

"""The native safetensors reader (include/imq_weights.h) on the CPU.

Fixtures are written with the `safetensors` package (its own writer is the
known answer for dtype, shape and data offsets); no device is touched.
Shard discovery follows SafetensorsLoader.shardFileNames
(Sources/ImarelloWeights/SafetensorsLoader.swift:6-25); merging follows
loadMergedArrays (SafetensorsLoader+MLX.swift:7-17).
"""

from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import load_file, save_file

from aestrix_amd import weights
from aestrix_amd.weights import SafetensorsSet, WeightsError


def _tensors(seed: int = 0, prefix: str = "blk") -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return {
        f"{prefix}.weight": torch.randint(0, 2 ** 31, (8, 16), generator=g).to(torch.int32)
        .view(torch.uint32),
        f"{prefix}.scales": torch.rand((8, 2), generator=g).to(torch.bfloat16),
        f"{prefix}.biases": (torch.rand((8, 2), generator=g) - 0.5).to(torch.bfloat16),
        f"{prefix}.norm": torch.rand((5,), generator=g),
        f"{prefix}.half": torch.rand((3, 4), generator=g).to(torch.float16),
        f"{prefix}.empty": torch.zeros((0, 4), dtype=torch.float32),
        f"{prefix}.i64": torch.arange(6, dtype=torch.int64).reshape(2, 3),
    }


def _raw(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def test_header_known_answer(tmp_path):
    ts = _tensors()
    path = tmp_path / "0.safetensors"
    save_file(ts, str(path), metadata={"format": "mlx"})
    with SafetensorsSet.open([path]) as st:
        assert st.names() == sorted(ts)
        assert st.shard_paths == [str(path)]
        assert st.metadata(0, "format") == "mlx"
        assert st.metadata(0, "absent") is None
        hlen = struct.unpack("<Q", open(path, "rb").read(8))[0]
        header = json.loads(open(path, "rb").read()[8:8 + hlen])
        for name, t in ts.items():
            info = st.info(name)
            assert info.dtype == header[name]["dtype"]
            assert info.shape == tuple(header[name]["shape"]) == tuple(t.shape)
            b0, b1 = header[name]["data_offsets"]
            assert info.nbytes == b1 - b0
            assert np.array_equal(st.numpy(name), _raw(t))
        assert "blk.weight" in st and "nope" not in st


def test_views_match_the_package_reader(tmp_path):
    ts = _tensors(seed=3)
    path = tmp_path / "m.safetensors"
    save_file(ts, str(path))
    back = load_file(str(path))
    with SafetensorsSet.open([path]) as st:
        for name in ts:
            assert np.array_equal(st.numpy(name), _raw(back[name]))
            assert not st.numpy(name).flags.writeable


def test_directory_listing_order_and_later_shard_wins(tmp_path):
    a = _tensors(seed=1)
    b = _tensors(seed=2)
    b2 = {k.replace("blk.", "other."): v for k, v in _tensors(seed=4).items()}
    save_file(a, str(tmp_path / "1.safetensors"))
    save_file({**b, **b2}, str(tmp_path / "0.safetensors"))
    (tmp_path / "notes.txt").write_text("not a shard")
    with SafetensorsSet.open_dir(tmp_path) as st:
        assert [os.path.basename(p) for p in st.shard_paths] == ["0.safetensors", "1.safetensors"]
        # blk.* is in both shards: the later one in sorted order (1.safetensors) wins
        assert np.array_equal(st.numpy("blk.norm"), a["blk.norm"].numpy())
        assert st.info("blk.norm").shard == 1
        assert np.array_equal(st.numpy("other.norm"), b2["other.norm"].numpy())


def test_index_json_selects_and_orders_shards(tmp_path):
    a = _tensors(seed=1)
    b = {k.replace("blk.", "b2."): v for k, v in _tensors(seed=2).items()}
    save_file(a, str(tmp_path / "model-00002.safetensors"))
    save_file(b, str(tmp_path / "model-00001.safetensors"))
    save_file(_tensors(seed=9, prefix="stray"), str(tmp_path / "zz-unlisted.safetensors"))
    wm = {k: "model-00002.safetensors" for k in a}
    wm.update({k: "model-00001.safetensors" for k in b})
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 1}, "weight_map": wm}))
    with SafetensorsSet.open_dir(tmp_path) as st:
        assert [os.path.basename(p) for p in st.shard_paths] == [
            "model-00001.safetensors", "model-00002.safetensors"]
        assert "stray.norm" not in st and "b2.norm" in st and "blk.norm" in st


def test_malformed_index_falls_back_to_the_listing(tmp_path):
    save_file(_tensors(), str(tmp_path / "0.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text('{"weight_map": {"a": 3}}')
    with SafetensorsSet.open_dir(tmp_path) as st:
        assert len(st.shard_paths) == 1


def test_empty_directory_is_weights_not_found(tmp_path):
    with pytest.raises(WeightsError, match="weights not found"):
        SafetensorsSet.open_dir(tmp_path)


def _write_raw(path, header: dict, data: bytes, pad: bytes = b""):
    h = json.dumps(header).encode() + pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("header,data,msg", [
    ({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4, "past the"),
    ({"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8, "8 bytes for 3"),
    ({"t": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 2]}}, b"\0" * 2, "unknown dtype"),
    ({"t": {"dtype": "F32", "shape": [2]}}, b"\0" * 8, "needs dtype"),
    ({"t": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, b"\0" * 8, "bad shape"),
    ({"t": {"dtype": "U8", "shape": [4], "data_offsets": [4, 2]}}, b"\0" * 8, "bad data_offsets"),
    ({"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]},
      "b": {"dtype": "U8", "shape": [4], "data_offsets": [2, 6]}}, b"\0" * 8, "overlap"),
    ({"__metadata__": {"k": 3}}, b"", "not a string"),
])
def test_malformed_headers_are_rejected(tmp_path, header, data, msg):
    path = tmp_path / "bad.safetensors"
    _write_raw(path, header, data)
    with pytest.raises(WeightsError, match=msg):
        SafetensorsSet.open([path])


def test_truncated_and_garbage_files_are_rejected(tmp_path):
    p = tmp_path / "short.safetensors"
    p.write_bytes(b"\1\0\0")
    with pytest.raises(WeightsError, match="too short"):
        SafetensorsSet.open([p])
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(WeightsError, match="exceeds the file"):
        SafetensorsSet.open([p])
    p.write_bytes(struct.pack("<Q", 5) + b"{\"a\":")
    with pytest.raises(WeightsError, match="header"):
        SafetensorsSet.open([p])
    with pytest.raises(WeightsError, match="cannot open"):
        SafetensorsSet.open([tmp_path / "absent.safetensors"])


def test_json_escapes_and_padding(tmp_path):
    """Names with escapes and a space-padded header (the writer pads to 8 bytes)."""
    path = tmp_path / "esc.safetensors"
    name = 'weïrd "name"\\x/€'
    _write_raw(path, {name: {"dtype": "U8", "shape": [3], "data_offsets": [0, 3]}}, b"abc",
               pad=b"   ")
    with SafetensorsSet.open([path]) as st:
        assert st.names() == [name]
        assert st.numpy(name).tobytes() == b"abc"


def test_missing_tensor_message(tmp_path):
    save_file(_tensors(), str(tmp_path / "0.safetensors"))
    with SafetensorsSet.open_dir(tmp_path) as st:
        with pytest.raises(WeightsError, match="missing tensor nope.weight"):
            st.info("nope.weight")


def test_text_encoder_key_filter():
    keys = ["rotary_emb.inv_freq", "norm.weight", "norm.bias", "lm_head.weight",
            "embed_tokens.weight", "embed_tokens.scales", "layers.0.mlp.up_proj.weight",
            "layers.17.self_attn.q_proj.scales", "layers.18.mlp.down_proj.weight",
            "layers.x.foo", "layers.3", "layers.+2.a", "layers.-1.b"]
    assert weights.text_encoder_keys(keys, 18) == [
        "embed_tokens.weight", "embed_tokens.scales", "layers.0.mlp.up_proj.weight",
        "layers.17.self_attn.q_proj.scales", "layers.+2.a", "layers.-1.b"]


def test_key_maps_match_the_reference_dimensions():
    d = {n: (nn, k) for n, nn, k in weights.dit_double_linears()}
    assert d["attn.to_q"] == (3072, 3072) and d["ff.linear_in"] == (18432, 3072)
    assert d["ff.linear_out"] == (3072, 9216) and len(d) == 12
    s = {n: (nn, k) for n, nn, k in weights.dit_single_linears()}
    assert s == {"attn.to_qkv_mlp_proj": (27648, 3072), "attn.to_out": (3072, 12288)}
    t = {n: (nn, k) for n, nn, k in weights.te_linears()}
    assert t["mlp.gate_proj"] == (9728, 2560) and t["mlp.down_proj"] == (2560, 9728)
    assert t["self_attn.k_proj"] == (1024, 2560) and t["self_attn.o_proj"] == (2560, 4096)
    c = {n: (nn, k, dt) for n, nn, k, dt in weights.conditioner_linears()}
    assert c["context_embedder"] == (3072, 7680, torch.bfloat16)
    assert c["double_stream_modulation_img.linear"] == (18432, 3072, torch.float32)

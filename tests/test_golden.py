"""The oracle and the seeded generator reproduce the committed fixtures."""

import os

import numpy as np

from aestrix_amd import synth
from oracle import cref, ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


def test_generator_reproduces_fixture_inputs():
    d = np.load(GOLDEN)
    p = synth.make_problem(0, 48, 320, seed=101)
    assert np.array_equal(p.w, d["deq_w"])
    assert np.array_equal(p.scales, d["deq_s"]) and np.array_equal(p.biases, d["deq_b"])
    for i, (m, n, k, seed) in enumerate(d["qmm_cases"]):
        q = synth.make_problem(int(m), int(n), int(k), seed=int(seed))
        assert np.array_equal(q.x, d[f"qmm{i}_x"]) and np.array_equal(q.w, d[f"qmm{i}_w"])


def test_oracle_reproduces_dequant_fixtures():
    d = np.load(GOLDEN)
    for tag in ("deq", "kat"):
        w, s, b = d[f"{tag}_w"], d[f"{tag}_s"], d[f"{tag}_b"]
        assert np.array_equal(ref.dequantize(w, s, b), d[f"{tag}_out"])
        assert np.array_equal(cref.dequantize(w, s, b), d[f"{tag}_out"])


def test_oracle_reproduces_qmm_fixtures():
    d = np.load(GOLDEN)
    for i in range(len(d["qmm_cases"])):
        args = [d[f"qmm{i}_{t}"] for t in "xwsb"]
        assert np.array_equal(ref.qmm_t(*args), d[f"qmm{i}_y"])
        assert np.array_equal(cref.qmm_t(*args), d[f"qmm{i}_y"])


def test_generator_distributions():
    p = synth.make_problem(256, 512, 1024, seed=0)
    x = ref.bf16_to_f32(p.x)
    s = ref.bf16_to_f32(p.scales)
    b = ref.bf16_to_f32(p.biases)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    assert (s >= 0).all() and abs(float(s.mean()) - 0.02 * np.sqrt(2 / np.pi)) < 5e-4
    assert abs(float((b + 8 * s).std()) - 0.002) < 1e-4
    codes = ref.unpack_codes(p.w)
    counts = np.bincount(codes.reshape(-1), minlength=16) / codes.size
    assert np.all(np.abs(counts - 1 / 16) < 2e-3)

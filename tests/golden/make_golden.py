"""Writes tests/golden/golden.npz: small input/output vectors for the path.

The reference holds no golden vectors for the quantized linear (its tests pin
no quantized numerics), so these fixtures are produced by this repository's
seeded generator (aestrix_amd.synth) and its pinned CPU oracle (oracle/), and
serve as regression pins for the oracle and the HIP kernels.

Cases:
  deq_*   dequantize, N=48, K=320, seed 101
  kat_*   known-answer words 0x76543210 / 0xFEDCBA98 with hand-picked scales
  qmm{i}_* quantized matmul cases (M, N, K, seed) below; y is the oracle output
           RNE_bf16(x . deq(W)^T) accumulated in double.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from aestrix_amd import synth  # noqa: E402
from oracle import cref, ref  # noqa: E402

QMM_CASES = [(1, 40, 256, 201), (5, 64, 192, 202), (16, 72, 128, 203), (37, 96, 384, 204)]


def main() -> None:
    out = {}
    p = synth.make_problem(0, 48, 320, seed=101)
    out["deq_w"], out["deq_s"], out["deq_b"] = p.w, p.scales, p.biases
    out["deq_out"] = ref.dequantize(p.w, p.scales, p.biases)
    assert np.array_equal(out["deq_out"], cref.dequantize(p.w, p.scales, p.biases))

    kat_w = np.array([[0x76543210, 0xFEDCBA98] * 4] * 4, dtype=np.uint32)
    kat_s = np.array([[0x3F80], [0x3F00], [0x3CA4], [0xBEAB]], dtype=np.uint16)
    kat_b = np.array([[0x0000], [0xC080], [0xBE24], [0x3F80]], dtype=np.uint16)
    out["kat_w"], out["kat_s"], out["kat_b"] = kat_w, kat_s, kat_b
    out["kat_out"] = ref.dequantize(kat_w, kat_s, kat_b)

    for i, (m, n, k, seed) in enumerate(QMM_CASES):
        q = synth.make_problem(m, n, k, seed=seed)
        y = ref.qmm_t(q.x, q.w, q.scales, q.biases)
        assert np.array_equal(y, cref.qmm_t(q.x, q.w, q.scales, q.biases))
        out[f"qmm{i}_x"], out[f"qmm{i}_w"] = q.x, q.w
        out[f"qmm{i}_s"], out[f"qmm{i}_b"], out[f"qmm{i}_y"] = q.scales, q.biases, y
    out["qmm_cases"] = np.array(QMM_CASES, dtype=np.int64)
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

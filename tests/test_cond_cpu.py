"""The conditioning chain's host parts without a GPU: the C library's
sinusoid (include/imq_cond.h) against the oracle's, and the argument checks
that run before any device call."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from aestrix_amd import _lib
from aestrix_amd.cond import HEADS, sinusoid, split_heads
from oracle import ref


def test_host_sinusoid_within_an_ulp_of_the_oracle():
    """The C library's expf / logf / cosf / sinf against correctly rounded
    float64 evaluations of the same float operations: at most one ulp of the
    frequency, which t multiplies, plus one output ulp."""
    t = np.float32([0.0, 1.0, 0.5, 3.0, 17.25, 250.0, 500.0, 750.0, 999.0, 1000.0, -3.0])
    got = sinusoid(t, 256)
    want = ref.cond_sinusoid(t, 256)
    assert got.shape == (t.size, 256) and got.dtype == np.float32
    assert np.array_equal(got[0], want[0])  # t = 0: ones then zeros
    half = np.float32(128)
    freq = np.exp(((-np.log(np.float32(10000)) * np.arange(128, dtype=np.float32)) / half)
                  .astype(np.float64)).astype(np.float32)
    bound = (np.spacing(np.maximum(np.abs(want), np.float32(2 ** -24)))
             + np.abs(t[:, None]) * np.tile(np.spacing(freq), 2)[None, :])
    assert np.all(np.abs(got - want) <= bound)
    exact = np.mean(got == want)
    print(f"sinusoid: {exact:.4f} of the values equal the oracle's bit for bit")
    assert exact > 0.9


def test_sinusoid_argument_checks():
    L = _lib.load()
    t = np.float32([1.0])
    out = np.empty(8, np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert L.imq_cond_sinusoid(p(t), 1, 7, p(out)) == _lib.IMQ_EINVAL  # odd width
    assert L.imq_cond_sinusoid(p(t), -1, 8, p(out)) == _lib.IMQ_EINVAL
    assert L.imq_cond_sinusoid(None, 1, 8, p(out)) == _lib.IMQ_EINVAL
    assert L.imq_cond_sinusoid(None, 0, 8, None) == _lib.IMQ_OK
    assert L.imq_cond_step_conditioning(None, p(t), 1, None, None, None) == _lib.IMQ_EINVAL
    assert L.imq_cond_create(None, None, None, None, None) == _lib.IMQ_EINVAL
    assert L.imq_cond_destroy(None) == _lib.IMQ_OK


def test_split_heads_layout():
    """The heads' concatenation order and the reference's triples: img (2 sets),
    txt (2 sets), single (1 set), then norm_out's scale and shift."""
    import torch
    dim = 4
    assert sum(r for _, r in HEADS) == 17
    heads = torch.arange(17 * dim, dtype=torch.float32)
    sc = split_heads(torch.zeros(dim), heads, dim)
    assert [int(t[0]) for t in sc.double_img[0]] == [0, 4, 8]
    assert [int(t[0]) for t in sc.double_img[1]] == [12, 16, 20]
    assert [int(t[0]) for t in sc.double_txt[1]] == [36, 40, 44]
    assert [int(t[0]) for t in sc.single] == [48, 52, 56]
    assert int(sc.out_scale[0]) == 60 and int(sc.out_shift[-1]) == 67
    with pytest.raises(ValueError):
        split_heads(torch.zeros(dim), heads[:-1], dim)

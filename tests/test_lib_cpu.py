"""The C-ABI library loads and exports the header's entry points (no GPU needed).

No kernel is launched here: only symbol lookup, status strings and argument
checks that fail before any device work.
"""

import ctypes
import glob
import os
import re

import pytest

from aestrix_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(imq_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run `python -m aestrix_amd.build` first"


def test_every_declared_symbol_is_exported_and_bound():
    L = _lib.load()
    declared = header_functions()
    assert len(declared) >= 16
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/ but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared)


def test_only_the_c_abi_is_exported():
    """The dynamic symbol table holds exactly the header's imq_* functions: the
    C++ internals are local, so another copy of them in the process cannot
    interpose on this library's calls (nor this library on its)."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert exported == set(header_functions()), sorted(exported ^ set(header_functions()))


def test_status_strings_and_version():
    L = _lib.load()
    assert L.imq_abi_version() == 2
    assert L.imq_status_string(0) == b"IMQ_OK"
    assert L.imq_status_string(1) == b"IMQ_EINVAL"
    assert L.imq_status_string(2) == b"IMQ_EUNSUPPORTED"
    assert L.imq_status_string(3) == b"IMQ_EHIP"
    assert L.imq_status_string(4) == b"IMQ_ENOMEM"
    assert L.imq_status_string(99) == b"IMQ_UNKNOWN"


def test_null_context_is_rejected_without_device_work():
    L = _lib.load()
    nul = ctypes.c_void_p()
    for fn in ("imq_qmm_t", "imq_qgemv", "imq_qgemm"):
        st = getattr(L, fn)(nul, nul, nul, nul, nul, nul, 64, 8, 1, 64, 4, 0, nul)
        assert st == _lib.IMQ_EINVAL
        assert b"null context" in L.imq_last_error(nul)
    st = L.imq_dequantize(nul, nul, nul, nul, nul, 64, 8, 64, 4, 0, nul)
    assert st == _lib.IMQ_EINVAL
    assert L.imq_create(0, None) == _lib.IMQ_EINVAL
    assert L.imq_stream_sync(nul, nul) == _lib.IMQ_EINVAL
    assert L.imq_malloc(nul, 16, None) == _lib.IMQ_EINVAL


def test_check_maps_status_to_exceptions():
    L = _lib.load()
    nul = ctypes.c_void_p()
    L.imq_qmm_t(nul, nul, nul, nul, nul, nul, 64, 8, 1, 64, 4, 0, nul)
    with pytest.raises(ValueError):
        _lib.check(_lib.IMQ_EINVAL, nul)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.IMQ_EUNSUPPORTED, nul)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.IMQ_EHIP, nul)


def test_device_index_normalisation():
    import torch

    from aestrix_amd import ops

    assert ops.device_index(3) == 3
    assert ops.device_index("cuda:2") == 2
    assert ops.device_index(torch.device("cuda", 1)) == 1
    with pytest.raises(ValueError):
        ops.device_index("cpu")


def test_plain_c_caller_without_device():
    """tests/c/abi_check.c binds the C ABI from C11 (no ctypes): version,
    status strings and null-context validation need no GPU."""
    import subprocess

    from aestrix_amd import build

    if not os.path.exists(build.ABI_CHECK):
        pytest.skip("abi_check is not built (python -m aestrix_amd.build)")
    r = subprocess.run([build.ABI_CHECK, "--no-device"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 0, r.stderr
    assert "checks passed" in r.stdout

"""libimq's host C++ under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

tests/sanitize/Makefile builds capi.cpp, weights.cpp and step.cpp -- the
safetensors reader (a hand-written JSON parser over untrusted headers and
index files, SafetensorsLoader.swift:6-25's discovery rule) and every C entry
point's argument checks -- with -fsanitize=address,undefined and stubs of the
device launchers, and a seeded fuzz driver: well-formed shards (every tensor's
bytes read back), truncated and bit-flipped files, random header lengths,
junk and deeply nested JSON, overlapping / out-of-range offsets, bad shapes
and dtypes, directories with malformed or dangling index files, and null /
malformed arguments to the C ABI.  Any sanitizer report fails the run.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "sanitize")
BIN = os.path.join(SAN, "_build", "fuzz_host")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.fixture(scope="module")
def fuzz_host():
    if not os.path.exists(CLANG) or shutil.which("make") is None:
        pytest.skip("ROCm clang++ or make not available")
    r = subprocess.run(["make", "-s", "-C", SAN], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return BIN


@pytest.mark.parametrize("seed", [1, 2])
def test_host_code_is_clean_under_asan_and_ubsan(fuzz_host, tmp_path, seed):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([fuzz_host, str(tmp_path / "fz"), "3000", str(seed)], capture_output=True,
                       text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    m = re.search(r"fuzz_host: (\d+) files, (\d+) opened, (\d+) rejected, (\d+) abi checks", out)
    assert m, out
    files, opened, rejected, checks = map(int, m.groups())
    assert files == 3000 and opened > 500 and rejected > 500 and checks >= 40

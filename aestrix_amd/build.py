"""Compile the gfx950 HIP library ``aestrix_amd/libimq.so`` in-tree.

Every HIP translation unit is compiled with
``-Xclang -target-feature -Xclang -packed-fp32-ops`` so that hipcc emits no
packed-fp32 VALU instructions.  Objects go to ``aestrix_amd/_build/``.

Usage: ``python -m aestrix_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libimq.so")
ARCH = os.environ.get("IMQ_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC, "-Wall", "-Wno-unused-function",
]


def sources() -> list[str]:
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, name))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    # Export the C ABI only (imq_*), the C++ internals stay local.
    exports = os.path.join(CSRC, "exports.map")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC",
           f"-Wl,--version-script={exports}", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    build_abi_check(verbose)
    return LIB


ABI_CHECK_SRC = os.path.join(ROOT, "tests", "c", "abi_check.c")
ABI_CHECK = os.path.join(ROOT, "tests", "c", "abi_check")


def build_abi_check(verbose: bool = False) -> str | None:
    """The plain-C11 caller of the C ABI (tests/c/abi_check.c), linked against
    the in-tree libimq.so with an rpath relative to itself."""
    if not os.path.exists(ABI_CHECK_SRC):
        return None
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        return None
    cmd = [cc, "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-ffp-contract=off",
           "-I", INCLUDE, ABI_CHECK_SRC, "-o", ABI_CHECK, "-L", PKG, "-limq",
           "-Wl,-rpath,$ORIGIN/../../aestrix_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {ABI_CHECK_SRC} failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {ABI_CHECK}")
    return ABI_CHECK


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

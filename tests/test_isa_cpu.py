"""The manual vector-memory waits of the built kernels, checked on their gfx950
machine code (CPU only: the code objects are taken out of aestrix_amd/libimq.so
with the ROCm LLVM tools and disassembled).

Several kernels count their own loads instead of waiting for all of them
(loads complete in issue order):

* qgemm_big_kernel: a K-step's top waits with `s_waitcnt vmcnt(n)` (n the
  loads the previous step issued, left in flight) and then `s_barrier`.  The
  wait is right only if every path from the previous step-top barrier to it
  issues at least n loads -- which the compiler can break by dropping loads
  whose registers are never read again.
* the qGEMV and the few-row kernels (qgemv_*kernel, qskinny_*_kernel): x goes
  to LDS by direct buffer->LDS loads, then the weight, scale and bias loads;
  a `vmcnt(n)` and a barrier make x visible while those n stay in flight, so
  every path from the last LDS load to the wait must issue at least n others
  -- which a load sunk past the wait into a conditional block breaks.

A min-over-paths dataflow over each kernel's control-flow graph (branch
targets from the disassembly) checks every such wait.
"""

from __future__ import annotations

import os
import re
import subprocess
from pathlib import Path

import pytest

from aestrix_amd import _lib

LLVM = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin"
TOOLS = {n: LLVM / n for n in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf",
                               "llvm-objdump")}
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
KERNELS = ("qgemm_big_kernel", "qskinny_", "qgemv_")

INSN = re.compile(r"^\s+(\S+)\s*([^/]*?)\s*//\s*([0-9A-Fa-f]+):")
TARGET_RE = re.compile(r"<(\S+)\+0x([0-9a-f]+)>")
VMCNT = re.compile(r"vmcnt\((\d+)\)")


def _run(*args: str) -> str:
    return subprocess.run(args, check=True, capture_output=True, text=True).stdout


@pytest.fixture(scope="module")
def disasm(tmp_path_factory) -> dict[str, list[tuple[int, str, str]]]:
    """{kernel symbol: [(address, mnemonic, operands + comment)]} for the two kernels."""
    if not all(p.exists() for p in TOOLS.values()):
        pytest.skip("ROCm LLVM tools are not installed")
    lib = Path(_lib.LIB_PATH)
    if not lib.exists():
        pytest.skip("libimq.so is not built")
    d = tmp_path_factory.mktemp("co")
    fat = d / "fatbin.bin"
    _run(str(TOOLS["llvm-objcopy"]), f"--dump-section=.hip_fatbin={fat}", str(lib), str(d / "x.so"))
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    out: dict[str, list[tuple[int, str, str]]] = {}
    for n, o in enumerate(starts):
        end = starts[n + 1] if n + 1 < len(starts) else len(data)
        b = d / f"b{n}.bin"
        b.write_bytes(data[o:end])
        co = d / f"b{n}.co"
        _run(str(TOOLS["clang-offload-bundler"]), "--unbundle", "--type=o", f"--input={b}",
             f"--targets={TARGET}", f"--output={co}")
        syms = [line.split()[-1] for line in _run(str(TOOLS["llvm-readelf"]), "-sW", str(co))
                .splitlines() if "FUNC" in line and any(k in line for k in KERNELS)]
        if not syms:
            continue
        # In batches: one argument naming every kernel is longer than the OS allows.
        text = "\n".join(
            _run(str(TOOLS["llvm-objdump"]), "-d",
                 f"--disassemble-symbols={','.join(syms[i:i + 100])}", str(co))
            for i in range(0, len(syms), 100))
        cur = None
        for line in text.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
            if m:
                cur = m.group(1)
                out[cur] = []
                continue
            m = INSN.match(line)
            if cur and m:
                out[cur].append((int(m.group(3), 16), m.group(1), line))
    return out


def _min_counts(insns, count, reset) -> list[int]:
    """Fewest counted instructions since the last reset (or the kernel's entry)
    on any path to each instruction (before it executes)."""
    addr = {a: i for i, (a, _, _) in enumerate(insns)}
    base = insns[0][0]
    big = 1 << 20
    best = [big] * len(insns)
    best[0] = 0
    work = [0]
    while work:
        i = work.pop()
        a, mn, line = insns[i]
        v = best[i]
        v = 0 if reset(mn, line) else v + (1 if count(mn, line) else 0)
        v = min(v, 64)
        succ = []
        if mn != "s_endpgm" and mn != "s_branch" and i + 1 < len(insns):
            succ.append(i + 1)
        if mn.startswith("s_cbranch") or mn == "s_branch":
            t = TARGET_RE.search(line)  # <kernel+offset>: offset from the kernel's start
            j = addr.get(base + int(t.group(2), 16)) if t else None
            assert j is not None, f"branch target not found: {line}"
            succ.append(j)
        for j in succ:
            if v < best[j]:
                best[j] = v
                work.append(j)
    return best


def _is_load(mn: str) -> bool:
    return mn.startswith(("buffer_load", "global_load"))


def _is_dma(mn: str, line: str) -> bool:
    return mn.startswith("buffer_load") and re.search(r"\blds\b", line) is not None


def _step_waits(insns):
    """(index, n) of each `s_waitcnt vmcnt(n)` directly followed by s_barrier."""
    res = []
    for i in range(len(insns) - 1):
        mn, line = insns[i][1], insns[i][2]
        if mn == "s_waitcnt" and insns[i + 1][1] == "s_barrier":
            m = VMCNT.search(line)
            if m:
                res.append((i, int(m.group(1))))
    return res


def _family(sym: str) -> str:
    m = re.search(r"N_1\d+(\w+?_kernel)", sym)
    return m.group(1) if m else sym


def test_kernels_found(disasm):
    fams = {}
    for sym in disasm:
        fams[_family(sym)] = fams.get(_family(sym), 0) + 1
    for fam, least in (("qgemm_big_kernel", 20), ("qskinny_rows_kernel", 8), ("qgemv_kernel", 20),
                       ("qskinny_lds8_kernel", 4), ("qskinny_half_kernel", 4)):
        assert fams.get(fam, 0) >= least, (fam, fams)


def test_tile_kernel_step_waits_cover_the_previous_step(disasm):
    bad = []
    checked = 0
    for sym, insns in disasm.items():
        if _family(sym) != "qgemm_big_kernel":
            continue
        cnt = _min_counts(insns, lambda mn, l: _is_load(mn), lambda mn, l: mn == "s_barrier")
        for i, n in _step_waits(insns):
            checked += 1
            if cnt[i] < n:
                bad.append((sym[-60:], hex(insns[i][0]), f"vmcnt({n}) after {cnt[i]} loads"))
    assert checked > 0
    assert not bad, bad


def test_lds_dma_waits_leave_only_later_loads(disasm):
    bad = []
    checked = 0
    for sym, insns in disasm.items():
        if _family(sym) == "qgemm_big_kernel" or not any(_is_dma(mn, l) for _, mn, l in insns):
            continue
        waits = [(i, n) for i, n in _step_waits(insns) if n > 0]
        if _family(sym) == "qskinny_rows_kernel":
            assert waits, f"{sym}: no wait before the first barrier"
        cnt = _min_counts(insns, lambda mn, l: _is_load(mn) and not _is_dma(mn, l),
                          lambda mn, l: _is_dma(mn, l))
        for i, n in waits:
            checked += 1
            if cnt[i] < n:
                bad.append((sym[-60:], hex(insns[i][0]),
                            f"vmcnt({n}) after {cnt[i]} loads since the last LDS load"))
    assert checked > 400
    assert not bad, bad

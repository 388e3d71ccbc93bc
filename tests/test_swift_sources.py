"""The Swift layer under swift/ is not compiled here (no Swift toolchain); this
checks what can be checked without one: every C entry point its sources call
is declared in include/*.h with the same number of arguments, and the module
map's shim includes every public header."""

from __future__ import annotations

import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declarations() -> tuple[dict[str, int], set[str]]:
    """Functions (name -> parameter count) and struct types of the headers."""
    decls, structs = {}, set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"\b(imq_\w+)\s*\(([^;{]*?)\)\s*;", text):
            args = m.group(2).strip()
            decls[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
        structs.update(re.findall(r"typedef struct (imq_\w+)\s*\{", text))
    return decls, structs


def _calls(text: str):
    """(name, argument count) of each imq_* call, counting top-level commas."""
    for m in re.finditer(r"\b(imq_\w+)\(", text):
        depth, i, commas, empty = 1, m.end(), 0, True
        while depth:
            c = text[i]
            if c in "([{":
                depth += 1
            elif c in ")]}":
                depth -= 1
            elif c == "," and depth == 1:
                commas += 1
            if depth and not c.isspace():
                empty = False
            i += 1
        yield m.group(1), 0 if empty else commas + 1


def test_swift_calls_match_the_headers():
    decls, structs = _declarations()
    sources = glob.glob(os.path.join(ROOT, "swift", "Sources", "**", "*.swift"), recursive=True)
    assert len(sources) >= 6
    seen = set()
    for path in sources:
        code = re.sub(r"//[^\n]*", "", open(path).read())  # comments name functions too
        for name, n in _calls(code):
            if name in structs:  # a C struct's memberwise initializer
                continue
            assert name in decls, f"{os.path.basename(path)} calls {name}, declared nowhere"
            assert n == decls[name], f"{os.path.basename(path)}: {name} with {n} args, header has {decls[name]}"
            seen.add(name)
    for needed in ("imq_qmm_t", "imq_dit_step_denoise", "imq_cond_step_conditioning",
                   "imq_dit_double_attn_in", "imq_dit_single_attn_out", "imq_dit_head_out",
                   "imq_te_attn_out_mlp", "imq_load_qlinear_cat", "imq_qmm_postscale_ex"):
        assert needed in seen, needed


def test_module_map_covers_every_header():
    shim = open(os.path.join(ROOT, "swift", "Sources", "CImq", "shim.h")).read()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        assert f'include/{os.path.basename(h)}"' in shim, os.path.basename(h)

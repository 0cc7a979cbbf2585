"""Compile every call that the integration guide documents against the library's
headers, so the integration guide cannot drift from the ABI.

Each ```c block of the guide becomes the body of a function of its own;
each `ane_lm::...(...)` replacement in the call-site table becomes a
statement of a function whose parameters are the reference's variables at
those call sites.  The names the blocks use are declared (never defined) in
tests/cpp/integration_prelude.hpp, and the translation unit is checked with
g++ -fsyntax-only -Werror: an argument of the wrong type (an int where a
pointer goes, as a swapped argument order gives) or a wrong argument count
fails.  build() runs this; tests/test_integration_doc.py also plants such a
mistake and expects the check to fail.

    python tests/cpp/integration_doc.py      # prints the generated file's path
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
DOC = os.path.join(ROOT, "INTEGRATION.md")
BUILD = os.path.join(ROOT, "ane-lm_amd", "_build")

_BLOCK = re.compile(r"^```c\n(.*?)^```", re.S | re.M)
_DROPIN_CALL = re.compile(r"`(ane_lm::[A-Za-z_][\w:]*\([^`]*\))`")


def extract(md: str) -> tuple[list[str], list[str]]:
    """(code blocks, ane_lm:: replacement calls) of the guide's text."""
    blocks = [b for b in _BLOCK.findall(md)]
    calls = _DROPIN_CALL.findall(md)
    return blocks, calls


def translation_unit(md: str) -> str:
    blocks, calls = extract(md)
    if not blocks or not calls:
        raise ValueError("INTEGRATION.md: no ```c blocks or ane_lm:: call-site replacements found")
    out = ['#include "integration_prelude.hpp"', "", "namespace doc {", ""]
    for i, b in enumerate(blocks):
        body = "\n".join(l for l in b.splitlines() if not l.lstrip().startswith("#include"))
        out += [f"void documented_block_{i}() {{", body, "}", ""]
    out += ["void documented_call_sites(ANELM_DOC_CALL_SITE_PARAMS) {"]
    out += [f"    {c};" for c in calls]
    out += ["}", "", "}  // namespace doc", ""]
    return "\n".join(out)


def check(md: str | None = None, out_dir: str = BUILD, cxx: str = "g++") -> str:
    """Write the translation unit for the guide's text (default: the file)
    and compile it; raises RuntimeError with the compiler's messages if any
    documented call does not compile.  Returns the generated file's path."""
    if md is None:
        with open(DOC, encoding="utf-8") as f:
            md = f.read()
    os.makedirs(out_dir, exist_ok=True)
    src = os.path.join(out_dir, f"integration_doc_{os.getpid()}.cpp")
    with open(src, "w", encoding="utf-8") as f:
        f.write(translation_unit(md))
    cmd = [cxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-Wno-unused-variable",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "ane-lm_amd", "host"), "-I", HERE, src]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("INTEGRATION.md: documented calls do not compile against the headers\n" + r.stdout)
    final = os.path.join(out_dir, "integration_doc.cpp")
    os.replace(src, final)
    return final


if __name__ == "__main__":
    try:
        print(check())
    except (RuntimeError, ValueError) as e:
        sys.stderr.write(str(e) + "\n")
        sys.exit(1)

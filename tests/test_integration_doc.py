"""The reference-side C++ adapter in the repository's integration guide (its
first cpp block) keeps compiling against the interface it implements
(engine/strata/warm/runtime.hpp:10-16, WarmRedirect) and this repository's C
ABI (include/crosslane.h), and every entry point the guide names exists in the
header. CPU only; the compile check is skipped
where the reference tree is absent (the GPU box)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE = "/root/reference"
DOC = os.path.join(ROOT, "INTEGRATION.md")
HEADER = os.path.join(ROOT, "include", "crosslane.h")


def cpp_blocks():
    return re.findall(r"```cpp\n(.*?)```", open(DOC).read(), re.S)


def test_adapter_compiles_against_warm_runtime(tmp_path):
    if not os.path.isfile(os.path.join(REFERENCE, "engine/strata/warm/runtime.hpp")):
        pytest.skip("reference tree absent")
    if shutil.which("g++") is None:
        pytest.skip("g++ absent")
    adapter = cpp_blocks()[0]
    assert "class Mi355xLane final : public WarmRedirect" in adapter
    src = tmp_path / "adapter.cpp"
    src.write_text(adapter)
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", f"-I{REFERENCE}",
                        f"-I{os.path.join(ROOT, 'include')}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_named_entry_points_are_declared():
    header = open(HEADER).read()
    declared = set(re.findall(r"\b(xl_[a-z0-9_]+)\s*\(", header))
    named = set(re.findall(r"\b(xl_[a-z0-9_]+)\b", open(DOC).read()))
    named -= {"xl_context", "xl_config", "xl_error"}   # types
    missing = sorted(n for n in named if n not in declared)
    assert not missing, missing

"""The C-ABI library loads without a GPU and exports every function that
include/qsrt_amd.h declares (no compute calls here)."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

from qsrt_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "qsrt_amd.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(qsrt_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_viterbi_boundary():
    names = declared_functions()
    assert {"qsrt_viterbi_tiles", "qsrt_viterbi_workspace_bytes", "qsrt_last_error", "qsrt_abi_version"} <= names


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    exported = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}\b", exported), f"{name} is declared but not exported"
        assert hasattr(lib, name)


def test_python_signatures_cover_the_header():
    assert declared_functions() == set(_native.SIGNATURES)


def test_abi_version_and_error_string_without_gpu():
    lib = _native.lib()
    assert lib.qsrt_abi_version() == 2
    assert isinstance(lib.qsrt_last_error(), bytes)

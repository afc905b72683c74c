"""libcfhip.so loads and exports every entry point include/cfhip.h declares (no GPU calls)."""
from __future__ import annotations

import re
from pathlib import Path

from chain_flow_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "cfhip.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(cfh_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert set(declared()) == set(_lib.SIGNATURES), set(declared()) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert _lib.LIB_PATH.exists(), "build libcfhip.so first (python chain-flow_amd/csrc/build.py)"
    assert _lib.missing_symbols() == []


def test_status_strings_without_a_device():
    L = _lib.lib()
    assert L.cfh_version() >= 100
    assert L.cfh_error_string(0) == b"ok"
    assert L.cfh_error_string(2) == b"unsupported shape"

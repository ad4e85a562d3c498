"""The C ABI library loads and exports every entry point include/nnhip.h
declares, and the Python binding binds each of them (no GPU needed: nothing
here calls into the device)."""
import ctypes
import os
import re

import pytest

from gpu_util import ROOT, nnhip

HEADER = os.path.join(ROOT, "include", "nnhip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nnhip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "nnhip_generate_speculative" in names
    assert len(names) >= 30


@pytest.mark.skipif(not os.path.exists(nnhip.LIB_PATH),
                    reason="libnnhip.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(nnhip.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    bound = set(nnhip.SIGNATURES) | {"nnhip_last_error"}
    assert set(declared()) == bound

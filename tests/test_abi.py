"""CPU checks of the C-ABI boundary: the library loads without a GPU and
exports exactly the functions include/uttt_hip.h declares, each with a ctypes
signature in uttt_amd._lib (no compute call is made here)."""
import ctypes
import os
import re

import pytest

from uttt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(uttt_[a-z0-9_]+)\s*\(", src))
    return names


def test_header_declares_functions():
    assert len(declared_functions()) >= 10


def test_signature_table_matches_header():
    assert set(_lib.SIGNATURES) == declared_functions()


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    l = _lib.lib()
    assert l.uttt_abi_version() >= 1
    assert l.uttt_last_error() == b""
    # size queries are pure host arithmetic
    assert l.uttt_row_id_map_workspace_bytes(1, 65536, 16) == 16 * 256 * 4

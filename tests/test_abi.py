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


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_wgrad_pair_split_rule():
    """Split K only where the output tiles fill under half of the 256 CUs: the
    dense 124M write (4 heads x 5 tiles) takes 12 runs of its 24576 tokens;
    the MoE shapes and short segments take none."""
    q = _lib.lib().uttt_grouped_wgrad_pair_workspace_bytes
    I, D = 384, 192
    assert q(4, 1, I, D, 24576) == 12 * 4 * 3 * I * D * 4
    assert q(1, 32, 3072, 1536, 65536) == 0      # 6912 tiles
    assert q(4, 1, 192, 96, 512) == 0            # 8 K steps per segment: one run
    assert q(1, 1, 64, 64, 64 * 8 * 40) == 32 * 3 * 64 * 64 * 4  # capped at 32 runs
    assert q(0, 1, I, D, 24576) == 0


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_inverse_row_map_rule_matches_the_library():
    """routing.src_rows_supported restates uttt_route_tokens_map_src_rows in
    Python (so torch.compile traces the routed read); both are pure host
    rules over (T, E)."""
    from uttt_amd import routing
    q = _lib.lib().uttt_route_tokens_map_src_rows
    for T in (1, 15, 16, 17, 2048, 4080, 4096, 4112, 65536):
        for E in (1, 16, 32, 63, 64, 65, 128):
            assert routing.src_rows_supported(T, E) == bool(q(T, E)), (T, E)
    g = _lib.lib().uttt_grouped_gate_up_gathers
    assert g(4096, 32) == 1 and g(4096, 16) == 1 and g(65536, 16) == 0

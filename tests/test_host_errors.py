"""Host-side contract checks that need no GPU: the product ops refuse CPU
tensors (no fallback path) and the C ABI rejects bad arguments with an error
code and a message instead of launching."""
import os

import pytest
import torch

from uttt_amd import _lib
from uttt_amd.lact_moe_triton import triton_permute as TP

needs_lib = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")


def test_cpu_tensors_are_rejected_not_computed():
    x = torch.randn(1, 8, 4)
    mask = torch.zeros(1, 2, 8, dtype=torch.bool)
    with pytest.raises(RuntimeError, match="GPU only"):
        TP.permute_with_expert_mask(x, mask, None, 1)


@needs_lib
def test_abi_rejects_bad_sizes_without_launch():
    lib = _lib.lib()
    rc = lib.uttt_make_row_id_map(None, 1, 0, 0, 0, 1, 16, 200, None, None, None, 0, None)
    assert rc == -1
    assert b"E=200" in lib.uttt_last_error()
    rc = lib.uttt_make_row_id_map(None, 3, 0, 0, 0, 1, 16, 4, None, None, None, 0, None)
    assert rc == -1 and b"mask element size" in lib.uttt_last_error()
    rc = lib.uttt_permute_fwd(None, 7, 1, 1, 1, None, 1, None, 0, 0, 0, None, 1, None, None)
    assert rc == -1 and b"dtype" in lib.uttt_last_error()


@needs_lib
def test_call_raises_runtime_error_with_message():
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("uttt_make_row_id_map", None, 1, 0, 0, 0, 1, 16, 4, None, None, None, 0, None)


@needs_lib
def test_write_step_rejects_bad_segments_without_launch():
    lib = _lib.lib()
    rc = lib.uttt_write_step(None, None, None, 0, None, None, 1.0, 1, 4, 96, 40, 0, 1,
                             None, None, None, None)
    assert rc == -1 and b"segment 40" in lib.uttt_last_error()
    rc = lib.uttt_write_step(None, None, None, 0, 8, None, 1.0, 1, 4, 96, 96, 0, 1,
                             None, None, None, None)
    assert rc == -1 and b"momentum" in lib.uttt_last_error()
    rc = lib.uttt_write_step(None, None, None, 0, None, None, 1.0, 1, 4, 96, 96, 1, 1,
                             None, None, None, None)
    assert rc == -1 and b"norm_from_fast" in lib.uttt_last_error()

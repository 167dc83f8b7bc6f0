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


@needs_lib
def test_new_entry_points_reject_bad_arguments_without_launch():
    """The decode read, Newton-Schulz, momentum and router entry points check
    sizes, dtypes and pointers before any GPU call (fake, never-dereferenced
    addresses stand in for device pointers where a check comes later)."""
    lib = _lib.lib()
    p = 1 << 20   # an aligned, non-null stand-in address

    def decode(B=1, T=1, D=64, E=8, I=32, mb=1, topk=2, ptr=p, ws_bytes=1 << 30):
        return lib.uttt_moe_decode_read(ptr, B, T, D, ptr, ptr, E, I, ptr, mb, 0, 0, 0, ptr, 0, 0,
                                        0, topk, ptr, ptr, ws_bytes, None)

    for kw, msg in ((dict(E=65), b"E=65 exceeds 64"), (dict(T=65), b"exceed 64"),
                    (dict(D=12), b"multiples of 8"), (dict(D=8192), b"at most"),
                    (dict(mb=2), b"mask element size"), (dict(topk=0), b"topk"),
                    (dict(ptr=None), b"null pointer"), (dict(ws_bytes=16), b"workspace")):
        assert decode(**kw) == -1, kw
        assert msg in lib.uttt_last_error(), (kw, lib.uttt_last_error())
    assert lib.uttt_newton_schulz5(p, 1, 2, 12, 16, 1.0, p, p, 1 << 30, None) == -1
    assert b"multiples of 8" in lib.uttt_last_error()
    assert lib.uttt_newton_schulz5(p, 2, 2, 16, 16, 1.0, p, p, 1 << 30, None) == -1
    assert b"fp32 or bf16" in lib.uttt_last_error()
    assert lib.uttt_momentum_add(p, 2, p, p, 1, 16, p, None) == -1
    assert b"fp32 or bf16" in lib.uttt_last_error()
    rc = lib.uttt_route_tokens(p, 1, p, 0, 1, 4, 64, 8, None, 0, 9, 0, 0, 1.0, 0.0, 1e-6, None,
                               p, p, p, p, p, None, p, 1 << 20, None)
    assert rc == -1 and b"topk" in lib.uttt_last_error()
    rc = lib.uttt_route_tokens(p, 1, p, 0, 1, 4, 64, 8, None, 0, 2, 7, 0, 1.0, 0.0, 1e-6, None,
                               p, p, p, p, p, None, p, 1 << 20, None)
    assert rc == -1 and b"router_type" in lib.uttt_last_error()


def test_new_wrappers_refuse_cpu_tensors():
    from uttt_amd import decode as DEC
    from uttt_amd import fast_weight_write as FWW

    with pytest.raises(RuntimeError, match="GPU only"):
        DEC.moe_decode_read(torch.zeros(1, 1, 8), torch.zeros(1, 2, 16, 8), torch.zeros(1, 2, 8, 8),
                            torch.zeros(1, 2, 1, dtype=torch.bool), torch.zeros(1, 2, 1), 1)
    with pytest.raises(RuntimeError, match="GPU only"):
        FWW.newton_schulz5(torch.zeros(1, 8, 8))


@needs_lib
def test_gemm_rejects_rows_past_2_pow_23_without_launch():
    """The GEMM tile loads keep per-lane 32-bit offsets below 2^31 (bit 31
    marks the K tail), so operand rows of 2^23 or more elements are refused
    before any launch (stand-in addresses are never dereferenced)."""
    lib = _lib.lib()
    p = 1 << 20
    K = 1 << 23
    # grouped_gemm_nt: M rows of K = 2^23 features
    rc = lib.uttt_grouped_gemm_nt(p, p, p, 1, 1, 256, K, 256, p, None)
    assert rc == -1 and b"2^23" in lib.uttt_last_error()
    # grouped_wgrad: R x C output with C = 2^23
    rc = lib.uttt_grouped_wgrad(p, p, p, 1, 1, 256, K, 256, p, 0, None)
    assert rc == -1 and b"2^23" in lib.uttt_last_error()

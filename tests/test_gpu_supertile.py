"""The XCD super-tile order of the token-grouped GEMMs against the oracle.

Grids of 2048 workgroup tiles or more (the batched UPDATE at configs[4], the
Newton-Schulz B X products of the 760M pool) map workgroups to tiles through
the super-tile index math of tn_kernel; smaller grids keep the plain order.
Here the threshold is lowered to one tile (uttt_debug_set_supertile_min_tiles,
a process-wide test hook), so every launch of the parity cases below -- APPLY
forward and backward, UPDATE forward and backward with every pre-pass and
chained product, the kernel-level compat pieces and Newton-Schulz -- takes
that order, with super-tiles that overhang the grid on both axes, and is
checked in full against the same oracle bars as the plain order.
"""
import pytest

from tests import test_gpu_compat_bwd as TC
from tests import test_gpu_grouped as TG
from tests import test_gpu_muon as TM
from uttt_amd import _lib as L

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def supertile_everywhere():
    prev = L.lib().uttt_debug_set_supertile_min_tiles(1)
    try:
        yield
    finally:
        L.lib().uttt_debug_set_supertile_min_tiles(prev)


def test_hook_round_trip():
    lib = L.lib()
    assert lib.uttt_debug_set_supertile_min_tiles(5) == 1
    assert lib.uttt_debug_set_supertile_min_tiles(-1) == 5
    assert lib.uttt_debug_set_supertile_min_tiles(1) == 2048


@pytest.mark.parametrize("name", ["ragged", "slack", "c3_chunk"])
def test_apply_forward_supertile(name):
    TG.test_apply_forward(name)


@pytest.mark.parametrize("name", ["ragged", "slack"])
def test_apply_backward_supertile(name):
    TG.test_apply_backward(name)


@pytest.mark.parametrize("name", ["ragged", "slack", "one_expert", "c3_chunk"])
def test_update_forward_supertile(name):
    import torch
    TG.test_update_forward(name, torch.bfloat16)


@pytest.mark.parametrize("name", ["ragged", "slack", "c3_chunk"])
def test_update_backward_supertile(name):
    import torch
    TG.test_update_backward(name, torch.float32 if name == "slack" else torch.bfloat16)


@pytest.mark.parametrize("name", ["ragged", "slack"])
def test_compat_pieces_supertile(name):
    TG.test_two_mm_swiglu_compat(name)
    TG.test_gemm_transpose_compat(name)
    TG.test_update_stage_compat(name)
    TC.test_four_grouped_gemm(name)
    TC.test_fused_grad_kv(name)


@pytest.mark.parametrize("n,R,C", [(3, 64, 128), (2, 256, 128), (1, 40, 200)])
def test_newton_schulz5_supertile(n, R, C):
    import torch
    TM.test_newton_schulz5_matches_oracle(n, R, C, torch.float32, 1.0)

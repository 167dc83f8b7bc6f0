"""UPDATE stage 2: the two grouped weight-gradient GEMMs.

Drop-in for the reference module uttt_llm/flame/custom_models/uttt_moe/
lact_moe_triton/triton_lact_bwd_grouped_two_mm_grad_fw.py (cited U2:line);
kernel in csrc/grouped_gemm.hip (wgrad_kernel).
"""
from __future__ import annotations

import torch

from . import _grouped


def grouped_two_gemm_fw_bwd_triton(
    DY0_DY2: torch.Tensor,
    K: torch.Tensor,
    Hidden: torch.Tensor,
    V: torch.Tensor,
    group_sizes: torch.Tensor,
):
    """U2:231-312.  DY0_DY2 [B, 2H, N], K [B, N, D], Hidden [B, H, N], V [B, N, D]
    (bf16) -> DW0_W2 [B, E, 2H, D] = DY0_DY2[:, seg] K[seg] and
    DW1 [B, E, D, H] = (Hidden[:, seg] V[seg])^T, bf16."""
    assert DY0_DY2.dtype == torch.bfloat16
    assert K.dtype == torch.bfloat16
    assert Hidden.dtype == torch.bfloat16
    assert V.dtype == torch.bfloat16
    assert group_sizes.dtype in (torch.int32, torch.int64)
    # [B, rows, N] intermediates are turned token-major for the kernel
    return _grouped.wgrad_pair(_grouped.transpose_last2(DY0_DY2), K.contiguous(),
                               _grouped.transpose_last2(Hidden), V.contiguous(), group_sizes)

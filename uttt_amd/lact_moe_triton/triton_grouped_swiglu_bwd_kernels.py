"""APPLY backward's three-GEMM pass (no learning rates).

Drop-in for the reference module uttt_llm/flame/custom_models/uttt_moe/
lact_moe_triton/triton_grouped_swiglu_bwd_kernels.py (cited SB:line).  It is
the UPDATE stage-1 kernels (csrc/grouped_gemm.hip) with lr = 1 and V the
APPLY's output gradient.
"""
from __future__ import annotations

import torch

from . import _grouped


def swiglu_backward_three_bmm_grouped_triton(
    W0_W2: torch.Tensor,
    W1: torch.Tensor,
    X: torch.Tensor,
    V: torch.Tensor,
    group_sizes: torch.Tensor,
):
    """SB:229-320.  V is the APPLY's output gradient [B, N, K].  Returns DY0_DY2
    [B, 2M, N] and Hidden [B, M, N] (bf16) with DY0 = sig(Y0) Y2 DH (1 + Y0
    (1 - sig(Y0))), DY2 = silu(Y0) DH, Hidden = silu(Y0) Y2, Y0 = w0 X^T,
    Y2 = w2 X^T, DH = w1^T V^T."""
    assert W0_W2.dtype == torch.bfloat16 and V.dtype == torch.bfloat16
    return _grouped.update_stage1(W0_W2, W1.contiguous(), X.contiguous(), V.contiguous(),
                                  None, None, None, group_sizes, token_major=False)

"""UPDATE stage 1 (three grouped GEMMs with the lr-scaled SwiGLU' epilogue).

Drop-in for the reference module uttt_llm/flame/custom_models/uttt_moe/
lact_moe_triton/triton_grouped_swiglu_bwd_with_lr_kernels.py (cited U1:line);
kernel in csrc/grouped_gemm.hip (update_s1_kernel).
"""
from __future__ import annotations

import torch

from . import _grouped


def swiglu_backward_three_bmm_grouped_with_lr_triton(
    W0_W2: torch.Tensor,
    W1: torch.Tensor,
    X: torch.Tensor,
    V: torch.Tensor,
    lr0: torch.Tensor,
    lr1: torch.Tensor,
    lr2: torch.Tensor,
    group_sizes: torch.Tensor,
):
    """U1:255-353.  Returns DY0_DY2 [B, 2M, N] and Hidden [B, M, N] (bf16):
    DY0 = lr0 sig(Y0) Y2 DH (1 + Y0 (1 - sig(Y0))), DY2 = lr2 silu(Y0) DH,
    Hidden = lr1 silu(Y0) Y2 with Y0 = w0 X^T, Y2 = w2 X^T, DH = w1^T V^T."""
    assert W0_W2.dtype == torch.bfloat16 and V.dtype == torch.bfloat16, "W0_W2 and V must be bf16"
    assert W0_W2.is_contiguous() and W1.is_contiguous() and X.is_contiguous() and V.is_contiguous()
    assert W0_W2.ndim == 4 and W1.ndim == 4 and X.ndim == 3 and V.ndim == 3
    assert W0_W2.shape[2] % 2 == 0, "2M must be even"
    return _grouped.update_stage1(W0_W2, W1, X, V, lr0, lr1, lr2, group_sizes, token_major=False)

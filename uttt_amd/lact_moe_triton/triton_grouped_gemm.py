"""Grouped GEMMs over expert token segments on gfx950.

Drop-in for the reference module
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/triton_grouped_gemm.py
(cited G:line); kernels in csrc/grouped_gemm.hip (gemm_nt_kernel,
wgrad_kernel, transpose16_kernel).
"""
from __future__ import annotations

import torch

from . import _grouped


def grouped_gemm_transpose_triton(
    W1: torch.Tensor,
    X: torch.Tensor,
    group_sizes: torch.Tensor,
    debug_autotune: bool = False,
) -> torch.Tensor:
    """G:170-243.  Y = (W1 @ X).transpose(1, 2) per expert segment:
    W1 [B, E, M, K] bf16, X [B, K, N] bf16 -> Y [B, N, M] bf16.
    `debug_autotune` exists for signature compatibility (nothing is tuned at
    run time here) and is ignored."""
    assert W1.dtype == torch.bfloat16 and X.dtype == torch.bfloat16
    assert W1.is_contiguous() and X.is_contiguous(), "W1 and X must be contiguous"
    assert W1.device == X.device == group_sizes.device
    B, E, M, K = W1.shape
    Bx, Kx, N = X.shape
    assert Bx == B and Kx == K, "X must be [B, K, N] with matching B,K."
    # the MFMA kernel reads token rows with 16-byte vectors; the token axis of
    # [B, K, N] is contiguous, so the operand is first turned token-major
    return _grouped.gemm_nt(W1, _grouped.transpose_last2(X), group_sizes)


def grouped_gemm_bwd_triton(
    output_grad: torch.Tensor,
    X: torch.Tensor,
    group_sizes: torch.Tensor,
) -> torch.Tensor:
    """G:349-404.  W_grad[b, e] = output_grad[b, :, seg(b,e)] @ X[b, seg(b,e), :]:
    output_grad [B, H, N], X [B, N, D] (bf16) -> [B, E, H, D] bf16."""
    assert output_grad.dtype == torch.bfloat16 and X.dtype == torch.bfloat16
    return _grouped.wgrad(_grouped.transpose_last2(output_grad), X.contiguous(), group_sizes,
                          transposed=False)

"""Grouped gate/up GEMM pair with the SwiGLU epilogue on gfx950.

Drop-in for the reference module
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/triton_grouped_swiglu_kernels.py
(cited S:line); kernels in csrc/grouped_gemm.hip (tn_kernel with the EpiSwiGLU
epilogue; apply_kernel<ApSwiGLU> for the token-major per-layer APPLY).
"""
from __future__ import annotations

import torch

from . import _grouped


def fused_two_mm_swiglu_triton(W0_W2: torch.Tensor, X: torch.Tensor, group_sizes: torch.Tensor):
    """S:273-338.  W0_W2 [B, E, 2M, K] bf16, X [B, N, K] bf16, group_sizes [B, E]
    -> O [B, M, N] bf16 with O[:, :, seg_e] = silu(w0 X_e^T) * (w2 X_e^T).
    Columns past sum(group_sizes) are left unwritten, as in the reference."""
    assert W0_W2.dtype == torch.bfloat16 and X.dtype == torch.bfloat16
    assert W0_W2.is_contiguous() and X.is_contiguous(), "W0_W2 and X must be contiguous"
    B, E, M2, K = W0_W2.shape
    Bx, N, Kx = X.shape
    assert Bx == B and Kx == K, "X must be [B, N, K] with matching B,K."
    return _grouped.gate_up(W0_W2, X, group_sizes, token_major=False)

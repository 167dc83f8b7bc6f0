"""The grouped SwiGLU fast-weight APPLY op on gfx950.

Drop-in for the reference module
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/lact_swiglu_ffn.py
(cited F:line).  Forward: gate/up GEMM pair with the SwiGLU epilogue, then
the down projection; Hidden stays token-major ([B, N, I]) between the two so
both kernels read 16-byte vectors.  Backward: the three-GEMM SwiGLU' pass,
the paired weight-gradient GEMMs and grad_X = W0_W2^T DY, all on the HIP
kernels of csrc/grouped_gemm.hip.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _grouped


class FusedSwiGLUFFNFwd(torch.autograd.Function):
    """F:31-104.  W1 @ [silu(W0 @ X^T) * (W2 @ X^T)] per expert segment."""

    @staticmethod
    @torch.amp.custom_fwd(cast_inputs=torch.bfloat16, device_type="cuda")
    def forward(ctx, W0_W2, W1, X, group_sizes):
        """W0_W2 [B, E, 2I, D], W1 [B, E, D, I], X [B, N, D], group_sizes [B, E]
        -> [B, N, D] bf16."""
        W0_W2, W1, X = W0_W2.contiguous(), W1.contiguous(), X.contiguous()
        hidden_tok = _grouped.gate_up(W0_W2, X, group_sizes, token_major=True)
        output = _grouped.gemm_nt(W1, hidden_tok, group_sizes)
        ctx.save_for_backward(W0_W2, W1, X, group_sizes)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        """F:63-104: (grad_W0_W2, grad_W1, grad_X, None)."""
        W0_W2, W1, X, group_sizes = ctx.saved_tensors
        g = grad_out.contiguous()
        if g.dtype != torch.bfloat16:
            g = g.to(torch.bfloat16)
        dy_tok, hid_tok = _grouped.update_stage1(W0_W2, W1, X, g, None, None, None, group_sizes,
                                                 token_major=True)
        grad_W0_W2, grad_W1 = _grouped.wgrad_pair(dy_tok, X, hid_tok, g, group_sizes)
        grad_X = _grouped.gemm_tn(W0_W2, dy_tok, group_sizes)
        return grad_W0_W2, grad_W1, grad_X, None


def grouped_swiglu_ffn_fwd(W0_W2, W1, X, group_sizes):
    """F:107-108: the APPLY op of uttt_moe (modeling_recurrent_lact.py:329-334)."""
    return FusedSwiGLUFFNFwd.apply(W0_W2, W1, X, group_sizes)

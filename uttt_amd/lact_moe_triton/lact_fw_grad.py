"""The grouped SwiGLU fast-weight UPDATE op on gfx950.

Drop-in for the reference module
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/lact_fw_grad.py
(cited FG:line).  Forward: the three-GEMM pass with the lr-scaled SwiGLU'
epilogue (DY0_DY2 and lr1*Hidden, token-major) followed by the paired
weight-gradient GEMMs over each expert's token segment.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _grouped


class FusedLactSwiGLUFFNBwd(torch.autograd.Function):
    """FG:51-300."""

    @staticmethod
    def forward(ctx, W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes):
        """W0_W2 [B,E,2I,D], W1 [B,E,D,I], K, V [B,N,D] (bf16), lr* [B,N],
        group_sizes [B,E] -> (dW0_W2 [B,E,2I,D], dW1 [B,E,D,I]) bf16
        (FG:54-114; 12*N*I*D FLOP)."""
        group_sizes = _grouped.group_sizes_i32(group_sizes)
        dy_tok, hid_tok = _grouped.update_stage1(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes,
                                                 token_major=True)
        dW0_W2, dW1 = _grouped.wgrad_pair(dy_tok, K, hid_tok, V, group_sizes)
        ctx.save_for_backward(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes)
        return dW0_W2, dW1

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_dw0_dw2, grad_dw1):
        from . import _update_bwd

        W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes = ctx.saved_tensors
        return _update_bwd.fast_weight_grads_backward(
            W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, grad_dw0_dw2, grad_dw1
        )


def grouped_lact_swiglu_ffn_fast_weight_grads(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes):
    """FG:306-309: the UPDATE op of uttt_moe (modeling_recurrent_lact.py:503-512)."""
    return FusedLactSwiGLUFFNBwd.apply(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes)

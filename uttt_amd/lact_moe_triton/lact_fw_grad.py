"""The grouped SwiGLU fast-weight UPDATE op on gfx950.

Drop-in for the reference module
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/lact_fw_grad.py
(cited FG:line).  Forward: the three-GEMM pass with the lr-scaled SwiGLU'
epilogue (DY0_DY2 and lr1*Hidden, token-major) followed by the paired
weight-gradient GEMMs over each expert's token segment.  When a backward
follows, the forward also keeps bf16 Y0 | Y2 and DH, which the reference's
backward recomputes (FG:131-176) and rounds to bf16; the backward reads them.
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
        # with a backward ahead, keep the bf16 Y0 | Y2 and DH it would recompute
        save = any(ctx.needs_input_grad[:7])
        out = _grouped.update_stage1(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes,
                                     token_major=True, save=save)
        dy_tok, hid_tok = out[0], out[1]
        dW0_W2, dW1 = _grouped.wgrad_pair(dy_tok, K, hid_tok, V, group_sizes)
        saved = (out[2], out[3]) if save else ()
        ctx.save_for_backward(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, *saved)
        return dW0_W2, dW1

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_dw0_dw2, grad_dw1):
        from . import _update_bwd

        W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, *saved = ctx.saved_tensors
        return _update_bwd.fast_weight_grads_backward(
            W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, grad_dw0_dw2, grad_dw1, *saved
        )


def grouped_lact_swiglu_ffn_fast_weight_grads(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes):
    """FG:306-309: the UPDATE op of uttt_moe (modeling_recurrent_lact.py:503-512)."""
    return FusedLactSwiGLUFFNBwd.apply(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes)

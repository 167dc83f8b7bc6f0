"""Drop-in for L/triton_pointwise_kernels.py (L =
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton): the second-order
SwiGLU pointwise pass of the UPDATE backward on one gfx950 kernel
(csrc/swiglu_pointwise.hip).  Both reference entry points -- the Triton one
and the torch.compile'd PyTorch one -- map to the same kernel."""
from __future__ import annotations

from . import _grouped


def triton_swiglu_bwd_bwd_fused_cat_inp_out(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2,
                                            grad_hidden_lr1):
    """L/triton_pointwise_kernels.py:240-351.  dh, grad_hidden_lr1 [B, D, L];
    x0_x2, grad_dx0_dx2 [B, 2D, L]; lr0/1/2 [B, L].  Returns (grad_dh,
    grad_x0_x2, grad_lr0, grad_lr1, grad_lr2, dx0_x2, hidden_lr1): element
    outputs in x0_x2's dtype, grad_lr* in the lrs' dtype (fp32 arithmetic,
    the lr sums over D reduced deterministically)."""
    return _grouped.swiglu_bwd_bwd(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1)


def ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2,
                                                 grad_hidden_lr1):
    """L/triton_pointwise_kernels.py:354-436: same computation and outputs."""
    return _grouped.swiglu_bwd_bwd(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1)

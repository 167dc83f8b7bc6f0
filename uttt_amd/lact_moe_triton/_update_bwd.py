"""Backward of the grouped UPDATE op (lact_fw_grad.FusedLactSwiGLUFFNBwd):
one C-ABI call, uttt_grouped_update_bwd, that runs the six-GEMM pass with the
fused second-order SwiGLU pointwise epilogue, the learning-rate gradient
reduction, grad_K / grad_V and the weight gradients (csrc/grouped_gemm.hip).
Reference: uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/lact_fw_grad.py:116-300.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from uttt_amd import _lib as L  # absolute: the package also works mounted in the reference tree
from uttt_amd._ops import traced_op
from . import _grouped


def fast_weight_grads_backward(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, grad_dw0_dw2,
                               grad_dw1, y0_y2_saved=None, dh_saved=None):
    """Returns (grad_W0_W2, grad_W1, grad_K, grad_V, grad_lr0, grad_lr1, grad_lr2, None)
    with the grad_lr* in the lr dtype and the lr tensors' shape.  y0_y2_saved /
    dh_saved: the forward's bf16 (Y0 | Y2) and DH (both or neither)."""
    return _backward(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, grad_dw0_dw2, grad_dw1,
                     y0_y2_saved, dh_saved) + (None,)


def _backward_fake(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, grad_dw0_dw2, grad_dw1,
                   y0_y2_saved, dh_saved):
    B, N, D = K.shape
    return (torch.empty_like(W0_W2), torch.empty_like(W1), K.new_empty((B, N, D)),
            K.new_empty((B, N, D)), torch.empty_like(lr0), torch.empty_like(lr1),
            torch.empty_like(lr2))


@traced_op("grouped_update_bwd", _backward_fake)
def _backward(W0_W2: Tensor, W1: Tensor, K: Tensor, V: Tensor, lr0: Tensor, lr1: Tensor,
              lr2: Tensor, group_sizes: Tensor, grad_dw0_dw2: Optional[Tensor],
              grad_dw1: Optional[Tensor], y0_y2_saved: Optional[Tensor],
              dh_saved: Optional[Tensor]
              ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = K.shape[1]
    dev = K.device
    gs = _grouped.group_sizes_i32(group_sizes)
    L.require_device(W0_W2, W1, K, V, lr0, lr1, lr2, gs, grad_dw0_dw2, grad_dw1)
    gw02 = grad_dw0_dw2 if grad_dw0_dw2 is not None else torch.zeros_like(W0_W2)
    gw1 = grad_dw1 if grad_dw1 is not None else torch.zeros_like(W1)
    gw02 = gw02.to(torch.bfloat16).contiguous()
    gw1 = gw1.to(torch.bfloat16).contiguous()
    lr_shape = lr0.shape
    lrs = [x.reshape(B, N).contiguous() for x in (lr0, lr1, lr2)]
    lr_dtype = lrs[0].dtype
    grad_W0_W2 = torch.empty_like(W0_W2)
    grad_W1 = torch.empty_like(W1)
    grad_K = torch.empty((B, N, D), dtype=torch.bfloat16, device=dev)
    grad_V = torch.empty((B, N, D), dtype=torch.bfloat16, device=dev)
    glr = [torch.empty(lr_shape, dtype=lr_dtype, device=dev) for _ in range(3)]  # B*N each
    ws_bytes = L.lib().uttt_update_bwd_workspace_bytes(B, I, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    L.call(
        "uttt_grouped_update_bwd",
        L.ptr(W0_W2), L.ptr(W1), L.ptr(K), L.ptr(V), L.ptr(lrs[0]), L.ptr(lrs[1]), L.ptr(lrs[2]),
        L.dtype_code(lr_dtype), L.ptr(gs), L.ptr(gw02), L.ptr(gw1), L.ptr(y0_y2_saved),
        L.ptr(dh_saved), B, E, I, D, N,
        L.ptr(grad_W0_W2), L.ptr(grad_W1), L.ptr(grad_K), L.ptr(grad_V),
        L.ptr(glr[0]), L.ptr(glr[1]), L.ptr(glr[2]), L.ptr(ws), ws_bytes, L.stream_of(K),
    )
    return grad_W0_W2, grad_W1, grad_K, grad_V, glr[0], glr[1], glr[2]

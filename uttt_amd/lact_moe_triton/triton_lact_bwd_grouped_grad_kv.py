"""Drop-in for L/triton_lact_bwd_grouped_grad_kv.py (L =
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton): grad_K and grad_V of
the UPDATE backward as two chained-pair grouped products on gfx950."""
from __future__ import annotations

import torch

from . import _grouped


def fused_grouped_grad_kv(G_W0_W2, W0_W2, DY_lr, dY_02, W1, G_W1, dH, H_lr, group_sizes):
    """L/triton_lact_bwd_grouped_grad_kv.py:227-340.  Per expert segment:
      grad_K = G_W0_W2^T DY_lr + W0_W2^T dY_02     -> [B, N, D]
      grad_V = W1 dH + G_W1 H_lr                    -> [B, N, D]
    with DY_lr, dY_02 [B, 2I, N] and dH, H_lr [B, I, N]; both sums accumulate
    in fp32 and round once to bf16."""
    for t in (G_W0_W2, W0_W2, DY_lr, dY_02, W1, G_W1, dH, H_lr):
        assert t.is_contiguous(), "All inputs must be contiguous"
        assert t.dtype == torch.bfloat16, "bf16 expected for all inputs"
    B, E, M2, D = W0_W2.shape
    assert M2 % 2 == 0
    I = M2 // 2
    _, _, N = DY_lr.shape
    assert DY_lr.shape == (B, M2, N) and dY_02.shape == (B, M2, N)
    assert dH.shape == (B, I, N) and H_lr.shape == (B, I, N)
    assert W1.shape == (B, E, D, I) and G_W1.shape == W1.shape
    gs = _grouped.group_sizes_i32(group_sizes)
    t = _grouped.transpose_last2
    grad_K = _grouped.gemm_tn2(G_W0_W2, t(DY_lr), W0_W2, t(dY_02), gs)
    grad_V = _grouped.gemm_nt2(W1, t(dH), G_W1, t(H_lr), gs)
    return grad_K, grad_V

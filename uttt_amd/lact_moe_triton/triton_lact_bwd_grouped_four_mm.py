"""Drop-in for L/triton_lact_bwd_grouped_four_mm.py (L =
uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton): the four grouped
products of the UPDATE backward's recompute, on the gfx950 grouped GEMMs."""
from __future__ import annotations

import torch

from . import _grouped


def grouping_four_grouped_gemm_triton(W0_W2, G_W0_W2, W1, G_W1, K, V, group_sizes):
    """L/triton_lact_bwd_grouped_four_mm.py:300-439.  Per expert segment of
    the token axis:
      Y0_Y2 = W0_W2 K^T, G_Y0_Y2 = G_W0_W2 K^T      -> [B, 2I, N]
      DHidden = W1^T V^T, G_DHidden = G_W1^T V^T    -> [B, I, N]
    bf16 outputs with fp32 accumulation.  Columns past sum(group_sizes) are
    unspecified, as in the reference (torch.empty)."""
    for t in (W0_W2, G_W0_W2, W1, G_W1, K, V):
        assert t.is_contiguous(), "All inputs must be contiguous"
        assert t.dtype == torch.bfloat16, "bf16 expected for all inputs"
    B, E, M2, D = W0_W2.shape
    assert M2 % 2 == 0
    I = M2 // 2
    assert G_W0_W2.shape == W0_W2.shape
    assert W1.shape == (B, E, D, I) and G_W1.shape == W1.shape, "W1 must be [B,E,D,I]"
    Bk, N, Dk = K.shape
    assert (Bk, Dk) == (B, D), "K must be [B,N,D] with D matching"
    assert V.shape == (B, N, D), "V must be [B,N,D] matching"
    gs = _grouped.group_sizes_i32(group_sizes)
    assert gs.shape == (B, E), "group_sizes must be [B,E]"
    t = _grouped.transpose_last2
    Y0_Y2 = t(_grouped.gemm_nt(W0_W2, K, gs))
    G_Y0_Y2 = t(_grouped.gemm_nt(G_W0_W2, K, gs))
    DHidden = t(_grouped.gemm_tn(W1, V, gs))
    G_DHidden = t(_grouped.gemm_tn(G_W1, V, gs))
    return Y0_Y2, G_Y0_Y2, DHidden, G_DHidden

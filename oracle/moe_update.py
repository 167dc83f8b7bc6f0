"""Oracle of the uTTT-MoE update glue (checker only; see oracle/__init__.py).

Reference (M:) uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py
and (RB:) uttt_llm/flame/custom_models/uttt_moe/ref_base.py:

  silu_l2norm_rows   the qkv_silu / v_norm / qk_norm steps of
                     _preprocess_update_inputs (M:641-648) with l2_norm
                     (RB:182-186): x / (|x| + 1e-5) in the tensor's dtype
  head_tokens, lr_tokens   M:132-137 and M:659-664
  writer_grads       _compute_moe_update_grads_grouped (M:484-512): lr cast
                     to bf16, k / v*p / lr permuted by expert, then the
                     grouped UPDATE; dW stored bf16
  aggregate_grads    the aggregate write's input (M:2428-2445): the writers'
                     bf16 dW upcast and summed
  writer_grads_bwd   the backward of writer_grads given upstream dW grads:
                     the UPDATE backward (lact_fw_grad.py:116-300) then the
                     permute's backward (triton_permute.py:1496-1727)

Composed from the pinned pieces of oracle/permute.py and
oracle/fastweight.py, so the rounding points are the reference's.
"""
from __future__ import annotations

import torch

from . import fastweight as FW
from . import permute as P


def silu_l2norm_rows(x: torch.Tensor, silu: bool, l2: bool, rows_of: int | None = None):
    """Rows of `rows_of` elements (default: the last dimension): y = silu(x)
    rounded to x's dtype (F.silu), then y / (|y| + 1e-5) with torch's rounding
    in x's dtype (RB:182-186): |y| is an fp32 sum rounded to the dtype, the
    eps is added in the dtype and the quotient rounded to the dtype."""
    dt = x.dtype
    D = x.shape[-1] if rows_of is None else rows_of
    y = x.reshape(-1, D).float()
    if silu:
        y = (y * torch.sigmoid(y)).to(dt).float()
    if l2:
        nrm = y.double().pow(2).sum(-1, keepdim=True).sqrt().float().to(dt).float()
        den = (nrm + 1e-5).to(dt).float()
        y = y / den
    return y.to(dt).reshape(x.shape)


def head_tokens(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    """b l (h hd) -> b (l h) hd (M:132-137)."""
    B, Lx, HD = x.shape
    return x.reshape(B, Lx, num_heads, HD // num_heads).reshape(B, Lx * num_heads, -1)


def lr_tokens(lr: torch.Tensor, num_heads: int) -> torch.Tensor:
    """[B, L, 3] shared by the heads or [B, L, 3H] -> [B, L*H, 3] (M:659-664)."""
    B, Lx, C = lr.shape
    if C == 3:
        lr_mh = lr.unsqueeze(2).expand(-1, -1, num_heads, -1)
    else:
        lr_mh = lr.reshape(B, Lx, num_heads, 3)
    return lr_mh.reshape(B, Lx * num_heads, 3)


def _permuted(k, v, lr, mask, probs, topk):
    m = mask.to(torch.int32)
    T = k.shape[1]
    rmap = P.make_row_id_map(m)
    num_out = topk * T
    lrs = [lr[:, :, j].contiguous().to(torch.bfloat16) for j in range(3)]
    kp, vp, l0, l1, l2 = P.permute_kv_lrs(k.to(torch.bfloat16), v, *lrs, rmap, probs.float(),
                                          num_out)
    gs = m.sum(-1).to(torch.int32)
    return rmap, num_out, kp, vp, [l0, l1, l2], gs


def writer_grads(k, v, lr, mask, probs, topk, W0_W2, W1):
    """M:484-512 for one writer: k, v [B, T, D] bf16, lr [B, T, 3], mask /
    probs [B, E, T] -> (dW0_W2 [B,E,2I,D], dW1 [B,E,D,I]) bf16."""
    _, _, kp, vp, lrp, gs = _permuted(k, v, lr, mask, probs, topk)
    return FW.fast_weight_grads(W0_W2, W1, kp, vp, *lrp, gs)


def aggregate_grads(writers, W0_W2, W1, topk):
    """M:2428-2445: sum over writers (k, v, lr, mask, probs) of the upcast
    bf16 dW, in fp64."""
    s02, s1 = 0, 0
    for (k, v, lr, mask, probs) in writers:
        d02, d1 = writer_grads(k, v, lr, mask, probs, topk, W0_W2, W1)
        s02 = s02 + d02.double()
        s1 = s1 + d1.double()
    return s02, s1


def writer_grads_bwd(k, v, lr, mask, probs, topk, W0_W2, W1, G_W0_W2, G_W1):
    """Backward of writer_grads: returns (grad_W0_W2, grad_W1, grad_k [B,T,D],
    grad_v [B,T,D], grad_lr [B,T,3] (bf16, the cast lrs' dtype), grad_probs
    [B,E,T] fp32)."""
    rmap, num_out, kp, vp, lrp, gs = _permuted(k, v, lr, mask, probs, topk)
    gw02, gw1, gkp, gvp, g0, g1, g2 = FW.fast_weight_grads_bwd(W0_W2, W1, kp, vp, *lrp, gs,
                                                                G_W0_W2, G_W1)
    T = k.shape[1]
    gk, gv, glr, gp = P.permute_kv_lrs_bwd(gkp, gvp, [g0, g1, g2], rmap, v, probs.float(), T)
    return gw02, gw1, gk, gv, torch.stack(glr, dim=-1), gp

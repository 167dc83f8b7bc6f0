"""Oracle of the router (checker only; see oracle/__init__.py).

Restates create_router_mask_sizes_probs
(uttt_llm/flame/custom_models/uttt_moe/moe_routing.py:7-75, cited R:line) in
fp32 torch on the CPU.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def create_router_mask_sizes_probs(router_logits, topk, alpha=1.0, use_sigmoid=False,
                                   router_type="softmax", combine_mode="selected_prob",
                                   router_scale=0.0, norm_eps=1e-6, routing_bias=None):
    """Returns (mask [B,E,T] bool, group_sizes [B,E] int32, combine [B,E,T],
    balance_probs [B,E,T], lb_loss)."""
    if use_sigmoid:                                                 # R:19-22
        raise NotImplementedError("sigmoid routing")
    E = router_logits.shape[-2]
    logits = router_logits.to(torch.float32)
    if router_type == "softmax":                                    # R:25-27
        sel = logits
        balance = torch.softmax(logits, dim=-2)
    elif router_type == "norm_softmax":                             # R:28-32
        scale = router_scale if router_scale > 0 else math.sqrt(float(E))
        z = logits / logits.norm(dim=-2, keepdim=True).clamp_min(norm_eps)
        sel = z * scale
        balance = torch.softmax(sel, dim=-2)
    elif router_type == "norm_relu":                                # R:33-43
        scale = router_scale if router_scale > 0 else math.sqrt(float(E))
        z = logits / logits.norm(dim=-2, keepdim=True).clamp_min(norm_eps)
        sel = F.relu(z) * scale
        s = sel.sum(dim=-2, keepdim=True)
        balance = torch.where(s > 0, sel / s.clamp_min(1e-9), torch.full_like(sel, 1.0 / E))
    else:
        raise ValueError(router_type)
    scores = sel if routing_bias is None else sel + routing_bias    # R:50
    _, idx = torch.topk(scores, k=topk, dim=-2)                     # R:51
    mask = torch.zeros_like(router_logits, dtype=torch.bool)
    mask.scatter_(-2, idx, True)
    gs = mask.sum(dim=-1).to(torch.int32)                           # R:55
    if combine_mode == "selected_prob":                             # R:57-58
        comb = balance.to(router_logits.dtype) * alpha
    elif combine_mode == "topk_renorm":                             # R:59-62
        s = balance * mask.to(balance.dtype)
        comb = (s / s.sum(dim=-2, keepdim=True).clamp_min(1e-9)).to(router_logits.dtype) * alpha
    else:
        raise ValueError(combine_mode)
    balance = balance.to(router_logits.dtype)
    pm = balance.mean(dim=0).mean(dim=-1)                           # R:71-74
    gm = gs.to(torch.float32).mean(dim=0)
    lb = (pm * (gm / gm.sum())).sum() * E
    return mask, gs, comb, balance, lb


def router_logits(x, router_w):
    """_route_tokens' logits (modeling_recurrent_lact.py:153-157): R x^T with
    fp32 operands; here accumulated in fp64 and returned as fp64 [B, E, T]."""
    R = router_w.double()
    if R.dim() == 2:
        R = R.unsqueeze(0)
    return torch.matmul(R, x.double().transpose(1, 2))

"""Oracle of the router (checker only; see oracle/__init__.py).

Restates, in fp32 torch on the CPU:
  create_router_mask_sizes_probs       uttt_llm/flame/custom_models/uttt_moe/
                                       moe_routing.py:7-75 (cited R:line)
  nvs_create_router_mask_sizes_probs   uttt_nvs/models/routing.py:4-44 (V:)
  LossFree                             the loss-free balancing bias of
                                       uttt_moe/modeling_recurrent_lact.py:1646-1712 (M:)
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


def nvs_create_router_mask_sizes_probs(router_logits, topk, alpha=1.0):
    """uttt_nvs/models/routing.py:4-44 (cited V:).  Returns (mask, group_sizes,
    router_probs, lb_loss)."""
    E = router_logits.shape[-2]
    _, idx = torch.topk(router_logits, k=topk, dim=-2)                 # V:16
    mask = torch.zeros_like(router_logits, dtype=torch.bool)
    mask.scatter_(-2, idx, True)                                       # V:17-18
    gs = mask.sum(dim=-1).to(torch.int32)                              # V:21
    probs = torch.softmax(router_logits.to(torch.float32), dim=-2).to(router_logits.dtype) * alpha
    pm = probs.mean(dim=0).mean(dim=-1)                                # V:38-42
    gm = gs.to(torch.float32).mean(dim=0)
    lb = (pm * (gm / gm.sum())).sum() * E
    return mask, gs, probs, lb


def _gpu_mean(x, dim=None):
    """torch's GPU mean: the fp32 sum times the fp32 reciprocal of the count
    (the sums here are of small integers or are compared with a tolerance)."""
    n = x.numel() if dim is None else x.shape[dim]
    s = x.double().sum() if dim is None else x.double().sum(dim=dim, keepdim=True)
    return (s.float() * torch.tensor(1.0 / n, dtype=torch.float32)).float()


class LossFree:
    """The loss-free balancing state, restating modeling_recurrent_lact.py
    (cited M:) _loss_free_counts_for_scope :1646-1654, _store_loss_free_counts
    :1695-1712 and _maybe_update_loss_free_bias :1662-1693 on fp32 CPU
    tensors, one process (no all-reduce)."""

    def __init__(self, num_layers, num_experts, scope, rate, bias_max, warmup, interval):
        shape = (num_experts,) if scope == "pool" else (num_layers, num_experts)
        self.scope, self.rate, self.bias_max = scope, rate, bias_max
        self.warmup, self.interval = warmup, interval
        self.bias = torch.zeros(shape)
        self.counts = torch.zeros(shape)
        self.steps = 0
        self.num_updates = 0

    def store(self, apply_freqs, update_freqs):
        c = apply_freqs.float().sum(dim=1) + update_freqs.float().sum(dim=1)   # M:1651
        if self.scope == "pool":
            c = c.sum(dim=0)                                                    # M:1652-1653
        self.counts = self.counts + c                                           # M:1711
        self.steps += 1                                                         # M:1712

    def maybe_update(self):
        if self.counts.sum() <= 0:                                              # M:1667-1668
            return
        if self.steps <= self.warmup:                                           # M:1670-1672
            self.counts = torch.zeros_like(self.counts)
            return
        if (self.steps - self.warmup) % self.interval != 0:                     # M:1673-1678
            return
        dim = None if self.scope == "pool" else -1
        target = _gpu_mean(self.counts, dim)                                    # M:1681
        step = torch.tensor(self.rate, dtype=torch.float32) * torch.sign(target - self.counts)
        self.bias = self.bias + step                                            # M:1682
        self.bias = self.bias - _gpu_mean(self.bias, dim)                       # M:1683-1686
        if self.bias_max >= 0:                                                  # M:1687-1691
            self.bias = self.bias.clamp(min=-self.bias_max, max=self.bias_max)
        self.counts = torch.zeros_like(self.counts)                             # M:1692
        self.num_updates += 1                                                   # M:1693

"""The NVS block's router selection on the kernels of csrc/router.hip.

create_router_mask_sizes_probs: same signature, outputs and errors as
uttt_nvs/models/routing.py:4-44 (the module the NVS block imports as
`.routing`): top-k over the raw logits (no selection bias), router_probs =
softmax over the experts in fp32, cast to the logits' dtype, times alpha
(not masked), and the load-balancing loss over those probabilities.  That is
the uTTT-MoE router (uttt_amd.routing) with router_type "softmax" and
combine_mode "selected_prob"; the loss differs from it only by alpha, so for
alpha != 1 it is recomputed from the returned probabilities with the
reference's own expression (three small reductions on the GPU).
"""
from __future__ import annotations

import torch

from . import routing


def create_router_mask_sizes_probs(router_logits, topk, alpha=1.0, use_sigmoid=False):
    """router_logits [B, E, L] -> (router_mask bool [B,E,L], group_sizes int32
    [B,E], router_probs [B,E,L] in router_logits' dtype, lb_loss fp32)."""
    if use_sigmoid:
        raise AssertionError("Please do not use sigmoid now; the average is not correct.")
    mask, gs, probs, _, lb = routing.create_router_mask_sizes_probs(
        router_logits, topk, alpha=alpha, router_type="softmax", combine_mode="selected_prob")
    if float(alpha) != 1.0:
        E = router_logits.shape[-2]
        pm = probs.mean(dim=0).mean(dim=-1)
        gm = gs.to(torch.float32).mean(dim=0)
        lb = (pm * (gm / gm.sum())).sum() * E
    return mask, gs, probs, lb

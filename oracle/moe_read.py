"""Oracle of the routed uTTT-MoE read (checker only; see oracle/__init__.py).

The reference's read after routing, uttt_llm/flame/custom_models/uttt_moe/
modeling_recurrent_lact.py:330-349 (M:): permute the tokens by expert,
grouped SwiGLU apply on the permuted rows, gate-weighted unpermute.  It is
composed here from the oracle's own pinned pieces (oracle/permute.py for the
row map, permute and unpermute; oracle/fastweight.py for the grouped apply),
so its rounding points are the reference's: the hidden and each expert's down
output are stored bf16, the merge accumulates fp32 fma in slot order.

`apply_moe_direct` restates the same read per token without the permuted
buffer (out[t] = sum over the token's experts of p * bf16(W1 bf16(h))), the
check that the composition indexes rows, experts and gates correctly.
"""
from __future__ import annotations

import torch

from . import fastweight as FW
from . import permute as P


def apply_moe_grouped(x, W0_W2, W1, expert_mask, probs, topk, fast=False):
    """M:330-349.  x [B, T, D] bf16, W0_W2 [B, E, 2I, D], W1 [B, E, D, I]
    (bf16), expert_mask [B, E, T], probs [B, E, T] (fp32 combine weights)
    -> out [B, T, D] bf16.  fast=True accumulates the products in fp32 (the
    CPU baseline) instead of the parity mode's fp64."""
    B, T, D = x.shape
    m = expert_mask.to(torch.int32)
    rmap = P.make_row_id_map(m)
    num_out = max(topk * T, int(m.sum(dim=(1, 2)).max().item()) if T else 0)
    xp, _ = P.permute(x.to(torch.bfloat16), rmap, probs, num_out)
    gs = m.sum(dim=-1).to(torch.int32)
    if fast:
        with FW.fp32_accumulate():
            y = FW.swiglu_ffn_fwd(W0_W2, W1, xp, gs)
    else:
        y = FW.swiglu_ffn_fwd(W0_W2, W1, xp, gs)
    return P.unpermute(y, rmap, probs.float(), T)


def apply_moe_direct(x, W0_W2, W1, expert_mask, probs):
    """The same read per token: experts in descending order (the unpermute's
    slot order), fp32 fma of the gate with the expert's bf16 output."""
    B, T, D = x.shape
    E, I = W0_W2.shape[1], W0_W2.shape[2] // 2
    out = torch.zeros(B, T, D, dtype=torch.bfloat16)
    for b in range(B):
        for t in range(T):
            acc = torch.zeros(D, dtype=torch.float32)
            xt = x[b, t].double()
            for e in reversed(range(E)):
                if not bool(expert_mask[b, e, t]):
                    continue
                w = W0_W2[b, e].double()
                y0 = (w[:I] @ xt).float().double()
                y2 = (w[I:] @ xt).float().double()
                h = (y2 * (y0 * torch.sigmoid(y0))).to(torch.bfloat16)
                y = (W1[b, e].double() @ h.double()).to(torch.bfloat16).double()
                p = float(probs[b, e, t].float())
                acc = (acc.double() + y * p).float()
            out[b, t] = acc.to(torch.bfloat16)
    return out

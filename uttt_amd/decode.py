"""uTTT-MoE fast-weight read for a few tokens per sequence (generation).

During decoding each sequence feeds one (or a few) new tokens through every
layer, so the routed read of modeling_recurrent_lact.py:296-349 (route ->
permute -> grouped SwiGLU apply -> gate-weighted unpermute; M:) gives every
selected expert one row.  `moe_decode_read` runs the read after routing as
two grouped GEMV kernels (csrc/decode_read.hip) that stream the selected
experts' weights once, straight from the router's mask and combine weights:
no row map, permuted copy or unpermute launch.  Rounding points are the
reference's: bf16 hidden, bf16 expert outputs, fp32 fma merge in slot order.

`apply_moe_fast_weights_decode` is the whole M:296-349 read (the fused router
of uttt_amd.routing, then `moe_decode_read`) for T <= 64 tokens per batch;
longer inputs belong on the grouped apply.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .routing import route_tokens

MAX_TOKENS = 64


def moe_decode_read(x, w0_w2, w1, expert_mask, router_probs, topk):
    """x [B, T, D]; w0_w2 [B, E, 2I, D], w1 [B, E, D, I] (bf16);
    expert_mask [B, E, T] (bool / uint8 / int32, any strides); router_probs
    [B, E, T] combine weights -> out [B, T, D] bf16 (M:330-349)."""
    L.require_device(x, w0_w2, w1, expert_mask, router_probs)
    assert x.dim() == 3 and w0_w2.dim() == 4 and w1.dim() == 4, "x [B,T,D], weights [B,E,rows,cols]"
    B, T, D = x.shape
    _, E, I2, D2 = w0_w2.shape
    I = I2 // 2
    assert w0_w2.shape[0] == B and D2 == D and I2 == 2 * I, "w0_w2 must be [B, E, 2I, D]"
    assert tuple(w1.shape) == (B, E, D, I), "w1 must be [B, E, D, I]"
    assert tuple(expert_mask.shape) == (B, E, T) and tuple(router_probs.shape) == (B, E, T)
    assert T <= MAX_TOKENS, f"the decode read takes at most {MAX_TOKENS} tokens per batch"
    x = x.to(torch.bfloat16).contiguous()
    w0_w2 = w0_w2.to(torch.bfloat16).contiguous()
    w1 = w1.to(torch.bfloat16).contiguous()
    m = expert_mask
    if m.dtype == torch.bool:
        m = m.view(torch.uint8)
    elif m.dtype not in (torch.uint8, torch.int32):
        m = m.to(torch.int32)
    p = router_probs if router_probs.dtype == torch.float32 else router_probs.float()
    out = torch.empty((B, T, D), dtype=torch.bfloat16, device=x.device)
    nbytes = L.lib().uttt_moe_decode_read_workspace_bytes(B, T, E, I)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    L.call("uttt_moe_decode_read", L.ptr(x), B, T, D, L.ptr(w0_w2), L.ptr(w1), E, I, L.ptr(m),
           m.element_size(), m.stride(0), m.stride(1), m.stride(2), L.ptr(p), p.stride(0),
           p.stride(1), p.stride(2), int(topk), L.ptr(out), L.ptr(ws), nbytes, L.stream_of(x))
    return out


def apply_moe_fast_weights_decode(x, w0, w1, w2, router_proj_weights, topk, *,
                                  routing_bias=None, precomputed_w0_w2=None, **router_kw):
    """FastWeightMLPSubNN._apply_moe_fast_weights_grouped (M:296-349) for
    T <= 64 tokens per batch: x [B, T, D], w0 / w2 [B, E, I, D], w1
    [B, E, D, I]; router keywords as uttt_amd.routing.route_tokens.  Returns
    (out [B, T, D] in x's dtype, (expert_mask, group_sizes, router_probs,
    balance_probs))."""
    w0_w2 = precomputed_w0_w2 if precomputed_w0_w2 is not None else torch.cat([w0, w2], dim=2)
    routed = route_tokens(x, router_proj_weights, topk, routing_bias=routing_bias, **router_kw)
    mask, _, probs, _ = routed
    out = moe_decode_read(x, w0_w2, w1, mask, probs, topk)
    return out.to(x.dtype), routed

"""MoE router on the gfx950 kernels of csrc/router.hip.

  create_router_mask_sizes_probs  same signature, outputs and errors as
      uttt_llm/flame/custom_models/uttt_moe/moe_routing.py:7-75
  route_tokens                    FastWeightMLPSubNN._route_tokens,
      uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:147-169:
      fp32 logits R x^T (D sliced across workgroups when the tokens are few),
      then the selection and two small deterministic reductions

Outputs are freshly allocated on the inputs' device.  Top-k keeps the lower
expert index among exactly equal routing scores (torch.topk leaves that
order unspecified).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib as L
from ._ops import none_if_empty, traced_op

ROUTER_TYPES = {"softmax": 0, "norm_softmax": 1, "norm_relu": 2}
COMBINE_MODES = {"selected_prob": 0, "topk_renorm": 1}


def _check_modes(use_sigmoid, router_type, combine_mode):
    if use_sigmoid:
        raise NotImplementedError("Sigmoid routing is not implemented for ttt_dense_base_moe.")
    if router_type not in ROUTER_TYPES:
        raise ValueError("`router_type` must be 'softmax', 'norm_softmax', or 'norm_relu', "
                         f"got {router_type!r}.")
    if combine_mode not in COMBINE_MODES:
        raise ValueError("`combine_mode` must be 'selected_prob' or 'topk_renorm', "
                         f"got {combine_mode!r}.")


def _bias_arg(routing_bias, B, E, device):
    """A selection bias broadcastable to [B, E, 1] as a contiguous fp32 [Bb, E]
    tensor and its batch stride (0 when shared)."""
    if routing_bias is None:
        return None, 0
    rb = routing_bias.to(device=device, dtype=torch.float32)
    if rb.dim() == 3:
        assert rb.shape[2] == 1 and rb.shape[1] == E, "routing_bias must broadcast to [B, E, 1]"
        rb = rb[:, :, 0]
    elif rb.dim() == 2:
        assert rb.shape == (E, 1), "routing_bias must broadcast to [B, E, 1]"
        rb = rb.reshape(1, E)
    else:
        assert rb.shape == (E,), "routing_bias must broadcast to [B, E, 1]"
        rb = rb.reshape(1, E)
    assert rb.shape[0] in (1, B), "routing_bias batch dimension must be 1 or B"
    rb = rb.contiguous()
    return rb, (E if rb.shape[0] > 1 else 0)


def _outputs(B, E, T, D, device):
    mask = torch.empty((B, E, T), dtype=torch.bool, device=device)
    gs = torch.empty((B, E), dtype=torch.int32, device=device)
    comb = torch.empty((B, E, T), dtype=torch.float32, device=device)
    bal = torch.empty((B, E, T), dtype=torch.float32, device=device)
    lb = torch.empty((), dtype=torch.float32, device=device)
    nbytes = L.lib().uttt_router_workspace_bytes(B, T, E, D)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    return mask, gs, comb, bal, lb, ws, nbytes


def create_router_mask_sizes_probs(router_logits, topk, alpha=1.0, use_sigmoid=False,
                                   router_type="softmax", combine_mode="selected_prob",
                                   router_scale=0.0, norm_eps=1e-6, routing_bias=None):
    """router_logits [B, E, T] (any strides) -> (router_mask bool [B,E,T],
    group_sizes int32 [B,E], combine_weights [B,E,T], balance_probs [B,E,T],
    lb_loss); combine and balance in router_logits' dtype."""
    _check_modes(use_sigmoid, router_type, combine_mode)
    return _select(router_logits, int(topk), float(alpha), router_type, combine_mode,
                   float(router_scale), float(norm_eps), routing_bias)


def _select_fake(router_logits, topk, alpha, router_type, combine_mode, router_scale, norm_eps,
                 routing_bias):
    B, E, T = router_logits.shape
    dt = router_logits.dtype
    e = router_logits.new_empty
    return (e((B, E, T), dtype=torch.bool), e((B, E), dtype=torch.int32), e((B, E, T), dtype=dt),
            e((B, E, T), dtype=dt), e((), dtype=torch.float32))


@traced_op("router_select", _select_fake)
def _select(router_logits: Tensor, topk: int, alpha: float, router_type: str, combine_mode: str,
            router_scale: float, norm_eps: float, routing_bias: Optional[Tensor]
            ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    L.require_device(router_logits)
    assert router_logits.dim() == 3, "router_logits must be [B, E, T]"
    B, E, T = router_logits.shape
    logits = router_logits if router_logits.dtype == torch.float32 else router_logits.float()
    bias, bias_sb = _bias_arg(routing_bias, B, E, logits.device)
    mask, gs, comb, bal, lb, ws, nbytes = _outputs(B, E, T, 0, logits.device)
    L.call("uttt_router_select", L.ptr(logits), logits.stride(0), logits.stride(1),
           logits.stride(2), L.ptr(bias), bias_sb, B, E, T, int(topk), ROUTER_TYPES[router_type],
           COMBINE_MODES[combine_mode], float(alpha), float(router_scale), float(norm_eps),
           L.ptr(mask), L.ptr(gs), L.ptr(comb), L.ptr(bal), L.ptr(lb), None, L.ptr(ws), nbytes,
           L.stream_of(logits))
    if router_logits.dtype != torch.float32:
        comb, bal = comb.to(router_logits.dtype), bal.to(router_logits.dtype)
    return mask, gs, comb, bal, lb


def route_tokens(x, router_proj_weights, topk, alpha=1.0, use_sigmoid=False,
                 router_type="softmax", combine_mode="selected_prob", router_scale=0.0,
                 norm_eps=1e-6, routing_bias=None, return_logits=False):
    """x [B, T, D] (bf16 / fp16 / fp32), router_proj_weights [E, D] or [B, E, D]
    -> (expert_mask, group_sizes, router_probs, balance_probs) as _route_tokens
    returns them (router_probs = the combine weights), plus the fp32 logits
    [B, E, T] when return_logits."""
    _check_modes(use_sigmoid, router_type, combine_mode)
    out = _route(x, router_proj_weights, int(topk), float(alpha), router_type, combine_mode,
                 float(router_scale), float(norm_eps), routing_bias, bool(return_logits))
    return out[:5] if return_logits else out[:4]


def route_tokens_lb(x, router_proj_weights, topk, alpha=1.0, use_sigmoid=False,
                    router_type="softmax", combine_mode="selected_prob", router_scale=0.0,
                    norm_eps=1e-6, routing_bias=None):
    """route_tokens plus the balance sums over the tokens [B, E] fp32 (the
    first half of _make_lb_info, M:171-176), added by the router's own
    reductions in a fixed order: (expert_mask, group_sizes, router_probs,
    balance_probs, balance_sums)."""
    _check_modes(use_sigmoid, router_type, combine_mode)
    out = _route(x, router_proj_weights, int(topk), float(alpha), router_type, combine_mode,
                 float(router_scale), float(norm_eps), routing_bias, False)
    return out[:4] + (out[5],)


def route_tokens_map(x, router_proj_weights, topk, alpha=1.0, use_sigmoid=False,
                     router_type="softmax", combine_mode="selected_prob", router_scale=0.0,
                     norm_eps=1e-6, routing_bias=None, with_src_rows=False):
    """route_tokens_lb followed by make_row_id_map of its mask, as the routed
    read calls them (M:296-349), in one library call (two launches where the
    row map's one-launch kernel fits: it also adds the router's balance
    partials): (expert_mask, group_sizes, router_probs, balance_probs,
    balance_sums, row_id_map [B, T, 2E+1] int32).  with_src_rows (only where
    src_rows_supported(T, E)): also the inverse map src_rows [B, T*topk] int32,
    the token routed to each permuted row, for the gathered gate/up."""
    _check_modes(use_sigmoid, router_type, combine_mode)
    out = _route_map(x, router_proj_weights, int(topk), float(alpha), router_type, combine_mode,
                     float(router_scale), float(norm_eps), routing_bias, bool(with_src_rows))
    return out if with_src_rows else out[:6]


def src_rows_supported(T: int, E: int) -> bool:
    """Whether route_tokens_map can return the inverse row map at (T, E): the
    one-launch row map's sizes (T a multiple of 16 up to 4096, E up to 64),
    the rule uttt_route_tokens_map_src_rows states (pure Python, so that
    torch.compile traces the routed read without calling the library)."""
    return 1 <= T <= 4096 and T % 16 == 0 and 1 <= E <= 64


def _route_fake(x, router_proj_weights, topk, alpha, router_type, combine_mode, router_scale,
                norm_eps, routing_bias, return_logits):
    B, T, _ = x.shape
    E = router_proj_weights.shape[-2]
    e = x.new_empty
    return (e((B, E, T), dtype=torch.bool), e((B, E), dtype=torch.int32),
            e((B, E, T), dtype=torch.float32), e((B, E, T), dtype=torch.float32),
            e((B, E, T) if return_logits else (0,), dtype=torch.float32),
            e((B, E), dtype=torch.float32))


@traced_op("route_tokens", _route_fake)
def _route(x: Tensor, router_proj_weights: Tensor, topk: int, alpha: float, router_type: str,
           combine_mode: str, router_scale: float, norm_eps: float,
           routing_bias: Optional[Tensor], return_logits: bool
           ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    L.require_device(x, router_proj_weights)
    assert x.dim() == 3, "x must be [B, T, D]"
    B, T, D = x.shape
    x = x.contiguous()
    R = router_proj_weights.to(torch.float32).contiguous()
    if R.dim() == 2:
        E = R.shape[0]
        w_sb = 0
    else:
        assert R.dim() == 3 and R.shape[0] in (1, B), "router weights must be [E,D] or [B,E,D]"
        E = R.shape[1]
        w_sb = E * D if R.shape[0] > 1 else 0
    assert R.shape[-1] == D, "router weights must have x's last dimension"
    bias, bias_sb = _bias_arg(routing_bias, B, E, x.device)
    mask, gs, comb, bal, _, ws, nbytes = _outputs(B, E, T, D, x.device)
    logits = torch.empty((B, E, T) if return_logits else (0,), dtype=torch.float32,
                         device=x.device)
    bal_sum = torch.empty((B, E), dtype=torch.float32, device=x.device)
    # no lb_loss here (_route_tokens returns none): its kernel is skipped
    L.call("uttt_route_tokens", L.ptr(x), L.dtype_code(x.dtype), L.ptr(R), w_sb, B, T, D, E,
           L.ptr(bias), bias_sb, int(topk), ROUTER_TYPES[router_type],
           COMBINE_MODES[combine_mode], float(alpha), float(router_scale), float(norm_eps),
           L.ptr(logits) if return_logits else None, L.ptr(mask), L.ptr(gs), L.ptr(comb),
           L.ptr(bal), None, L.ptr(bal_sum), L.ptr(ws), nbytes, L.stream_of(x))
    return mask, gs, comb, bal, logits, bal_sum


def _route_map_fake(x, router_proj_weights, topk, alpha, router_type, combine_mode, router_scale,
                    norm_eps, routing_bias, with_src_rows):
    B, T, _ = x.shape
    E = router_proj_weights.shape[-2]
    e = x.new_empty
    return (e((B, E, T), dtype=torch.bool), e((B, E), dtype=torch.int32),
            e((B, E, T), dtype=torch.float32), e((B, E, T), dtype=torch.float32),
            e((B, E), dtype=torch.float32), e((B, T, 2 * E + 1), dtype=torch.int32),
            e((B, T * topk) if with_src_rows else (0,), dtype=torch.int32))


@traced_op("route_tokens_map", _route_map_fake)
def _route_map(x: Tensor, router_proj_weights: Tensor, topk: int, alpha: float, router_type: str,
               combine_mode: str, router_scale: float, norm_eps: float,
               routing_bias: Optional[Tensor], with_src_rows: bool
               ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    L.require_device(x, router_proj_weights)
    assert x.dim() == 3, "x must be [B, T, D]"
    B, T, D = x.shape
    x = x.contiguous()
    R = router_proj_weights.to(torch.float32).contiguous()
    if R.dim() == 2:
        E = R.shape[0]
        w_sb = 0
    else:
        assert R.dim() == 3 and R.shape[0] in (1, B), "router weights must be [E,D] or [B,E,D]"
        E = R.shape[1]
        w_sb = E * D if R.shape[0] > 1 else 0
    assert R.shape[-1] == D, "router weights must have x's last dimension"
    bias, bias_sb = _bias_arg(routing_bias, B, E, x.device)
    dev = x.device
    mask = torch.empty((B, E, T), dtype=torch.bool, device=dev)
    gs = torch.empty((B, E), dtype=torch.int32, device=dev)
    comb = torch.empty((B, E, T), dtype=torch.float32, device=dev)
    bal = torch.empty((B, E, T), dtype=torch.float32, device=dev)
    bal_sum = torch.empty((B, E), dtype=torch.float32, device=dev)
    rmap = torch.empty((B, T, 2 * E + 1), dtype=torch.int32, device=dev)
    src = torch.empty((B, T * topk) if with_src_rows else (0,), dtype=torch.int32, device=dev)
    nbytes = L.lib().uttt_route_tokens_map_workspace_bytes(B, max(T, 1), E, D)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    L.call("uttt_route_tokens_map", L.ptr(x), L.dtype_code(x.dtype), L.ptr(R), w_sb, B, T, D, E,
           L.ptr(bias), bias_sb, int(topk), ROUTER_TYPES[router_type],
           COMBINE_MODES[combine_mode], float(alpha), float(router_scale), float(norm_eps),
           L.ptr(mask), L.ptr(gs), L.ptr(comb), L.ptr(bal), L.ptr(bal_sum), L.ptr(rmap),
           L.ptr(src) if with_src_rows else None, L.ptr(ws), nbytes, L.stream_of(x))
    return mask, gs, comb, bal, bal_sum, rmap, src

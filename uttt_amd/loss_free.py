"""Loss-free load balancing of the MoE router (the selection bias the router
adds to its scores before top-k) on the kernels of csrc/loss_free.hip.

`LossFreeBalancer` holds the state the reference keeps as model buffers and
offers the reference's methods under the same names without the leading
underscore (uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py):

  loss_free_enabled            _loss_free_enabled        :1630-1635
  get_router_bias              _get_router_bias          :1637-1644
  store_loss_free_counts       _store_loss_free_counts   :1695-1712
  maybe_update_loss_free_bias  _maybe_update_loss_free_bias :1662-1693

The configuration fields (memory_lb_mode, memory_lb_scope, ...) become
constructor arguments with the reference's defaults and checks
(configuration_recurrent_lact.py:24-29, 111-122).  Buffers: `bias` and
`pending_counts` fp32 [L, E] (scope "layer") or [E] (scope "pool"), `steps`
and `num_updates` int64 scalars, all on the GPU.

One GPU: with torch.distributed initialised over several ranks the counts of
one call are summed across ranks (all_reduce) before they are added, as the
reference's _sync_loss_free_counts does.
"""
from __future__ import annotations

import torch

from . import _lib as L

_CLEAR, _STEP = 1, 2


class LossFreeBalancer:
    def __init__(self, num_layers: int, num_experts: int, *, lb_mode: str = "loss",
                 lb_scope: str = "layer", update_rate: float = 1e-4, bias_max: float = 2.0,
                 warmup_steps: int = 0, update_interval: int = 1, device="cuda"):
        if lb_scope not in {"layer", "pool"}:
            raise ValueError("`memory_lb_scope` must be 'layer' or 'pool'.")
        if lb_mode not in {"loss", "loss_free", "none"}:
            raise ValueError("`memory_lb_mode` must be 'loss', 'loss_free', or 'none'.")
        if update_rate < 0:
            raise ValueError("`memory_loss_free_update_rate` must be non-negative.")
        if bias_max < 0:
            raise ValueError("`memory_loss_free_bias_max` must be non-negative.")
        if warmup_steps < 0:
            raise ValueError("`memory_loss_free_warmup_steps` must be non-negative.")
        if update_interval < 1:
            raise ValueError("`memory_loss_free_update_interval` must be >= 1.")
        self.num_layers, self.num_experts = int(num_layers), int(num_experts)
        self.lb_mode, self.lb_scope = lb_mode, lb_scope
        self.update_rate, self.bias_max = float(update_rate), float(bias_max)
        self.warmup_steps, self.update_interval = int(warmup_steps), int(update_interval)
        self.training = True
        shape = (self.num_experts,) if lb_scope == "pool" else (self.num_layers, self.num_experts)
        self.bias = torch.zeros(shape, dtype=torch.float32, device=device)
        self.pending_counts = torch.zeros(shape, dtype=torch.float32, device=device)
        self.steps = torch.zeros((), dtype=torch.long, device=device)
        self.num_updates = torch.zeros((), dtype=torch.long, device=device)
        L.require_device(self.bias)

    def loss_free_enabled(self) -> bool:
        return self.lb_mode == "loss_free" and self.update_rate > 0 and self.num_experts > 1

    def get_router_bias(self, layer_idx: int):
        """The routing_bias of layer `layer_idx` as [1, E, 1], or None."""
        if not self.loss_free_enabled():
            return None
        bias = self.bias if self.lb_scope == "pool" else self.bias[layer_idx]
        return bias.view(1, self.num_experts, 1)

    def store_loss_free_counts(self, apply_accum_freqs, update_accum_freqs) -> None:
        """apply_accum_freqs, update_accum_freqs: fp32 [L, B, E] per-layer row
        counts of the read and the write passes."""
        if not self.training or not self.loss_free_enabled():
            return
        a, u = apply_accum_freqs, update_accum_freqs
        L.require_device(a, u)
        assert a.dim() == 3 and a.shape == u.shape, "accumulated frequencies must be [L, B, E]"
        assert a.shape[0] == self.num_layers and a.shape[2] == self.num_experts
        a = a.to(torch.float32).contiguous()
        u = u.to(torch.float32).contiguous()
        nl, b, e = a.shape
        pool = int(self.lb_scope == "pool")
        dist = torch.distributed
        if dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1:
            part = torch.zeros_like(self.pending_counts)
            L.call("uttt_loss_free_store_counts", L.ptr(a), L.ptr(u), nl, b, e, pool, L.ptr(part),
                   L.ptr(self.steps), L.stream_of(a))
            dist.all_reduce(part, op=dist.ReduceOp.SUM)
            self.pending_counts.add_(part)
            return
        L.call("uttt_loss_free_store_counts", L.ptr(a), L.ptr(u), nl, b, e, pool,
               L.ptr(self.pending_counts), L.ptr(self.steps), L.stream_of(a))

    def maybe_update_loss_free_bias(self) -> None:
        """One bias step per `update_interval` stored passes after the warm-up
        (the warm-up passes' counts are dropped).  Reads the step counter on
        the host, as the reference does."""
        if not self.training or not self.loss_free_enabled():
            return
        steps = int(self.steps.item())
        if steps <= self.warmup_steps:
            mode = _CLEAR
        elif (steps - self.warmup_steps) % self.update_interval != 0:
            return
        else:
            mode = _STEP
        rows = 1 if self.lb_scope == "pool" else self.num_layers
        L.call("uttt_loss_free_bias_step", L.ptr(self.bias), L.ptr(self.pending_counts), rows,
               self.num_experts, mode, self.update_rate, self.bias_max, L.ptr(self.num_updates),
               L.stream_of(self.bias))

    def state_dict(self):
        """The reference's persistent buffers (pending counts are not)."""
        return {"memory_loss_free_bias": self.bias, "memory_loss_free_steps": self.steps,
                "memory_loss_free_num_updates": self.num_updates}

    def load_state_dict(self, sd):
        self.bias.copy_(sd["memory_loss_free_bias"])
        self.steps.copy_(sd["memory_loss_free_steps"])
        self.num_updates.copy_(sd["memory_loss_free_num_updates"])

"""uTTT-MoE caller glue on the gfx950 ops: the routed fast-weight read, one
writer's fast-weight gradients, and the gradients of all writers of a chunk
summed in one grouped call (the aggregate write's input).

Reference (cited M:line):
uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py
  reshape_head_tokens / merge_head_tokens   M:132-144
  route, route_writers                      M:147-169 (_route_tokens; route_writers:
                                            all writers of a chunk in one launch)
  apply_moe_fast_weights_grouped            M:296-349
  preprocess_update_inputs                  M:630-665 (silu, v norm, per-head k norm, rotary)
  preprocess_read_query                     M:588-601 (the read's q path)
  rows_preprocess, Rope                     l2_norm / rms_norm of ref_base.py:181-195 (+ silu,
                                            + the rotary of ref_base.py:342-355, rotary.py)
  moe_update_grads_packed /
  compute_moe_update_grads_grouped          M:453-518
  aggregate_moe_update_grads                M:2381-2546 (the writers' raw
                                            gradients summed at M:2444-2445)

Every kernel call goes through the drop-in ops of uttt_amd.lact_moe_triton
(autograd included), so gradients flow back to k, v, lr and the router
probabilities as in the reference.  There is no CPU path.

The aggregate update concatenates the writers' tokens and runs ONE grouped
UPDATE over them: each expert's segment then holds every writer's rows, and
the weight-gradient GEMM returns sum_l dW_l accumulated in fp32 and rounded
to bf16 once, where the reference rounds each writer's dW_l to bf16 and sums
the upcast terms in the master dtype.  Both are the same sum; the batched
form is one MFMA-bound call instead of L HBM-bound ones.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib as L
from .lact_moe_triton import _grouped
from .lact_moe_triton.lact_fw_grad import grouped_lact_swiglu_ffn_fast_weight_grads
from .lact_moe_triton.lact_swiglu_ffn import grouped_swiglu_ffn_fwd
from .lact_moe_triton.triton_permute import (permute_kv_and_lrs, permute_with_expert_mask,
                                             unpermute_and_merge_with_probs)
from .routing import route_tokens, route_tokens_map, src_rows_supported


@dataclass(frozen=True)
class RouterConfig:
    """The router attributes _route_tokens reads (M:158-168)."""

    topk: int
    alpha: float = 1.0
    use_sigmoid: bool = False
    router_type: str = "softmax"
    combine_mode: str = "selected_prob"
    router_scale: float = 0.0
    norm_eps: float = 1e-6

    def kwargs(self):
        return dict(alpha=self.alpha, use_sigmoid=self.use_sigmoid, router_type=self.router_type,
                    combine_mode=self.combine_mode, router_scale=self.router_scale,
                    norm_eps=self.norm_eps)


def reshape_head_tokens(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    """b l (h hd) -> b (l h) hd (M:132-137): a view of a contiguous x."""
    B, Lx, HD = x.shape
    assert HD % num_heads == 0, "last dimension must split into num_heads heads"
    return x.contiguous().view(B, Lx * num_heads, HD // num_heads)


def merge_head_tokens(x: torch.Tensor, seq_len: int, num_heads: int) -> torch.Tensor:
    """b (l h) hd -> b l (h hd) (M:139-144)."""
    B, LH, hd = x.shape
    assert LH == seq_len * num_heads, "token axis must be seq_len * num_heads"
    return x.contiguous().view(B, seq_len, num_heads * hd)


def route(x_tokens, router_proj_weights, cfg: RouterConfig, routing_bias=None):
    """_route_tokens (M:147-169): fp32 logits R x^T and the top-k selection on
    the fused router kernel.  Returns (expert_mask bool [B,E,T], group_sizes
    int32 [B,E], router_probs fp32 [B,E,T], balance_probs fp32 [B,E,T])."""
    return route_tokens(x_tokens, router_proj_weights, cfg.topk, routing_bias=routing_bias,
                        **cfg.kwargs())


def route_writers(k_cat, num_writers: int, router_proj_weights, cfg: RouterConfig,
                  routing_bias=None):
    """The routing of `num_writers` writers with equal token counts whose
    tokens are concatenated writer-major in k_cat [1, L*T, D], in ONE router
    launch: the writers are the router's batches, with one shared router
    ([E, D]) or one per writer ([L, E, D], memory_router_share_mode
    "per_layer"); routing_bias [E] or [L, E].  Each writer's routing is
    _route_tokens of its own tokens (M:147-169).  Returns (expert_mask
    [1,E,L*T], group_sizes [1,E] summed over the writers, router_probs
    [1,E,L*T], balance_probs [L,E,T]) on the concatenated token axis."""
    B1, LT, D = k_cat.shape
    assert B1 == 1 and LT % num_writers == 0, "k_cat must be [1, L*T, D]"
    T = LT // num_writers
    mask, gs, probs, bal = route_tokens(k_cat.contiguous().view(num_writers, T, D),
                                        router_proj_weights, cfg.topk, routing_bias=routing_bias,
                                        **cfg.kwargs())
    E = mask.shape[1]
    m = mask.transpose(0, 1).reshape(1, E, LT)
    p = probs.transpose(0, 1).reshape(1, E, LT)
    return m, gs.sum(0, keepdim=True, dtype=torch.int32), p, bal


def lb_info(balance_probs, group_sizes):
    """_make_lb_info (M:171-176)."""
    return balance_probs.sum(dim=-1), group_sizes


def _w0_w2(w0, w2, precomputed_w0_w2):
    if precomputed_w0_w2 is not None:
        return precomputed_w0_w2
    return torch.cat([w0, w2], dim=2).contiguous()


def apply_moe_fast_weights_grouped(x, w0, w1, w2, router_proj_weights, cfg: RouterConfig,
                                   num_heads: int, routing_bias=None, precomputed_w0_w2=None):
    """_apply_moe_fast_weights_grouped (M:296-349): x [B, L, H*hd] is split into
    head tokens, routed, permuted by expert, run through the grouped SwiGLU
    APPLY (w0, w2 [B,E,I,hd], w1 [B,E,hd,I]) and merged back with the gates.
    Returns (out [B, L, H*hd] in x's dtype, lb_info = (balance sums [B,E],
    group_sizes [B,E]))."""
    seq_len = x.shape[1]
    input_dtype = x.dtype
    xt = reshape_head_tokens(x, num_heads)
    w0_w2 = _w0_w2(w0, w2, precomputed_w0_w2)
    T, E = xt.shape[1], router_proj_weights.shape[-2]
    # Where no gradient flows through the read, the gate/up reads the routed
    # rows of xt through the inverse row map instead of a permuted copy (one
    # launch and the copy's traffic less, identical results)
    no_grad = not torch.is_grad_enabled() or not any(
        t is not None and t.requires_grad for t in (x, w0, w1, w2, precomputed_w0_w2))
    gather = no_grad and w0_w2.dtype == torch.bfloat16 and src_rows_supported(T, E)
    # the routing and its row map in one call (route_tokens_lb, then
    # make_row_id_map of its mask)
    routed = route_tokens_map(xt, router_proj_weights, cfg.topk, routing_bias=routing_bias,
                              with_src_rows=gather, **cfg.kwargs())
    expert_mask, group_sizes, router_probs, _, balance_sums, row_id_map = routed[:6]
    if gather:
        w1c = w1.contiguous()
        hidden = _grouped.gate_up_gather(w0_w2.contiguous(), xt.to(w0_w2.dtype).contiguous(),
                                         routed[6], group_sizes)
        y_perm = _grouped.gemm_nt(w1c, hidden, group_sizes)
    else:
        x_perm, _, row_id_map = permute_with_expert_mask(
            xt.to(w0_w2.dtype).contiguous(), expert_mask, router_probs, cfg.topk, row_id_map)
        y_perm = grouped_swiglu_ffn_fwd(w0_w2, w1.contiguous(), x_perm, group_sizes)
    out = unpermute_and_merge_with_probs(y_perm, row_id_map, router_probs)
    # _make_lb_info (M:171-176): the balance sums come from the router kernel
    return merge_head_tokens(out.to(input_dtype), seq_len, num_heads), (balance_sums, group_sizes)


@dataclass(frozen=True)
class Rope:
    """The fast-weight rotary embedding of one call: the reference's bf16
    cos / sin caches ([positions, rope_dim / 2], RotaryEmbedding
    _update_cos_sin_cache, rotary.py:394-433, as ref_base.py:342-355 builds
    it) and the call's seqlen_offset.  Rotary blocks of rope_dim features tile
    each token's feature vector (rearrange 'b l (nh d) -> b l nh d')."""

    cos: torch.Tensor
    sin: torch.Tensor
    seqlen_offset: int = 0

    @property
    def dim(self) -> int:
        return 2 * self.cos.shape[-1]

    @staticmethod
    def tables(dim: int, base: float, max_len: int, device, dtype=torch.bfloat16):
        """The cos / sin cache as RotaryEmbedding builds it (rotary.py:385-433,
        no xpos scale): fp32 positions, inv_freq = 1 / base^(2i / dim), freqs =
        outer(t, inv_freq), cos / sin in fp32 rounded to `dtype`."""
        inv_freq = 1.0 / (float(base) ** (torch.arange(0, dim, 2, device=device,
                                                       dtype=torch.float32) / dim))
        t = torch.arange(max_len, device=device, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        return torch.cos(freqs).to(dtype).contiguous(), torch.sin(freqs).to(dtype).contiguous()


_NORMS = {None: 0, "l2": 1, "rms": 2}


def _prep_geometry(x, rows_of, rope):
    B, Lx, HD = x.shape
    D = HD if rows_of is None else rows_of
    assert HD % D == 0, "rows must tile each token's features"
    if rope is None:
        return D, HD // D, Lx, 0, 0, None, None, 0, 0
    assert rope.cos.dtype == torch.bfloat16 and rope.sin.dtype == torch.bfloat16, (
        "the rotary tables must be bf16 (the reference's cache dtype)")
    assert rope.cos.shape == rope.sin.shape, "cos / sin tables of one shape"
    assert rope.seqlen_offset + Lx <= rope.cos.shape[0], "positions past the rotary tables"
    assert HD % rope.dim == 0, "rotary blocks must tile the features"
    return (D, HD // D, Lx, rope.dim, rope.seqlen_offset, rope.cos.contiguous(),
            rope.sin.contiguous(), rope.cos.shape[0], 1)


class _RowsPreprocess(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, silu, norm, rows_of, rope):
        L.require_device(x)
        x = x.contiguous()
        D, rpt, Lx, rdim, off, cos, sin, trows, _ = _prep_geometry(x, rows_of, rope)
        out_dtype = torch.bfloat16 if rope is not None else x.dtype
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        rows = x.numel() // D
        L.call("uttt_rows_preprocess", L.ptr(x), L.dtype_code(x.dtype), rows, D, D, int(silu),
               _NORMS[norm], L.ptr(cos) if cos is not None else None,
               L.ptr(sin) if sin is not None else None, rdim, rpt, Lx, off, trows, L.ptr(out), D,
               L.stream_of(x))
        ctx.save_for_backward(x)
        ctx.args = (silu, norm, rows_of, rope)
        return out

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        silu, norm, rows_of, rope = ctx.args
        D, rpt, Lx, rdim, off, cos, sin, trows, _ = _prep_geometry(x, rows_of, rope)
        out_dtype = torch.bfloat16 if rope is not None else x.dtype
        g = g.to(out_dtype).contiguous()
        gin = torch.empty_like(x)
        L.call("uttt_rows_preprocess_bwd", L.ptr(x), L.dtype_code(x.dtype), L.ptr(g),
               x.numel() // D, D, D, D, int(silu), _NORMS[norm],
               L.ptr(cos) if cos is not None else None, L.ptr(sin) if sin is not None else None,
               rdim, rpt, Lx, off, trows, L.ptr(gin), L.stream_of(x))
        return gin, None, None, None, None


def rows_preprocess(x: torch.Tensor, *, silu: bool = False, norm: str | None = None,
                    rows_of: int | None = None, rope: Rope | None = None) -> torch.Tensor:
    """The reference's row preprocessing of q / k / v [B, L, H*hd] on one HIP
    kernel: optional F.silu, then the optional parameter-free norm over rows
    of `rows_of` features (default: the whole vector) -- "l2" is l2_norm,
    x / (|x| + 1e-5), "rms" is rms_norm, x * rsqrt(mean(x^2) + 1e-5)
    (ref_base.py:181-195) -- then the optional rotary embedding (the input
    cast to the bf16 tables' dtype, rotated, bf16 out; rotary.py:83-104).
    Differentiable: the backward is the conjugate rotation, the norm's and the
    silu's backward on one kernel, rounded where the reference's autograd
    rounds.  Returns a new tensor (bf16 with rope, else x's dtype)."""
    assert norm in _NORMS, f"norm must be None, 'l2' or 'rms', got {norm!r}"
    return _RowsPreprocess.apply(x, bool(silu), norm, rows_of, rope)


def _norm_name(flag: bool, kind: str):
    assert kind in ("l2", "rms"), f"norm type must be 'l2' or 'rms', got {kind!r}"
    return kind if flag else None


def preprocess_update_inputs(k, v, lr, num_heads: int, *, qkv_silu: bool = False,
                             v_norm: bool = False, qk_norm: bool = False,
                             norm_type: str = "rms", qk_norm_type: str = "l2",
                             rope: Rope | None = None):
    """_preprocess_update_inputs (M:630-665) after the learned qk rescale:
    k -> [silu] -> [qk norm per head, qk_norm_type] -> [rotary] and
    v -> [silu] -> [v norm over the whole vector, norm_type], in the
    reference's order (rotary last, on the normalised k), then head tokens,
    and lr [B, L, 3] (shared by the heads) or [B, L, 3H] spread to
    [B, L*H, 3].  norm_type / qk_norm_type default to the reference's config
    defaults (memory_norm_type "rms", memory_qk_norm_type "l2",
    configuration_recurrent_lact_base.py:66-67).  Differentiable in k, v and
    lr.  The learned qk rescale (memory_qk_rescale, M:637-638) comes first in
    the reference and stays with the model: apply it to k before this call."""
    B, Lx, HD = k.shape
    hd = HD // num_heads
    if qkv_silu or qk_norm or rope is not None:
        k = rows_preprocess(k, silu=qkv_silu, norm=_norm_name(qk_norm, qk_norm_type),
                            rows_of=hd if qk_norm else None, rope=rope)
    if qkv_silu or v_norm:
        v = rows_preprocess(v, silu=qkv_silu, norm=_norm_name(v_norm, norm_type))
    k_tokens = reshape_head_tokens(k, num_heads)
    v_tokens = reshape_head_tokens(v, num_heads)
    if lr.shape[2] == 3:
        lr_mh = lr.unsqueeze(2).expand(-1, -1, num_heads, -1)
    else:
        lr_mh = lr.view(B, Lx, num_heads, 3)
    lr_tokens = lr_mh.reshape(B, Lx * num_heads, 3).contiguous()
    return k_tokens, v_tokens, lr_tokens


def preprocess_read_query(q, num_heads: int, *, qkv_silu: bool = False, qk_norm: bool = False,
                          qk_norm_type: str = "l2", rope: Rope | None = None):
    """The MoE read's q path (M:588-601) after the learned qk rescale:
    q -> [silu] -> [qk norm per head] -> [rotary], one kernel; returns
    [B, L, H*hd] for apply_moe_fast_weights_grouped.  Differentiable."""
    if not (qkv_silu or qk_norm or rope is not None):
        return q
    hd = q.shape[-1] // num_heads
    return rows_preprocess(q, silu=qkv_silu, norm=_norm_name(qk_norm, qk_norm_type),
                           rows_of=hd if qk_norm else None, rope=rope)


def moe_update_grads_packed(k_tokens, v_tokens, lr_tokens, w0_w2, w1, expert_mask, group_sizes,
                            router_probs, topk: int):
    """The grouped part of _compute_moe_update_grads_grouped (M:484-512): lr
    split and cast to the fast-weight dtype, k / v*p / lr permuted by expert,
    then the grouped UPDATE.  Returns (dW0_W2 [B,E,2I,D], dW1 [B,E,D,I]) in
    bf16, differentiable with respect to k, v, lr and the router probs."""
    target_dtype = w0_w2.dtype
    lrs = [lr_tokens[:, :, j].contiguous().to(target_dtype) for j in range(3)]
    k_perm, v_perm, lr0_p, lr1_p, lr2_p = permute_kv_and_lrs(
        k_tokens.contiguous().to(target_dtype), v_tokens.contiguous(), *lrs, expert_mask,
        router_probs, topk)
    return grouped_lact_swiglu_ffn_fast_weight_grads(w0_w2, w1.contiguous(), k_perm, v_perm,
                                                     lr0_p, lr1_p, lr2_p, group_sizes)


def compute_moe_update_grads_grouped(k_tokens, v_tokens, lr_tokens, w0, w1, w2, expert_mask,
                                     group_sizes, router_probs, topk: int,
                                     master_dtype=torch.float32, precomputed_w0_w2=None):
    """_compute_moe_update_grads_grouped (M:453-518): returns (dW0, dW1, dW2)
    upcast to the master dtype (M:514-518)."""
    dw0_w2, dw1 = moe_update_grads_packed(k_tokens, v_tokens, lr_tokens,
                                          _w0_w2(w0, w2, precomputed_w0_w2), w1, expert_mask,
                                          group_sizes, router_probs, topk)
    inter_dim = w0.shape[2]
    return (dw0_w2[:, :, :inter_dim, :].to(master_dtype), dw1.to(master_dtype),
            dw0_w2[:, :, inter_dim:, :].to(master_dtype))


@dataclass
class WriterInputs:
    """One writer layer's preprocessed update inputs and its routing."""

    k_tokens: torch.Tensor      # [B, T, D]
    v_tokens: torch.Tensor      # [B, T, D]
    lr_tokens: torch.Tensor     # [B, T, 3]
    expert_mask: torch.Tensor   # [B, E, T]
    router_probs: torch.Tensor  # [B, E, T]


def concat_writers(writers: Sequence[WriterInputs]):
    """The writers' tokens one after another: (k, v, lr, mask, probs, group
    sizes) of the concatenated token axis.  Row order inside each expert's
    segment is then writer-major, token-ascending."""
    assert len(writers) > 0, "at least one writer"
    if len(writers) == 1:
        w = writers[0]
        m, p = w.expert_mask, w.router_probs
    else:
        m = torch.cat([w.expert_mask for w in writers], dim=2)
        p = torch.cat([w.router_probs for w in writers], dim=2)
    cat = (lambda ts: ts[0]) if len(writers) == 1 else (lambda ts: torch.cat(ts, dim=1))
    k = cat([w.k_tokens for w in writers])
    v = cat([w.v_tokens for w in writers])
    lr = cat([w.lr_tokens for w in writers])
    gs = m.sum(dim=-1, dtype=torch.int32)
    return k, v, lr, m, p, gs


def aggregate_moe_update_grads(writers: Sequence[WriterInputs], w0, w1, w2, topk: int,
                               master_dtype=torch.float32, precomputed_w0_w2=None,
                               packed: bool = False):
    """The writers' raw gradients of one chunk summed (M:2428-2445), as one
    grouped UPDATE over their concatenated tokens.  Returns (dW0, dW1, dW2)
    in master_dtype, or (dW0_W2, dW1) in bf16 when `packed`."""
    k, v, lr, m, p, gs = concat_writers(writers)
    w0_w2 = _w0_w2(w0, w2, precomputed_w0_w2)
    dw0_w2, dw1 = moe_update_grads_packed(k, v, lr, w0_w2, w1, m, gs, p, topk)
    if packed:
        return dw0_w2, dw1
    inter_dim = w0_w2.shape[2] // 2
    return (dw0_w2[:, :, :inter_dim, :].to(master_dtype), dw1.to(master_dtype),
            dw0_w2[:, :, inter_dim:, :].to(master_dtype))

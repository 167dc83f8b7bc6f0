"""Token permute / unpermute by expert on the gfx950 kernels of libuttt_hip.so.

Drop-in for the reference module
``uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/triton_permute.py``
(cited as P:line): same public names, signatures, argument meaning, return
values, autograd behaviour and AssertionError checks.  All work runs in the
HIP kernels of csrc/permute.hip on torch's current stream; no CPU path.  Each
launch is a registered torch.ops.uttt_hip op (uttt_amd._ops) so that
torch.compile traces it; optional outputs cross the op as 0-element tensors.
"""
from __future__ import annotations

from typing import Optional, Union

import torch
from torch import Tensor

from uttt_amd import _lib as L  # absolute: the package also works mounted in the reference tree
from uttt_amd._ops import none_if_empty, traced_op


def _mask_arg(routing_map: torch.Tensor):
    """(tensor, element bytes) for the row-map kernel; bool/uint8 and int32 pass as is."""
    if routing_map.dtype in (torch.bool, torch.uint8, torch.int8):
        return routing_map, 1
    if routing_map.dtype == torch.int32:
        return routing_map, 4
    return routing_map.to(torch.int32), 4


def _probs_f32(probs):
    if probs is None:
        return None
    return probs if probs.dtype == torch.float32 else probs.float()


def make_row_id_map(
    routing_map: torch.Tensor,
    batch_size: int,
    num_tokens: int,
    num_experts: int,
    group_sizes: torch.Tensor | None = None,
):
    """Row map of the permutation (P:283-393).

    routing_map: [B, E, T] 0/1 mask (bool or integer, any strides).
    Returns row_id_map [B, T, 2E+1] int32, identical to the reference's: for
    token t with n routed experts, columns [0, n) hold its destination rows in
    descending order, [E, E+n) the matching experts, [2E] holds n.
    `group_sizes` (optional, [B, E] int32) additionally receives the per-expert
    token counts; this keyword is an extension (the reference has none).
    """
    if group_sizes is None:
        return _row_id_map(routing_map, batch_size, num_tokens, num_experts)
    return _row_id_map_impl(routing_map, batch_size, num_tokens, num_experts, group_sizes)


def _row_id_map_fake(routing_map, batch_size, num_tokens, num_experts):
    return routing_map.new_empty((batch_size, num_tokens, 2 * num_experts + 1), dtype=torch.int32)


@traced_op("make_row_id_map", _row_id_map_fake)
def _row_id_map(routing_map: Tensor, batch_size: int, num_tokens: int,
                num_experts: int) -> Tensor:
    return _row_id_map_impl(routing_map, batch_size, num_tokens, num_experts, None)


def _row_id_map_impl(routing_map, batch_size, num_tokens, num_experts, group_sizes):
    L.require_device(routing_map)
    assert routing_map.shape == (batch_size, num_experts, num_tokens)
    m, mb = _mask_arg(routing_map)
    row_id_map = torch.empty(
        (batch_size, num_tokens, 2 * num_experts + 1), dtype=torch.int32, device=m.device
    )
    ws_bytes = L.lib().uttt_row_id_map_workspace_bytes(batch_size, max(num_tokens, 1), num_experts)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=m.device)
    if group_sizes is not None:
        assert group_sizes.dtype == torch.int32 and group_sizes.is_contiguous()
        assert group_sizes.shape == (batch_size, num_experts)
    L.call(
        "uttt_make_row_id_map",
        L.ptr(m), mb, m.stride(0), m.stride(1), m.stride(2),
        batch_size, num_tokens, num_experts,
        L.ptr(row_id_map), L.ptr(group_sizes), L.ptr(ws), ws_bytes, L.stream_of(m),
    )
    return row_id_map


def triton_permute_with_mask_map(
    inp: torch.Tensor,
    row_id_map: torch.Tensor,
    probs: torch.Tensor,
    batch_size: int,
    num_tokens: int,
    num_experts: int,
    num_out_tokens: int,
    hidden_size: int,
):
    """Scatter each token row to its expert slots (P:493-571).

    Returns (output [B, num_out_tokens, H], permuted_probs [B, num_out_tokens]
    or None).  Slots whose prob is exactly 0 get a zero row (P:466-469); rows
    that no token fills are left uninitialised, as in the reference.
    """
    out, pp = _permute(inp, row_id_map, probs, batch_size, num_tokens, num_experts,
                       num_out_tokens, hidden_size)
    return out, none_if_empty(pp)


def _permute_fake(inp, row_id_map, probs, batch_size, num_tokens, num_experts, num_out_tokens,
                  hidden_size):
    out = inp.new_empty((batch_size, num_out_tokens, hidden_size))
    pp = inp.new_empty((batch_size, num_out_tokens) if probs is not None else (0,),
                       dtype=probs.dtype if probs is not None else torch.float32)
    return out, pp


@traced_op("permute_fwd", _permute_fake)
def _permute(inp: Tensor, row_id_map: Tensor, probs: Optional[Tensor], batch_size: int,
             num_tokens: int, num_experts: int, num_out_tokens: int,
             hidden_size: int) -> tuple[Tensor, Tensor]:
    L.require_device(inp, row_id_map, probs)
    inp = inp.contiguous()
    assert inp.shape == (batch_size, num_tokens, hidden_size)
    assert row_id_map.dtype == torch.int32 and row_id_map.is_contiguous()
    output = torch.empty(
        (batch_size, num_out_tokens, hidden_size), dtype=inp.dtype, device=inp.device
    )
    p32 = _probs_f32(probs)
    permuted_probs = None
    pp32 = None
    if probs is not None:
        pp32 = torch.empty((batch_size, num_out_tokens), dtype=torch.float32, device=inp.device)
    L.call(
        "uttt_permute_fwd",
        L.ptr(inp), L.dtype_code(inp.dtype), batch_size, num_tokens, hidden_size,
        L.ptr(row_id_map), num_experts,
        L.ptr(p32),
        p32.stride(0) if p32 is not None else 0,
        p32.stride(1) if p32 is not None else 0,
        p32.stride(2) if p32 is not None else 0,
        L.ptr(output), num_out_tokens, L.ptr(pp32), L.stream_of(inp),
    )
    if probs is not None:
        permuted_probs = pp32 if probs.dtype == torch.float32 else pp32.to(probs.dtype)
    else:
        permuted_probs = torch.empty((0,), dtype=torch.float32, device=inp.device)
    return output, permuted_probs


def triton_permute_with_mask_map_bwd_batched(
    fwd_output_grad: torch.Tensor,
    row_id_map: torch.Tensor,
    permuted_probs_grad: Union[torch.Tensor, None],
    batch_size: int,
    num_tokens: int,
    num_experts: int,
    hidden_size: int,
):
    """Backward of the permute (P:700-762): returns (grad_inp, grad_probs)."""
    gi, gp = _permute_bwd(fwd_output_grad, row_id_map, permuted_probs_grad, batch_size,
                          num_tokens, num_experts, hidden_size)
    return gi, none_if_empty(gp)


def _permute_bwd_fake(fwd_output_grad, row_id_map, permuted_probs_grad, batch_size, num_tokens,
                      num_experts, hidden_size):
    gi = fwd_output_grad.new_empty((batch_size, num_tokens, hidden_size))
    if permuted_probs_grad is None:
        return gi, fwd_output_grad.new_empty((0,), dtype=torch.float32)
    return gi, fwd_output_grad.new_empty((batch_size, num_experts, num_tokens),
                                         dtype=permuted_probs_grad.dtype)


@traced_op("permute_bwd", _permute_bwd_fake)
def _permute_bwd(fwd_output_grad: Tensor, row_id_map: Tensor,
                 permuted_probs_grad: Optional[Tensor], batch_size: int, num_tokens: int,
                 num_experts: int, hidden_size: int) -> tuple[Tensor, Tensor]:
    L.require_device(fwd_output_grad, row_id_map, permuted_probs_grad)
    fwd_output_grad = fwd_output_grad.contiguous()
    device, dtype = fwd_output_grad.device, fwd_output_grad.dtype
    num_out = fwd_output_grad.shape[1]
    grad_inp = torch.empty((batch_size, num_tokens, hidden_size), dtype=dtype, device=device)
    grad_probs = None
    gpp32 = None
    gp32 = None
    if permuted_probs_grad is not None:
        gpp32 = _probs_f32(permuted_probs_grad).contiguous()
        gp32 = torch.empty((batch_size, num_experts, num_tokens), dtype=torch.float32, device=device)
    L.call(
        "uttt_permute_bwd",
        L.ptr(fwd_output_grad), L.dtype_code(dtype), batch_size, num_tokens, hidden_size,
        L.ptr(row_id_map), num_experts, num_out, L.ptr(gpp32), L.ptr(grad_inp), L.ptr(gp32),
        L.stream_of(fwd_output_grad),
    )
    if permuted_probs_grad is not None:
        grad_probs = gp32 if permuted_probs_grad.dtype == torch.float32 else gp32.to(
            permuted_probs_grad.dtype
        )
    else:
        grad_probs = torch.empty((0,), dtype=torch.float32, device=device)
    return grad_inp, grad_probs


def triton_unpermute_with_mask_map(
    inp: torch.Tensor,
    row_id_map: torch.Tensor,
    merging_probs: Union[torch.Tensor, None],
    batch_size: int,
    num_tokens: int,
    num_experts: int,
    hidden_size: int,
):
    """Gate-weighted merge of the expert rows back to tokens (P:870-928).

    out[t] = cast(sum_j y[row_j] * p[e_j, t]) accumulated in fp32.
    merging_probs may be [B, E, T] or any strided view of that shape.
    """
    return _unpermute(inp, row_id_map, merging_probs, batch_size, num_tokens, num_experts,
                      hidden_size)


def _unpermute_fake(inp, row_id_map, merging_probs, batch_size, num_tokens, num_experts,
                    hidden_size):
    return inp.new_empty((batch_size, num_tokens, hidden_size))


@traced_op("unpermute_fwd", _unpermute_fake)
def _unpermute(inp: Tensor, row_id_map: Tensor, merging_probs: Optional[Tensor], batch_size: int,
               num_tokens: int, num_experts: int, hidden_size: int) -> Tensor:
    L.require_device(inp, row_id_map, merging_probs)
    inp = inp.contiguous()
    num_out = inp.shape[1]
    output = torch.empty((batch_size, num_tokens, hidden_size), dtype=inp.dtype, device=inp.device)
    p32 = _probs_f32(merging_probs)
    L.call(
        "uttt_unpermute_fwd",
        L.ptr(inp), L.dtype_code(inp.dtype), batch_size, num_out, hidden_size,
        L.ptr(row_id_map), num_tokens, num_experts, L.ptr(p32),
        p32.stride(0) if p32 is not None else 0,
        p32.stride(1) if p32 is not None else 0,
        p32.stride(2) if p32 is not None else 0,
        L.ptr(output), L.stream_of(inp),
    )
    return output


def triton_unpermute_with_mask_map_bwd_with_merging_probs(
    fwd_output_grad: torch.Tensor,
    row_id_map: torch.Tensor,
    fwd_input: torch.Tensor,
    merging_probs: torch.Tensor,
    batch_size: int,
    num_tokens: int,
    num_experts: int,
    num_out_tokens: int,
    hidden_size: int,
):
    """Backward of the merge (P:1078-1141): returns (act_grad, merging_probs_grad)."""
    return _unpermute_bwd(fwd_output_grad, row_id_map, fwd_input, merging_probs, batch_size,
                          num_tokens, num_experts, num_out_tokens, hidden_size)


def _unpermute_bwd_fake(fwd_output_grad, row_id_map, fwd_input, merging_probs, batch_size,
                        num_tokens, num_experts, num_out_tokens, hidden_size):
    return (fwd_output_grad.new_empty((batch_size, num_out_tokens, hidden_size)),
            merging_probs.new_empty(merging_probs.shape))


@traced_op("unpermute_bwd", _unpermute_bwd_fake)
def _unpermute_bwd(fwd_output_grad: Tensor, row_id_map: Tensor, fwd_input: Tensor,
                   merging_probs: Tensor, batch_size: int, num_tokens: int, num_experts: int,
                   num_out_tokens: int, hidden_size: int) -> tuple[Tensor, Tensor]:
    L.require_device(fwd_output_grad, row_id_map, fwd_input, merging_probs)
    fwd_output_grad = fwd_output_grad.contiguous()
    fwd_input = fwd_input.contiguous()
    assert fwd_input.dtype == fwd_output_grad.dtype
    device, dtype = fwd_output_grad.device, fwd_output_grad.dtype
    act_grad = torch.empty((batch_size, num_out_tokens, hidden_size), dtype=dtype, device=device)
    p32 = _probs_f32(merging_probs)
    gp = torch.empty(p32.shape, dtype=torch.float32, device=device)
    L.call(
        "uttt_unpermute_bwd",
        L.ptr(fwd_output_grad), L.ptr(fwd_input), L.dtype_code(dtype), batch_size, num_tokens,
        hidden_size, L.ptr(row_id_map), num_experts, num_out_tokens,
        L.ptr(p32), p32.stride(0), p32.stride(1), p32.stride(2),
        L.ptr(act_grad), L.ptr(gp), gp.stride(0), gp.stride(1), gp.stride(2),
        L.stream_of(fwd_output_grad),
    )
    if merging_probs.dtype != torch.float32:
        gp = gp.to(merging_probs.dtype)
    return act_grad, gp


class PermuteWithMaskMap(torch.autograd.Function):
    """Autograd wrapper of the permute (P:1169-1238)."""

    @staticmethod
    def forward(ctx, inp, expert_mask, probs, topk: int, row_id_map: torch.Tensor):
        B, num_tokens, hidden_size = inp.shape
        num_experts = expert_mask.shape[1]
        num_output_tokens = topk * num_tokens
        if row_id_map is None:
            row_id_map = make_row_id_map(expert_mask, B, num_tokens, num_experts)
        out, permuted_probs = triton_permute_with_mask_map(
            inp, row_id_map, probs, B, num_tokens, num_experts, num_output_tokens, hidden_size
        )
        ctx.num_tokens = num_tokens
        ctx.num_experts = num_experts
        ctx.hidden_size = hidden_size
        ctx.batch_size = B
        ctx.save_for_backward(probs, row_id_map)
        ctx.mark_non_differentiable(row_id_map)
        return out, permuted_probs, row_id_map

    @staticmethod
    def backward(ctx, grad_permuted_output, grad_permuted_probs, grad_row_id_map):
        probs, row_id_map = ctx.saved_tensors
        if grad_permuted_probs is not None:
            grad_permuted_probs = grad_permuted_probs.contiguous()
        grad_inp, grad_probs = triton_permute_with_mask_map_bwd_batched(
            grad_permuted_output.contiguous(),
            row_id_map,
            grad_permuted_probs,
            ctx.batch_size,
            ctx.num_tokens,
            ctx.num_experts,
            ctx.hidden_size,
        )
        return grad_inp, None, grad_probs, None, None


def permute_with_expert_mask(
    inp: torch.Tensor,
    expert_mask: torch.Tensor,
    probs: torch.Tensor,
    topk: int,
    row_id_map: torch.Tensor = None,
):
    """(out [B, topk*T, H], permuted_probs [B, topk*T] or None, row_id_map) (P:1241-1248)."""
    return PermuteWithMaskMap.apply(inp, expert_mask, probs, topk, row_id_map)


class UnPermuteWithMaskMap(torch.autograd.Function):
    """Autograd wrapper of the gate-weighted merge (P:1251-1313)."""

    @staticmethod
    def forward(ctx, permuted_inps, row_id_map, original_probs):
        B, num_output_tokens, hidden_size = permuted_inps.shape
        _, num_experts, num_tokens = original_probs.shape
        merged = triton_unpermute_with_mask_map(
            permuted_inps, row_id_map, original_probs, B, num_tokens, num_experts, hidden_size
        )
        ctx.num_tokens = num_tokens
        ctx.num_experts = num_experts
        ctx.hidden_size = hidden_size
        ctx.batch_size = B
        ctx.num_output_tokens = num_output_tokens
        ctx.save_for_backward(permuted_inps, row_id_map, original_probs)
        return merged

    @staticmethod
    def backward(ctx, grad_merged_output):
        fwd_input, row_id_map, merging_probs = ctx.saved_tensors
        grad_permuted, grad_probs = triton_unpermute_with_mask_map_bwd_with_merging_probs(
            grad_merged_output.contiguous(),
            row_id_map,
            fwd_input,
            merging_probs,
            ctx.batch_size,
            ctx.num_tokens,
            ctx.num_experts,
            ctx.num_output_tokens,
            ctx.hidden_size,
        )
        return grad_permuted, None, grad_probs


def unpermute_and_merge_with_probs(permuted_x, row_id_map, original_probs):
    """[B, T, H] merge of the permuted rows with the router probs (P:1316-1325)."""
    return UnPermuteWithMaskMap.apply(permuted_x, row_id_map, original_probs)


class PermuteKVAndLRs(torch.autograd.Function):
    """Permute k, v*p and the three per-token lrs in one pass (P:1730-1980)."""

    @staticmethod
    def forward(ctx, k, v, lr0, lr1, lr2, expert_mask, probs, topk):
        B, T, H = k.shape
        E = expert_mask.shape[1]
        assert expert_mask.shape == (B, E, T)
        assert probs.shape == (B, E, T)
        lr_was_3d = lr0.ndim == 3
        if lr_was_3d:
            lr0_2d, lr1_2d, lr2_2d = lr0.squeeze(-1), lr1.squeeze(-1), lr2.squeeze(-1)
        else:
            lr0_2d, lr1_2d, lr2_2d = lr0, lr1, lr2
        assert lr0_2d.shape == (B, T)
        assert lr1_2d.shape == (B, T)
        assert lr2_2d.shape == (B, T)
        assert lr0_2d.dtype == lr1_2d.dtype == lr2_2d.dtype
        L.require_device(k, v, lr0_2d, expert_mask, probs)
        k = k.contiguous()
        v = v.contiguous()
        lr0_2d, lr1_2d, lr2_2d = (x.contiguous() for x in (lr0_2d, lr1_2d, lr2_2d))
        # bool / uint8 / int32 masks are read as stored (no int32 copy)
        row_id_map = make_row_id_map(expert_mask, B, T, E)
        num_out = topk * T
        out_k, out_v, out_lr0, out_lr1, out_lr2 = _kv_fwd(k, v, lr0_2d, lr1_2d, lr2_2d,
                                                          row_id_map, probs, num_out)
        ctx.batch_size, ctx.num_tokens, ctx.num_experts, ctx.hidden_size = B, T, E, H
        ctx.lr_was_3d = lr_was_3d
        ctx.topk = topk
        ctx.save_for_backward(v, probs, row_id_map)
        return out_k, out_v, out_lr0, out_lr1, out_lr2

    @staticmethod
    def backward(ctx, grad_out_k, grad_out_v_scaled, grad_out_lr0, grad_out_lr1, grad_out_lr2):
        B, T, E, H = ctx.batch_size, ctx.num_tokens, ctx.num_experts, ctx.hidden_size
        v, probs, row_id_map = ctx.saved_tensors
        num_out = ctx.topk * T
        dev = v.device
        # autograd passes None for an output that got no gradient
        kv_dtype = next(
            (g.dtype for g in (grad_out_k, grad_out_v_scaled) if g is not None), v.dtype
        )
        gk, gv = (
            (g if g is not None else torch.zeros((B, num_out, H), dtype=kv_dtype, device=dev))
            .contiguous()
            for g in (grad_out_k, grad_out_v_scaled)
        )
        assert gk.dtype == gv.dtype
        glr = [g for g in (grad_out_lr0, grad_out_lr1, grad_out_lr2) if g is not None]
        lr_dtype = glr[0].dtype if glr else torch.float32
        glr0, glr1, glr2 = (
            (g if g is not None else torch.zeros((B, num_out), dtype=lr_dtype, device=dev))
            .reshape(B, num_out).to(lr_dtype).contiguous()
            for g in (grad_out_lr0, grad_out_lr1, grad_out_lr2)
        )
        grad_k, grad_v, grad_lr0, grad_lr1, grad_lr2, gp32 = _kv_bwd(
            gk, gv, glr0, glr1, glr2, v, probs, row_id_map, T)
        grad_probs = gp32 if probs.dtype == torch.float32 else gp32.to(probs.dtype)
        if ctx.lr_was_3d:
            grad_lr0, grad_lr1, grad_lr2 = (g.unsqueeze(-1) for g in (grad_lr0, grad_lr1, grad_lr2))
        return grad_k, grad_v, grad_lr0, grad_lr1, grad_lr2, None, grad_probs, None


def _kv_fwd_fake(k, v, lr0, lr1, lr2, row_id_map, probs, num_out):
    B, T, H = k.shape
    return (k.new_empty((B, num_out, H)), k.new_empty((B, num_out, H)),
            lr0.new_empty((B, num_out)), lr0.new_empty((B, num_out)), lr0.new_empty((B, num_out)))


@traced_op("permute_kv_lrs_fwd", _kv_fwd_fake)
def _kv_fwd(k: Tensor, v: Tensor, lr0: Tensor, lr1: Tensor, lr2: Tensor, row_id_map: Tensor,
            probs: Tensor, num_out: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """k, v*p and the lrs to their expert slots (P:1345-1493); lr [B, T]."""
    B, T, H = k.shape
    E = (row_id_map.shape[-1] - 1) // 2
    out_k = torch.empty((B, num_out, H), dtype=k.dtype, device=k.device)
    out_v = torch.empty_like(out_k)
    out_lr0 = torch.empty((B, num_out), dtype=lr0.dtype, device=k.device)
    out_lr1 = torch.empty_like(out_lr0)
    out_lr2 = torch.empty_like(out_lr0)
    p32 = _probs_f32(probs)
    L.call(
        "uttt_permute_kv_lrs_fwd",
        L.ptr(k), L.dtype_code(k.dtype), L.ptr(v), L.dtype_code(v.dtype),
        L.ptr(lr0), L.ptr(lr1), L.ptr(lr2), lr0.element_size(),
        B, T, H, L.ptr(row_id_map), E,
        L.ptr(p32), p32.stride(0), p32.stride(1), p32.stride(2),
        L.ptr(out_k), L.ptr(out_v), L.ptr(out_lr0), L.ptr(out_lr1), L.ptr(out_lr2),
        num_out, L.stream_of(k),
    )
    return out_k, out_v, out_lr0, out_lr1, out_lr2


def _kv_bwd_fake(gk, gv, glr0, glr1, glr2, v, probs, row_id_map, num_tokens):
    B, _, H = gk.shape
    E = (row_id_map.shape[-1] - 1) // 2
    return (gk.new_empty((B, num_tokens, H)), v.new_empty((B, num_tokens, H)),
            glr0.new_empty((B, num_tokens)), glr0.new_empty((B, num_tokens)),
            glr0.new_empty((B, num_tokens)),
            gk.new_empty((B, E, num_tokens), dtype=torch.float32))


@traced_op("permute_kv_lrs_bwd", _kv_bwd_fake)
def _kv_bwd(gk: Tensor, gv: Tensor, glr0: Tensor, glr1: Tensor, glr2: Tensor, v: Tensor,
            probs: Tensor, row_id_map: Tensor, num_tokens: int
            ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Backward of _kv_fwd (P:1508-1727): grads of k, v, the lrs and the probs (fp32)."""
    B, num_out, H = gk.shape
    T = num_tokens
    E = (row_id_map.shape[-1] - 1) // 2
    dev = gk.device
    lr_dtype = glr0.dtype
    grad_k = torch.empty((B, T, H), dtype=gk.dtype, device=dev)
    grad_v = torch.empty((B, T, H), dtype=v.dtype, device=dev)
    grad_lr0 = torch.empty((B, T), dtype=lr_dtype, device=dev)
    grad_lr1 = torch.empty_like(grad_lr0)
    grad_lr2 = torch.empty_like(grad_lr0)
    p32 = _probs_f32(probs)
    gp32 = torch.empty((B, E, T), dtype=torch.float32, device=dev)
    L.call(
        "uttt_permute_kv_lrs_bwd",
        L.ptr(gk), L.ptr(gv), L.dtype_code(gk.dtype),
        L.ptr(glr0), L.ptr(glr1), L.ptr(glr2), L.dtype_code(lr_dtype),
        L.ptr(v), L.dtype_code(v.dtype),
        L.ptr(p32), p32.stride(0), p32.stride(1), p32.stride(2),
        B, T, H, L.ptr(row_id_map), E, num_out,
        L.ptr(grad_k), L.ptr(grad_v), L.ptr(grad_lr0), L.ptr(grad_lr1), L.ptr(grad_lr2),
        L.ptr(gp32), L.stream_of(gk),
    )
    return grad_k, grad_v, grad_lr0, grad_lr1, grad_lr2, gp32


def permute_kv_and_lrs(
    k: torch.Tensor,
    v: torch.Tensor,
    lr0: torch.Tensor,
    lr1: torch.Tensor,
    lr2: torch.Tensor,
    expert_mask: torch.Tensor,
    probs: torch.Tensor,
    topk: int,
):
    """(k_p, (v*p)_p, lr0_p, lr1_p, lr2_p), each [B, topk*T, ...] (P:1983-1993)."""
    return PermuteKVAndLRs.apply(k, v, lr0, lr1, lr2, expert_mask, probs, topk)

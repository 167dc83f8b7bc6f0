"""Oracle of the uTTT-MoE update glue (checker only; see oracle/__init__.py).

Reference (M:) uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py,
(RB:) uttt_llm/flame/custom_models/uttt_moe/ref_base.py and
(RO:) uttt_llm/flame/custom_models/uttt_moe/rotary.py:

  preprocess_rows    the qkv_silu / v_norm / qk_norm / rotary steps of
                     _preprocess_update_inputs (M:641-654) and of the read's
                     q path (M:588-601): F.silu, then l2_norm or rms_norm
                     (RB:181-195, torch.compile'd: fp32 inside, the result
                     rounded to the dtype), then the rotary embedding
                     (RB:342-355; RO: rotary.py:83-104 non-interleaved, bf16
                     cos / sin tables of RO:394-433)
  preprocess_rows_bwd  its backward with the reference autograd's rounding
                     points (the conjugate rotation RO:245-266 stored bf16,
                     the norm's and silu's backward stored in the dtype)
  rope_tables        the cos / sin cache of RO:385-433
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


def rope_tables(dim: int, base: float, max_len: int, dtype=torch.bfloat16):
    """RO:385-433 without the xpos scale: inv_freq = 1 / base^(2i / dim) in
    fp32, fp32 positions, freqs = outer(t, inv_freq), cos / sin rounded to
    dtype.  Returns (cos, sin) [max_len, dim / 2]."""
    inv_freq = 1.0 / (float(base) ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    freqs = torch.outer(torch.arange(max_len, dtype=torch.float32), inv_freq)
    return torch.cos(freqs).to(dtype), torch.sin(freqs).to(dtype)


def _rope_fp32(y, cos, sin, offset, conj=False):
    """The non-interleaved rotary of RO:86-104 in fp32 on y [B, L, F] (F a
    multiple of rope_dim): pair (j, j + R) of every rope_dim block rotated by
    the bf16 table values at position l + offset; conj: the backward's
    conjugate rotation (RO:263)."""
    B, Lx, Fdim = y.shape
    R = cos.shape[-1]
    c = cos[offset:offset + Lx].float().view(1, Lx, 1, R)
    s = sin[offset:offset + Lx].float().view(1, Lx, 1, R)
    if conj:
        s = -s
    blk = y.reshape(B, Lx, Fdim // (2 * R), 2 * R)
    x0, x1 = blk[..., :R], blk[..., R:]
    o0 = x0 * c - x1 * s
    o1 = x0 * s + x1 * c
    return torch.cat([o0, o1], dim=-1).reshape(B, Lx, Fdim)


def _norm_fp32(y, norm):
    if norm == "l2":
        return y / (y.double().pow(2).sum(-1, keepdim=True).sqrt().float() + 1e-5)
    if norm == "rms":
        return y * torch.rsqrt(y.double().pow(2).mean(-1, keepdim=True).float() + 1e-5)
    return y


def preprocess_rows(x, silu=False, norm=None, rows_of=None, rope=None):
    """x [B, L, F] -> [silu] -> [norm over rows of `rows_of` features] ->
    [rotary], each step rounded as the reference: F.silu to x's dtype; the
    compiled norm in fp32, its result to x's dtype (RB:181-195); the rotary
    input cast to the tables' bf16, rotated in fp32, stored bf16.
    rope = (cos, sin, seqlen_offset) or None."""
    dt = x.dtype
    B, Lx, Fdim = x.shape
    D = Fdim if rows_of is None else rows_of
    y = x.float()
    if silu:
        y = (y * torch.sigmoid(y)).to(dt).float()
    y = _norm_fp32(y.reshape(B, Lx, Fdim // D, D), norm).reshape(B, Lx, Fdim).to(dt).float()
    if rope is None:
        return y.to(dt)
    cos, sin, offset = rope
    y = y.to(torch.bfloat16).float()
    return _rope_fp32(y, cos, sin, offset).to(torch.bfloat16)


def preprocess_rows_bwd(x, g, silu=False, norm=None, rows_of=None, rope=None):
    """grad_x of preprocess_rows given its output's gradient g, with the
    reference autograd's rounding points: the conjugate rotation stored bf16
    (then cast to x's dtype), the norm's backward (fp32, stored in x's
    dtype), F.silu's backward (fp32, stored in x's dtype).  The formulas:
    l2  y = s / (n + e):  g_s = g / (n + e) - s (s . g) / (n (n + e)^2);
    rms y = s r, r = (mean s^2 + e)^-1/2:  g_s = r g - s (s . g) r^3 / D;
    silu:  g_x = g_s sig(x) (1 + x (1 - sig(x)))."""
    dt = x.dtype
    B, Lx, Fdim = x.shape
    D = Fdim if rows_of is None else rows_of
    gg = g.float()
    if rope is not None:
        cos, sin, offset = rope
        gg = _rope_fp32(gg, cos, sin, offset, conj=True).to(torch.bfloat16).to(dt).float()
    xf = x.float()
    s = (xf * torch.sigmoid(xf)).to(dt).float() if silu else xf
    if norm is not None:
        sr = s.reshape(B, Lx, Fdim // D, D)
        gr = gg.reshape(B, Lx, Fdim // D, D)
        dot = (sr.double() * gr.double()).sum(-1, keepdim=True).float()
        ss = sr.double().pow(2).sum(-1, keepdim=True).float()
        if norm == "l2":
            n = ss.sqrt()
            den = n + 1e-5
            coef = torch.where(n > 0, dot / (n * den * den), torch.zeros_like(n))
            gs = gr / den - sr * coef
        else:
            r = torch.rsqrt(ss / D + 1e-5)
            gs = r * gr - sr * (dot * r * r * r / D)
        gg = gs.reshape(B, Lx, Fdim).to(dt).float()
    if silu:
        sg = torch.sigmoid(xf)
        gg = gg * (sg * (1 + xf * (1 - sg)))
    return gg.to(dt)


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

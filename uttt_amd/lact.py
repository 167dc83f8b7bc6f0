"""Single-layer LaCT with the prenorm write, on the gfx950 kernels.

Reference (cited T:line):
uttt_nvs/models/kernels/ttt_operation.py:217-367,
prenorm_block_causal_lact_swiglu -- the shifted block-causal test-time
training loop of one layer: every chunk is read with the current fast weights
(apply), then the chunk's k / v / lr update them (UPDATE, optional momentum
and Muon), and the new weights are projected per row back onto the row norms
the weights had at the start of the sequence (the prenorm write).  The last
chunk is read and never written.

Kernels per chunk: the grouped APPLY (E = 1 per batch row), the grouped
UPDATE, uttt_momentum_add and uttt_newton_schulz5 when asked, and
uttt_write_prenorm for the write, whose sequence-start norms come from
uttt_row_norms.  w0 and w2 are kept packed as the grouped kernels take them
([b, 1, 2 d_h, d]): their rows are written in one launch and orthogonalised
as 2b separate matrices.  Forward only (no autograd through the loop).
"""
from __future__ import annotations

import torch

from . import _lib as L
from .fast_weight_write import newton_schulz5
from .lact_moe_triton.lact_fw_grad import grouped_lact_swiglu_ffn_fast_weight_grads
from .lact_moe_triton.lact_swiglu_ffn import grouped_swiglu_ffn_fwd


def row_norms(w: torch.Tensor) -> torch.Tensor:
    """|row| over the last dimension in fp32 (T:258-260): w [..., C] -> [...]."""
    L.require_device(w)
    w = w.contiguous()
    C = w.shape[-1]
    out = torch.empty(w.shape[:-1], dtype=torch.float32, device=w.device)
    L.call("uttt_row_norms", L.ptr(w), L.dtype_code(w.dtype), w.numel() // C, C, L.ptr(out),
           L.stream_of(w))
    return out


def write_prenorm(main: torch.Tensor, grad: torch.Tensor, norms: torch.Tensor,
                  fast_out: torch.Tensor) -> None:
    """T:341-353 in place: main += grad (fp32); fast_out = bf16(main / (|main|
    + 1e-5) * norms) row by row (norms: the sequence-start row norms)."""
    L.require_device(main, grad, norms, fast_out)
    assert main.dtype == torch.float32 and main.is_contiguous()
    assert grad.shape == main.shape and fast_out.shape == main.shape
    assert fast_out.dtype == torch.bfloat16 and fast_out.is_contiguous()
    C = main.shape[-1]
    assert norms.dtype == torch.float32 and norms.numel() == main.numel() // C
    grad = grad.contiguous()
    L.call("uttt_write_prenorm", L.ptr(main), L.ptr(grad), L.dtype_code(grad.dtype),
           L.ptr(norms.contiguous()), main.numel() // C, C, L.ptr(main), L.ptr(fast_out),
           L.stream_of(main))


def _momentum_step(g, mom, coeff_b):
    """g + mom * coeff_b[b] (fp32): the new momentum buffer (T:318-327)."""
    out = torch.empty(g.shape, dtype=torch.float32, device=g.device)
    B = g.shape[0]
    L.call("uttt_momentum_add", L.ptr(g), L.dtype_code(g.dtype), L.ptr(mom), L.ptr(coeff_b), B,
           g.numel() // B, L.ptr(out), L.stream_of(g))
    return out


@torch.no_grad()
def prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, lr0, lr1, lr2,
                                     chunk_size: int = 2048, kv_repeat: int = 1,
                                     use_muon: bool = False, momentum=None,
                                     return_weights: bool = False):
    """T:217-367 with the same arguments: w0, w2 [b, d_h, d], w1 [b, d, d_h]
    (any float dtype), q [b, l, d], k and v [b, l * kv_repeat, d], lr0, lr1,
    lr2 [b, l * kv_repeat, 1], momentum [b, l, 1] or None.  The key and value
    widths must be equal (one d for the grouped kernels).  Returns the output
    [b, l, d] in bf16 (and, with return_weights, the final (w0, w1, w2)
    bf16 fast weights and fp32 main weights)."""
    b, dh, d = w0.shape
    assert w2.shape == w0.shape and tuple(w1.shape) == (b, d, dh), "w1 must be [b, d, d_h]"
    seq = q.shape[1]
    assert q.shape == (b, seq, d) and k.shape == (b, seq * kv_repeat, d) and v.shape == k.shape
    L.require_device(w0, w1, w2, q, k, v, lr0, lr1, lr2)
    dev = q.device
    # fp32 main weights and their sequence-start row norms (T:258-262); w0 | w2 packed
    main02 = torch.cat([w0, w2], dim=1).float().contiguous()        # [b, 2 d_h, d]
    main1 = w1.float().contiguous()                                   # [b, d, d_h]
    norms02, norms1 = row_norms(main02), row_norms(main1)
    W02 = main02.to(torch.bfloat16).reshape(b, 1, 2 * dh, d).contiguous()
    W1 = main1.to(torch.bfloat16).reshape(b, 1, d, dh).contiguous()
    mom02 = mom1 = None
    if momentum is not None:
        mom02 = torch.zeros_like(main02)
        mom1 = torch.zeros_like(main1)
    out = torch.empty(b, seq, d, dtype=torch.bfloat16, device=dev)
    qb = q.to(torch.bfloat16)
    kb = k.to(torch.bfloat16)
    vb = v.to(torch.bfloat16)

    def gs(n):
        return torch.full((b, 1), n, dtype=torch.int32, device=dev)

    def read(s, e):
        out[:, s:e] = grouped_swiglu_ffn_fwd(W02, W1, qb[:, s:e].contiguous(), gs(e - s))

    e = 0
    for s in range(0, seq - chunk_size, chunk_size):
        e = s + chunk_size
        read(s, e)                                                    # T:290-295
        ks, ke = s * kv_repeat, e * kv_repeat
        lrs = [x[:, ks:ke].reshape(b, ke - ks).contiguous() for x in (lr0, lr1, lr2)]
        dW02, dW1 = grouped_lact_swiglu_ffn_fast_weight_grads(        # T:297-316
            W02, W1, kb[:, ks:ke].contiguous(), vb[:, ks:ke].contiguous(), *lrs, gs(ke - ks))
        g02 = dW02.reshape(b, 2 * dh, d)
        g1 = dW1.reshape(b, d, dh)
        if momentum is not None:                                      # T:318-327
            m_i = momentum[:, s:e].float().mean(dim=1).reshape(b).contiguous()
            g02 = mom02 = _momentum_step(g02, mom02, m_i)
            g1 = mom1 = _momentum_step(g1, mom1, m_i)
        if use_muon:                                                  # T:329-332, per matrix
            g1 = newton_schulz5(g1)
            g02 = newton_schulz5(g02.reshape(2 * b, dh, d)).reshape(b, 2 * dh, d)
        write_prenorm(main02, g02, norms02, W02.view(b, 2 * dh, d))   # T:341-353
        write_prenorm(main1, g1, norms1, W1.view(b, d, dh))
    read(e, seq)                                                      # T:355-365
    if not return_weights:
        return out
    fast = (W02[:, 0, :dh], W1[:, 0], W02[:, 0, dh:])
    mains = (main02[:, :dh], main1, main02[:, dh:])
    return out, fast, mains

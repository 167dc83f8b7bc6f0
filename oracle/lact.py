"""Oracle of the single-layer LaCT with the prenorm write (checker only; see
oracle/__init__.py).

Restates prenorm_block_causal_lact_swiglu,
uttt_nvs/models/kernels/ttt_operation.py:217-367 (cited T:), in torch on the
CPU.  The reference runs under autocast bf16, so every bmm takes bf16
operands, accumulates in fp32 and returns bf16 (_bmm below); the elementwise
chains between the bmms are fp32 (one fused compiled region each) and are
rounded to bf16 where a bmm consumes them; the main weights, the momentum and
the projection are fp32.  exact=True runs everything in fp64 without any
rounding (for the autograd and invariant pins).

  chunk_grads  T:297-316: (dw0, dw1, dw2) of one chunk from the current
               weights and the chunk's k, v, lr
  prenorm_block_causal_lact_swiglu  T:217-367; returns the output, and the
               final fast / main weights
"""
from __future__ import annotations

import torch

from . import write as OW


def _bmm(a, b, exact):
    if exact:
        return torch.bmm(a.double(), b.double())
    return torch.bmm(a.to(torch.bfloat16).float(), b.to(torch.bfloat16).float()).to(torch.bfloat16)


def _r(x, exact):
    """Where the reference materialises a bf16 tensor (a bmm operand)."""
    return x.double() if exact else x.to(torch.bfloat16)


def _read(w0, w1, w2, qT, exact):
    """T:290-295: w1 (silu(w0 q) * (w2 q)) on qT [b, d, l] -> [b, d, l]."""
    h = _bmm(w2, qT, exact).float() if not exact else _bmm(w2, qT, exact)
    g0 = _bmm(w0, qT, exact)
    g0 = g0.float() if not exact else g0
    gate = g0 * torch.sigmoid(g0)
    return _bmm(w1, _r(gate * h, exact), exact)


def chunk_grads(w0, w1, w2, k, vT, lr0, lr1, lr2, exact=False):
    """T:297-316.  k [b, n, d], vT [b, d, n], lr* [b, n, 1] -> (dw0, dw1, dw2)
    [b, d_h, d], [b, d, d_h], [b, d_h, d] (bf16 unless exact)."""
    if exact:
        w0, w1, w2, k, vT, lr0, lr1, lr2 = (t.double() for t in (w0, w1, w2, k, vT, lr0, lr1, lr2))
    kT = k.transpose(1, 2)
    gba = _bmm(w0, kT, exact)                       # gate_before_act
    hbm = _bmm(w2, kT, exact)                       # hidden_before_mul
    dhid = _bmm(w1.transpose(1, 2), vT, exact)      # dhidden
    f = (lambda t: t) if exact else (lambda t: t.float())
    gba, hbm, dhid = f(gba), f(hbm), f(dhid)
    sg = torch.sigmoid(gba)
    silu = gba * sg
    hidden = silu * hbm
    dhbm = dhid * silu                              # dhidden_before_mul
    dgate = dhid * hbm
    dgba = dgate * sg * (1 + gba * (1 - sg))        # silu_backprop, ttt_operation.py:4-15
    dw1 = _bmm(vT, _r(hidden.transpose(1, 2) * f(lr1), exact), exact)
    dw0 = _bmm(_r(dgba, exact), _r(k * f(lr0), exact), exact)
    dw2 = _bmm(_r(dhbm, exact), _r(k * f(lr2), exact), exact)
    return dw0, dw1, dw2


def prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, lr0, lr1, lr2, chunk_size=2048,
                                     kv_repeat=1, use_muon=False, momentum=None, exact=False):
    """T:217-367.  Returns (output [b, l, d_v] (bf16 unless exact),
    final fast (w0, w1, w2), final main (w0, w1, w2))."""
    dt = torch.float64 if exact else torch.float32
    seq = q.shape[1]
    ws = [w.to(dt) for w in (w0, w1, w2)]
    norms = [w.double().norm(dim=2, keepdim=True).to(dt) for w in ws]      # T:258-260
    mains = [w.clone() for w in ws]                                        # T:262
    moms = [torch.zeros_like(w) for w in ws] if momentum is not None else None
    qT = q.transpose(1, 2)
    vT = v.transpose(1, 2)
    out = torch.zeros(q.shape[0], v.shape[2], seq, dtype=torch.float64 if exact else torch.bfloat16)
    e = 0
    for s in range(0, seq - chunk_size, chunk_size):                       # T:273
        e = s + chunk_size
        ks, ke = s * kv_repeat, e * kv_repeat
        out[:, :, s:e] = _read(ws[0], ws[1], ws[2], qT[:, :, s:e], exact)
        dws = chunk_grads(ws[0], ws[1], ws[2], k[:, ks:ke], vT[:, :, ks:ke],
                          lr0[:, ks:ke], lr1[:, ks:ke], lr2[:, ks:ke], exact)
        if momentum is not None:                                           # T:318-327
            m_i = momentum[:, s:e].to(dt).mean(dim=1, keepdim=True)
            dws = [dw.to(dt) + mo * m_i for dw, mo in zip(dws, moms)]
            moms = dws
        if use_muon:                                                       # T:329-332
            dws = [OW.newton_schulz5(dw) for dw in dws]
        mains = [m + dw.to(dt) for m, dw in zip(mains, dws)]               # T:346-348
        ws = [m / (m.double().norm(dim=2, keepdim=True).to(dt) + 1e-5) * n   # T:351-353
              for m, n in zip(mains, norms)]
    out[:, :, e:seq] = _read(ws[0], ws[1], ws[2], qT[:, :, e:seq], exact)  # T:355-365
    return out.transpose(1, 2), tuple(ws), tuple(mains)

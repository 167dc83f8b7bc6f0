"""Oracle of the uTTT-Dense fast-weight path (checker only; see
oracle/__init__.py).  fp32 torch on the CPU, restating
uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py (cited D:):

  read            _apply_fast_weights  D:241-268   out = w1 (silu(w0 x) * (w2 x))
                                                   per fast-weight head
  compute_update  compute_update       D:333-449   raw dW of the lr-weighted
                                                   dot-product loss per head,
                                                   stored bf16 then widened
  sweep           the chunk loop D:1801-1863 with _aggregate_memory_update
                  D:1302-1386 and _apply_shared_update D:1109-1240: every
                  layer reads a chunk with the chunk-start snapshot; all but
                  the last chunk are then written once from the mean (or sum)
                  of the layers' raw updates.

Only the fast-weight path is restated: the layers' q, k, v and lr are inputs
(the q/k/v projections, normalisations and rotary embedding that produce
them sit outside the path), and momentum / Muon are left out (no Muon is
built; momentum is covered by oracle/write.py).

Heads: x [b, l, H*d] is split into H heads of width d; w0, w2 [b, H, d_h, d],
w1 [b, H, d, d_h].  `exact=False` keeps the reference's bf16 storage points
(GEMM outputs bf16 under autocast); the arithmetic between them is fp32.
"""
from __future__ import annotations

import torch

from . import fastweight as FW
from . import write as OW


def _heads(x, H):
    b, l, hd = x.shape
    return x.reshape(b, l, H, hd // H).permute(0, 2, 1, 3).reshape(b * H, l, hd // H)


def _unheads(x, b, H):
    bh, l, d = x.shape
    return x.reshape(b, H, l, d).permute(0, 2, 1, 3).reshape(b, l, H * d)


def _ones_gs(B, N):
    return torch.full((B, 1), N, dtype=torch.int32)


def read(x, w0, w1, w2, exact=False):
    """D:241-268.  x [b, l, H*d]; returns [b, l, H*d] (bf16 unless exact).
    One head is one E = 1 group of the grouped apply."""
    b, H = w0.shape[:2]
    xh = _heads(x, H)
    W02 = torch.cat([w0, w2], dim=2).reshape(b * H, 1, 2 * w0.shape[2], w0.shape[3])
    W1 = w1.reshape(b * H, 1, w1.shape[2], w1.shape[3])
    if not exact:
        xh, W02, W1 = xh.to(torch.bfloat16), W02.to(torch.bfloat16), W1.to(torch.bfloat16)
    out = FW.swiglu_ffn_fwd(W02, W1, xh, _ones_gs(b * H, xh.shape[1]), exact=exact)
    return _unheads(out, b, H)


def _lr_heads(lr, b, l, H):
    """D:381-398: lr [b, l, 3] (shared by the heads) or [b, l, H*3]."""
    if lr.shape[2] == 3:
        lr = lr.unsqueeze(2).expand(b, l, H, 3)
    else:
        lr = lr.reshape(b, l, H, 3)
    lr = lr.permute(0, 2, 1, 3).reshape(b * H, l, 3)
    return lr[..., 0], lr[..., 1], lr[..., 2]


def compute_update(k, v, lr, fastw, exact=False):
    """D:333-449 (after the q/k/v preprocessing): per head the UPDATE
    dW0 = DY0 diag(lr0) K, dW2 = DY2 diag(lr2) K, dW1 = V^T diag(lr1) Hid^T,
    bf16 then fp32.  Returns (dw0 [b,H,d_h,d], dw1 [b,H,d,d_h], dw2)."""
    w0, w1, w2 = fastw
    b, H, dh, d = w0.shape
    l = k.shape[1]
    kh, vh = _heads(k, H), _heads(v, H)
    l0, l1, l2 = _lr_heads(lr, b, l, H)
    W02 = torch.cat([w0, w2], dim=2).reshape(b * H, 1, 2 * dh, d)
    W1 = w1.reshape(b * H, 1, d, dh)
    if not exact:
        kh, vh, W02, W1 = (t.to(torch.bfloat16) for t in (kh, vh, W02, W1))
    dw02, dw1 = FW.fast_weight_grads(W02, W1, kh, vh, l0, l1, l2, _ones_gs(b * H, l), exact=exact)
    dw02 = dw02.float().reshape(b, H, 2 * dh, d)
    return dw02[:, :, :dh], dw1.float().reshape(b, H, d, dh), dw02[:, :, dh:]


def sweep(qs, ks, vs, lrs, fastw, masterw, r, chunk, lr_scale=1.0, reduce="mean",
          master_renorm=False, exact=False):
    """D:1801-1863 with the aggregate write.  qs, ks, vs: per layer [b, S, H*d];
    lrs: per layer [b, S, 3]; fastw (bf16) / masterw (fp32): (w0, w1, w2).
    Returns (outputs per layer [b, S, H*d], final fast weights, final masters)."""
    L = len(qs)
    S = qs[0].shape[1]
    outs = [[] for _ in range(L)]
    fastw, masterw = tuple(fastw), tuple(masterw)
    for c0 in range(0, S, chunk):
        c1 = min(c0 + chunk, S)
        for li in range(L):
            outs[li].append(read(qs[li][:, c0:c1], *fastw, exact=exact))
        if c1 >= S:
            break   # the last chunk is read, never written
        agg = None
        for li in range(L):
            g = compute_update(ks[li][:, c0:c1], vs[li][:, c0:c1], lrs[li][:, c0:c1], fastw,
                               exact=exact)
            agg = list(g) if agg is None else [a + x for a, x in zip(agg, g)]
        if reduce == "mean":
            agg = [a / float(L) for a in agg]
        fastw, masterw, _ = OW.dense_write(agg, fastw, masterw, r, lr_scale=lr_scale,
                                           master_renorm=master_renorm)
    return [torch.cat(o, dim=1) for o in outs], fastw, masterw

"""The fast-weight WRITE step on the gfx950 kernel of csrc/write_step.hip.

Functions with the argument meaning and return values of the reference's
write methods (self's configuration becomes keyword arguments):

  apply_moe_update_dense    _apply_moe_update_dense,
                            uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:754-825
  apply_moe_update_packed   the same write on the packed [B,E,2I,D] pool
  apply_shared_update       _apply_shared_update,
                            uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py:1109-1240
  apply_raw_update          the NVS block's write, apply_raw_update,
                            uttt_nvs/models/uttt_moe_block.py:665-714 (unit rows)

They return freshly allocated (fast bf16, master fp32, momentum) tuples and
never modify their inputs, as the reference does.  With use_moun the step is
orthogonalised between the momentum and the write (newton_schulz5 below):
the momentum runs on its own kernel, Newton-Schulz on the grouped GEMMs, and
the write takes the bf16 result with the step size already applied, as the
reference's bf16 `g * lr_scale` is.
"""
from __future__ import annotations

import torch

from . import _lib as L

_NAMES = ("w0", "w1", "w2")


def _write_one(master, grad, mom, m_coeff_b, lr_scale, rows, C, seg, fast_in, renorm_master):
    L.require_device(master, grad, mom, m_coeff_b, fast_in)
    assert master.dtype == torch.float32 and master.is_contiguous(), "master must be fp32 contiguous"
    assert grad.shape == master.shape and grad.is_contiguous(), "grad must match the master"
    B = master.shape[0]
    master_out = torch.empty_like(master)
    fast_out = torch.empty(master.shape, dtype=torch.bfloat16, device=master.device)
    mom_out = None
    if mom is not None:
        assert mom.dtype == torch.float32 and mom.shape == master.shape and mom.is_contiguous()
        mom_out = torch.empty_like(mom)
    if fast_in is not None:
        assert fast_in.dtype == torch.bfloat16 and fast_in.shape == master.shape
        fast_in = fast_in.contiguous()
    L.call("uttt_write_step", L.ptr(master), L.ptr(fast_in), L.ptr(grad), L.dtype_code(grad.dtype),
           L.ptr(mom), L.ptr(m_coeff_b), float(lr_scale), B, rows, C, seg,
           int(fast_in is not None), int(renorm_master), L.ptr(master_out), L.ptr(fast_out),
           L.ptr(mom_out), L.stream_of(master))
    return fast_out, master_out, mom_out


def newton_schulz5(G, out_scale=1.0):
    """zeropower_via_newtonschulz5 (uttt_llm/flame/custom_models/uttt_moe/
    ttt_operation.py:19-46) on the gfx950 kernels: G [n, R, C] fp32 or bf16 ->
    bf16(NS5(G) * out_scale) [n, R, C]."""
    L.require_device(G)
    assert G.dim() == 3, "G must be [n, R, C]"
    assert G.dtype in (torch.float32, torch.bfloat16), "G must be fp32 or bf16"
    G = G.contiguous()
    n, R, C = G.shape
    out = torch.empty((n, R, C), dtype=torch.bfloat16, device=G.device)
    nbytes = L.lib().uttt_newton_schulz5_workspace_bytes(n, R, C)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=G.device)
    L.call("uttt_newton_schulz5", L.ptr(G), L.dtype_code(G.dtype), n, R, C, float(out_scale),
           L.ptr(out), L.ptr(ws), nbytes, L.stream_of(G))
    return out


def _momentum(g, mom, coeff_b):
    """g + mom * m_coeff[b] (fp32), the new momentum buffer."""
    L.require_device(g, mom, coeff_b)
    g, mom = g.contiguous(), mom.contiguous()
    assert mom.dtype == torch.float32 and mom.shape == g.shape
    out = torch.empty(g.shape, dtype=torch.float32, device=g.device)
    B = g.shape[0]
    L.call("uttt_momentum_add", L.ptr(g), L.dtype_code(g.dtype), L.ptr(mom), L.ptr(coeff_b), B,
           g.numel() // max(B, 1), L.ptr(out), L.stream_of(g))
    return out


def _coeff_per_batch(m_coeff, B, device):
    c = m_coeff.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    assert c.numel() == B, f"momentum coefficient must hold one value per batch, got {c.numel()}"
    return c


def apply_moe_update_dense(grads, fastw, masterw, momentum_buf=None, m_coeff=None, lr_scale=1.0,
                           use_momentum=True, use_moun=False):
    """uTTT-MoE write (modeling_recurrent_lact.py:754-825).  grads, masterw:
    (w0, w1, w2) [B,E,R,C] (grads fp32 or bf16, masters fp32); momentum_buf:
    fp32 tuple or None; m_coeff: [B,1,1,1] or None.  `fastw` is accepted for
    signature parity; the new fast weights are bf16 of the new masters.
    Returns (fast, master, momentum_buf)."""
    del fastw
    use_mom = use_momentum and momentum_buf is not None and m_coeff is not None
    B = masterw[0].shape[0]
    coeff = _coeff_per_batch(m_coeff, B, masterw[0].device) if use_mom else None
    fast, master, mom = [], [], []
    for i, (g, w) in enumerate(zip(grads, masterw)):
        assert w.dim() == 4, "masters are [B, E, R, C]"
        _, E, R, C = w.shape
        if use_moun:                               # M:781-810, then M:813-815
            if use_mom:
                g = _momentum(g, momentum_buf[i], coeff)
                mom.append(g)
            step = newton_schulz5(g.reshape(B * E, R, C), lr_scale).reshape(g.shape)
            f, m, _ = _write_one(w.contiguous(), step, None, None, 1.0, E * R, C, C, None, True)
        else:
            f, m, mo = _write_one(w.contiguous(), g.contiguous(),
                                  momentum_buf[i].contiguous() if use_mom else None, coeff,
                                  lr_scale, E * R, C, C, None, True)
            mom.append(mo)
        fast.append(f)
        master.append(m)
    return tuple(fast), tuple(master), (tuple(mom) if use_mom else momentum_buf)


def apply_moe_update_packed(dW0_W2, dW1, M0_W2, M1, momentum_buf=None, m_coeff=None,
                            lr_scale=1.0, use_momentum=True, use_moun=False, out=None):
    """apply_moe_update_dense on the packed pool: dW0_W2 / M0_W2 [B,E,2I,D]
    (w0 rows then w2 rows of each expert, the layout the grouped kernels
    read), dW1 / M1 [B,E,D,I].  The write is per row and Newton-Schulz per
    [I, D] matrix, so the result is the three-matrix write's (M:754-825)
    without splitting or concatenating the pool.  momentum_buf: (mom0_w2,
    mom1) fp32 or None.  Returns ((fast0_w2, fast1) bf16, (master0_w2,
    master1) fp32, momentum_buf).  out: optional ((fast0_w2, fast1),
    (master0_w2, master1)) to write in place of new tensors (masters may be
    the inputs: each row is read before it is written)."""
    use_mom = use_momentum and momentum_buf is not None and m_coeff is not None
    B = M0_W2.shape[0]
    coeff = _coeff_per_batch(m_coeff, B, M0_W2.device) if use_mom else None
    fast, master, mom = [], [], []
    for i, (g, w) in enumerate(((dW0_W2, M0_W2), (dW1, M1))):
        assert w.dim() == 4 and w.dtype == torch.float32 and w.is_contiguous(), \
            "masters are contiguous fp32 [B, E, R, C]"
        assert g.shape == w.shape, "gradient must match the master"
        _, E, R, C = w.shape
        fo = mo_ = None
        if out is not None:
            fo, mo_ = out[0][i], out[1][i]
            assert fo.dtype == torch.bfloat16 and fo.shape == w.shape and fo.is_contiguous()
            assert mo_.dtype == torch.float32 and mo_.shape == w.shape and mo_.is_contiguous()
        if use_moun:
            if use_mom:
                g = _momentum(g, momentum_buf[i], coeff)
                mom.append(g)
            nmat = B * E * (2 if i == 0 else 1)    # w0 and w2 are separate matrices
            step = newton_schulz5(g.reshape(nmat, R * B * E // nmat, C), lr_scale).reshape(g.shape)
            g_use, mom_in, cb, scale = step, None, None, 1.0
        else:
            g_use = g.contiguous()
            mom_in, cb, scale = (momentum_buf[i].contiguous() if use_mom else None), coeff, lr_scale
        f, m, mo = _write_into(w, g_use, mom_in, cb, scale, E * R, C, fo, mo_)
        if not use_moun and use_mom:
            mom.append(mo)
        fast.append(f)
        master.append(m)
    return tuple(fast), tuple(master), (tuple(mom) if use_mom else momentum_buf)


def _write_into(master, grad, mom, m_coeff_b, lr_scale, rows, C, fast_out=None, master_out=None):
    """_write_one with optional caller-provided outputs (norm-preserving
    master renorm, norms from the master)."""
    L.require_device(master, grad, mom, m_coeff_b)
    B = master.shape[0]
    master_out = torch.empty_like(master) if master_out is None else master_out
    fast_out = (torch.empty(master.shape, dtype=torch.bfloat16, device=master.device)
                if fast_out is None else fast_out)
    mom_out = torch.empty_like(mom) if mom is not None else None
    L.call("uttt_write_step", L.ptr(master), None, L.ptr(grad), L.dtype_code(grad.dtype),
           L.ptr(mom), L.ptr(m_coeff_b), float(lr_scale), B, rows, C, C, 0, 1,
           L.ptr(master_out), L.ptr(fast_out), L.ptr(mom_out), L.stream_of(master))
    return fast_out, master_out, mom_out


def apply_shared_update(agg_grads, fastw, masterw, momentum_buf=None, momentum_coeffs=None, *,
                        r: int, lr_scale: float = 1.0, master_renorm: bool = False,
                        use_momentum: bool = True, use_moun: bool = False):
    """uTTT-Dense write (modeling_recurrent_lact.py:1109-1240).  Shapes: w0, w2
    [b,h,r*d,d], w1 [b,h,d,r*d]; every d x d slice is written on its own, so a
    w1 row is cut into r segments of d.  momentum_coeffs: a tensor, a list of
    per-layer tensors (averaged) or None.  Returns (fast, master, momentum_buf)."""
    if len(agg_grads) != 3 or len(fastw) != 3 or len(masterw) != 3:
        raise ValueError("uTTT-Dense expects three fast-weight matrices")
    b, h, inter, d = fastw[0].shape
    if inter != r * d or tuple(fastw[1].shape) != (b, h, d, r * d) or fastw[2].shape != fastw[0].shape:
        raise ValueError(f"invalid shared fast state shapes for r={r}: "
                         f"{[tuple(w.shape) for w in fastw]}")
    if torch.is_tensor(momentum_coeffs):
        coeff = momentum_coeffs
    elif momentum_coeffs:
        coeff = torch.stack(list(momentum_coeffs), dim=0).mean(dim=0)
    else:
        coeff = None
    use_mom = use_momentum and momentum_buf is not None and coeff is not None
    cb = _coeff_per_batch(coeff, b, fastw[0].device) if use_mom else None
    fast, master, mom = [], [], []
    for i, name in enumerate(_NAMES):
        w = masterw[i].contiguous()
        rows, C = (h * r * d, d) if name != "w1" else (h * d, r * d)
        norm_src = None if master_renorm else fastw[i]
        if use_moun:                               # D:1175-1185, D:1192-1209
            g = agg_grads[i]
            if use_mom:
                g = _momentum(g, momentum_buf[i], cb)
                mom.append(g)
            step = _slices_to_wide(newton_schulz5(_wide_to_slices(g, name, r), lr_scale),
                                   name, b, h, r)
            f, m, _ = _write_one(w, step, None, None, 1.0, rows, C, d, norm_src, master_renorm)
        else:
            f, m, mo = _write_one(w, agg_grads[i].contiguous(),
                                  momentum_buf[i].contiguous() if use_mom else None, cb, lr_scale,
                                  rows, C, d, norm_src, master_renorm)
            mom.append(mo)
        fast.append(f)
        master.append(m)
    return tuple(fast), tuple(master), (tuple(mom) if use_mom else momentum_buf)


def _wide_to_slices(x, name, r):
    """D:1068-1086 layout: [b,h,r*d,d] (w0, w2) or [b,h,d,r*d] (w1) -> [b*h*r, d, d]
    (a copy for w1, whose slices are column blocks)."""
    if name != "w1":
        b, h, inter, d = x.shape
        return x.reshape(b * h * r, d, d)
    b, h, d, inter = x.shape
    return x.reshape(b, h, d, r, d).permute(0, 1, 3, 2, 4).reshape(b * h * r, d, d)


def _slices_to_wide(s, name, b, h, r):
    """D:1088-1106, the inverse of _wide_to_slices (contiguous)."""
    d = s.shape[-1]
    if name != "w1":
        return s.reshape(b, h, r * d, d)
    return s.reshape(b, h, r, d, d).permute(0, 1, 3, 2, 4).reshape(b, h, d, r * d).contiguous()


def _group_stride(t, name):
    """Group stride of a [b, e, R, C] tensor whose rows are contiguous and
    whose b*e groups sit at one stride (a whole tensor, or the w0 / w2 half
    of a packed [b, e, 2I, C] tensor)."""
    assert t.dim() == 4, f"{name} must be [b, e, R, C]"
    b, e, R, C = t.shape
    assert t.stride(3) == 1 and (R <= 1 or t.stride(2) == C), f"{name}: rows must be contiguous"
    assert b <= 1 or t.stride(0) == e * t.stride(1), f"{name}: groups must sit at one stride"
    return t.stride(1) if e > 1 else (t.stride(0) if b > 1 else R * C)


def _unit_rows_into(master, grad, fast_view):
    """master + grad -> (new master, unit rows written into fast_view)."""
    L.require_device(master, grad, fast_view)
    assert master.dtype == torch.float32 and master.is_contiguous(), "masters must be contiguous fp32"
    assert grad.shape == master.shape and fast_view.shape == master.shape, "shape mismatch"
    assert fast_view.dtype == torch.bfloat16
    b, e, R, C = master.shape
    out = torch.empty_like(master)
    L.call("uttt_write_unit_rows", L.ptr(master), R * C, L.ptr(grad), L.dtype_code(grad.dtype),
           _group_stride(grad, "grad"), b * e, R, C, L.ptr(out), R * C, L.ptr(fast_view),
           _group_stride(fast_view, "fast"), L.stream_of(master))
    return out


def apply_raw_update(raw_grads, masterw, *, inter_dim, use_muon=False):
    """NVS write, apply_raw_update (uttt_nvs/models/uttt_moe_block.py:665-714),
    with self.inter_dim and self.use_muon as keyword arguments.

    raw_grads: (dw0_w2 [b,e,2I,D], dw1 [b,e,D,I]) packed, or (dw0, dw1, dw2);
    fp32 (or bf16) gradients, summed over writers, with the step size already
    in them.  masterw: (w0, w1, w2) fp32 masters.  No momentum and no
    norm-preserving projection: master' = master + step (step = the gradient,
    or its Newton-Schulz orthogonalisation per expert matrix when use_muon),
    and the fast weights are bf16 unit rows of master' (F.normalize over the
    last dim, clamped at 1e-5).  Returns (new_fastw, new_masterw):
    new_fastw = (fast0_w2 [b,e,2I,D], fast1) for packed gradients (the
    reference's torch.cat, written in place here), else three matrices."""
    w0, w1, w2 = masterw
    if len(raw_grads) == 2:
        dw0_w2, dw1 = raw_grads
        b, e, two_i, D = dw0_w2.shape
        assert two_i == 2 * inter_dim, "dw0_w2 must hold 2 * inter_dim rows"
        if use_muon:                               # uttt_moe_block.py:674-678, w0 and w2 apart
            dw0_w2 = newton_schulz5(dw0_w2.contiguous().reshape(b * e * 2, inter_dim, D)
                                    ).reshape(b, e, two_i, D)
            dw1 = newton_schulz5(dw1.contiguous().reshape(b * e, *dw1.shape[2:])
                                 ).reshape(dw1.shape)
        fast02 = torch.empty((b, e, two_i, D), dtype=torch.bfloat16, device=w0.device)
        fast1 = torch.empty(w1.shape, dtype=torch.bfloat16, device=w1.device)
        m0 = _unit_rows_into(w0, dw0_w2[:, :, :inter_dim], fast02[:, :, :inter_dim])
        m2 = _unit_rows_into(w2, dw0_w2[:, :, inter_dim:], fast02[:, :, inter_dim:])
        m1 = _unit_rows_into(w1, dw1.contiguous(), fast1)
        return (fast02, fast1), (m0, m1, m2)
    if len(raw_grads) != 3:
        raise ValueError("raw_grads must be (dw0_w2, dw1) or (dw0, dw1, dw2)")
    fast, master = [], []
    for g, w in zip(raw_grads, masterw):
        g = g.contiguous()
        if use_muon:                               # uttt_moe_block.py:697-701
            g = newton_schulz5(g.reshape(-1, *g.shape[2:])).reshape(g.shape)
        f = torch.empty(w.shape, dtype=torch.bfloat16, device=w.device)
        master.append(_unit_rows_into(w, g, f))
        fast.append(f)
    return tuple(fast), tuple(master)

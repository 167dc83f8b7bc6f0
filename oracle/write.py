"""Oracle of the fast-weight WRITE step (checker only; see oracle/__init__.py).

fp32 torch on the CPU, written from the two reference call sites:

  moe_write    _apply_moe_update_dense,
               uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:754-825
               (cited M:).  Row norms over the last dim of the fp32 masters,
               taken before the step; optional momentum; W + s * G; the
               masters are projected back onto the old norms; fast = bf16.
  dense_write  _apply_shared_update and _wide_to_slices / _slices_to_wide,
               uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py:1068-1240
               (cited D:).  The same step on d x d slices: w0 / w2 rows are
               whole slice rows, w1 rows are cut into r segments of d; the old
               norms come from the fast (bf16) weights unless master renorm is
               on, and the master keeps the unprojected value unless master
               renorm is on.

  nvs_write    apply_raw_update, uttt_nvs/models/uttt_moe_block.py:665-714
               (cited V:).  master + raw gradient (no momentum, no step
               size), the master kept unprojected, fast = bf16 unit rows of
               the new master (F.normalize, clamped at 1e-5).

newton_schulz5  zeropower_via_newtonschulz5,
               uttt_llm/flame/custom_models/uttt_moe/ttt_operation.py:19-46 (cited N:),
               the Muon orthogonalisation both writes run between the momentum
               and the step when use_moun is on (M:781-810, D:1192-1203).  It
               is bf16 tensor arithmetic in the reference, so it is restated in
               bf16 torch on the CPU (bf16 matmuls accumulate in fp32 and round
               their result, like the GPU's), operation by operation.

Every operation follows the reference's operation order (separate multiply
and add, divide then multiply) in fp32; only the norm reductions differ in
summation order (the oracle sums in fp64), which the tests cover with a
1e-5 relative tolerance.
"""
from __future__ import annotations

import torch

EPS = 1e-5


def _norm(x: torch.Tensor, dim: int) -> torch.Tensor:
    return x.double().pow(2).sum(dim=dim, keepdim=True).sqrt().float()


# N:34-40, the per-step (a, b, c) coefficients
NS5_COEFFS = ((4.0848, -6.8946, 2.9270),
              (3.9505, -6.3029, 2.6377),
              (3.7418, -5.5913, 2.3037),
              (2.8769, -3.1427, 1.2046),
              (2.8366, -3.0525, 1.2012))


def newton_schulz5(G: torch.Tensor) -> torch.Tensor:
    """N:19-46.  G [n, R, C] (any float dtype) -> bf16 [n, R, C]."""
    assert G.dim() == 3
    X = G.to(torch.bfloat16)                               # N:31
    tr = G.size(1) > G.size(2)
    if tr:
        X = X.transpose(1, 2)                              # N:32-33
    X = X / (X.norm(dim=(1, 2), keepdim=True) + 1e-7)      # N:34
    for a, b, c in NS5_COEFFS:                             # N:35-44
        A = X @ X.transpose(1, 2)
        B = b * A + c * A @ A                              # i.e. b A + (c A) @ A
        X = a * X + B @ X
    if tr:
        X = X.transpose(1, 2)                              # N:45-46
    return X


def moe_write(grads, masterw, momentum_buf=None, m_coeff=None, lr_scale=1.0, use_moun=False):
    """M:754-825.  grads, masterw: (w0, w1, w2), fp32 [B,E,R,C]; momentum_buf:
    same shapes or None; m_coeff: [B,1,1,1] or None; use_moun: orthogonalise
    each expert's step with newton_schulz5 (then the step is bf16 and
    g * lr_scale is a bf16 product, as in the reference).
    Returns (fast bf16 tuple, new masters, new momentum or None)."""
    new_master, new_mom, fast = [], [], []
    use_mom = momentum_buf is not None and m_coeff is not None
    for i, (g, w) in enumerate(zip(grads, masterw)):
        w = w.float()
        nu = _norm(w, 3)                                   # M:766-768
        g = g.float()
        if use_mom:
            g = g + momentum_buf[i].float() * m_coeff      # M:772-774
            new_mom.append(g.clone())                      # M:775-779
        if use_moun:                                       # M:781-810
            B, E, R, C = g.shape
            g = newton_schulz5(g.reshape(B * E, R, C)).reshape(B, E, R, C)
        u = w + g * lr_scale                               # M:813-815
        p = u / (_norm(u, 3) + EPS) * nu                   # M:817-819
        new_master.append(p)
        fast.append(p.to(torch.bfloat16))                  # M:822
    return tuple(fast), tuple(new_master), (tuple(new_mom) if use_mom else momentum_buf)


def _unit_rows(u: torch.Tensor) -> torch.Tensor:
    """u / max(|u|, eps) over the last dim (F.normalize's clamped divide),
    the norm summed in fp64."""
    n = _norm(u, u.dim() - 1)
    return u / torch.where(n < EPS, torch.full_like(n, EPS), n)


def nvs_write(raw_grads, masterw, inter_dim, use_muon=False):
    """apply_raw_update, uttt_nvs/models/uttt_moe_block.py:665-714 (cited V:).
    raw_grads: (dw0_w2 [b,e,2I,D], dw1) packed (V:669-693) or (dw0, dw1, dw2)
    (V:695-714), fp32; masterw (w0, w1, w2) fp32.  No momentum and no step
    size: the masters take the raw (or orthogonalised) gradient and keep the
    unprojected sum; the fast weights are bf16 unit rows of the new masters.
    Returns (new fast, new masters): fast = (bf16 cat[w0, w2] rows, bf16 w1)
    for packed grads, else the three bf16 matrices."""
    if len(raw_grads) == 2:
        dw0_w2, dw1 = raw_grads
        dws = [dw0_w2[:, :, :inter_dim], dw1, dw0_w2[:, :, inter_dim:]]   # V:672-673
    else:
        dws = list(raw_grads)
    if use_muon:                                                           # V:674-678
        out = []
        for g in dws:
            b, e, r, c = g.shape
            out.append(newton_schulz5(g.reshape(b * e, r, c)).reshape(b, e, r, c))
        dws = out
    new_master = [w.float() + g.float() for w, g in zip(masterw, dws)]     # V:679-681
    unit = [_unit_rows(m).to(torch.bfloat16) for m in new_master]          # V:683-691
    if len(raw_grads) == 2:
        return (torch.cat([unit[0], unit[2]], dim=2), unit[1]), tuple(new_master)
    return tuple(unit), tuple(new_master)


def wide_to_slices(weight: torch.Tensor, name: str, r: int) -> torch.Tensor:
    """D:1068-1086: [b,h,r*d,d] (w0, w2) or [b,h,d,r*d] (w1) -> [b*h*r, d, d]."""
    if name in ("w0", "w2"):
        b, h, inter, d = weight.shape
        return weight.reshape(b, h, r, d, d).reshape(b * h * r, d, d)
    b, h, d, inter = weight.shape
    return weight.reshape(b, h, d, r, d).permute(0, 1, 3, 2, 4).reshape(b * h * r, d, d)


def slices_to_wide(slices: torch.Tensor, name: str, b: int, h: int, r: int) -> torch.Tensor:
    """D:1088-1106, the inverse of wide_to_slices."""
    _, d, _ = slices.shape
    if name in ("w0", "w2"):
        return slices.reshape(b, h, r * d, d)
    return slices.reshape(b, h, r, d, d).permute(0, 1, 3, 2, 4).reshape(b, h, d, r * d)


def dense_write(agg_grads, fastw, masterw, r, momentum_buf=None, coeff=None, lr_scale=1.0,
                master_renorm=False, use_moun=False):
    """D:1109-1240.  fastw bf16, masterw fp32, shapes w0/w2 [b,h,r*d,d], w1
    [b,h,d,r*d]; coeff: [b,1,1,1] or None; use_moun: orthogonalise each d x d
    slice of the step with newton_schulz5 (D:1192-1203).
    Returns (fast bf16 tuple, new masters, new momentum or None)."""
    names = ("w0", "w1", "w2")
    b, h = fastw[0].shape[:2]
    fast_s = [wide_to_slices(w, n, r) for n, w in zip(names, fastw)]
    master_s = [wide_to_slices(w.float(), n, r) for n, w in zip(names, masterw)]
    src = master_s if master_renorm else fast_s
    old = [_norm(s.float(), 2) for s in src]                           # D:1164-1167
    deltas = [g.float() for g in agg_grads]
    if momentum_buf is not None and coeff is not None:
        deltas = [dl + m.float() * coeff for dl, m in zip(deltas, momentum_buf)]  # D:1175-1178
        momentum_buf = tuple(deltas)
    delta_s = [wide_to_slices(dl, n, r) for n, dl in zip(names, deltas)]
    if use_moun:
        delta_s = [newton_schulz5(dl) for dl in delta_s]               # D:1192-1203
    delta_s = [dl * lr_scale for dl in delta_s]                        # D:1206-1209
    upd = [m + dl.to(m.dtype) for m, dl in zip(master_s, delta_s)]     # D:1210-1213
    proj = [u / (_norm(u, 2) + EPS) * o for u, o in zip(upd, old)]     # D:1214-1222
    if master_renorm:
        upd = proj
    new_master = tuple(slices_to_wide(s, n, b, h, r) for n, s in zip(names, upd))
    fast = tuple(slices_to_wide(s, n, b, h, r).to(torch.bfloat16) for n, s in zip(names, proj))
    return fast, new_master, momentum_buf

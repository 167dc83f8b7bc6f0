"""Pins of the WRITE-step oracle (oracle/write.py) by properties the
mathematics fixes, not by re-typing its formula:

* the projection restores every row (segment) norm to the pre-step norm, up to
  the 1e-5 epsilon;
* G = 0 leaves each row scaled by nu / (nu + eps); G = c W keeps the direction;
* G orthogonal to W: the new row makes the angle atan(s |G| / |W|) with the
  old one (Pythagoras), which pins the lr_scale factor and the sign of the step;
* momentum: a step with (G, M, m) equals a step with G + m M and no momentum,
  and the returned buffer is G + m M;
* the dense slice views: w1's slice (h, s) is the column block
  [s*d, (s+1)*d) of every row (checked against plain slicing), and the round
  trip wide -> slices -> wide is the identity.
"""
import math

import pytest
import torch

from oracle import write as OW


def _rownorm(x, dim=-1):
    return x.double().norm(dim=dim)


def _rand(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def test_moe_write_restores_row_norms():
    B, E, R, C = 2, 3, 5, 8
    masters = tuple(_rand(B, E, R, C, seed=i) for i in range(3))
    grads = tuple(_rand(B, E, R, C, seed=10 + i) * 0.3 for i in range(3))
    fast, new_m, mom = OW.moe_write(grads, masters, lr_scale=0.7)
    assert mom is None
    for w, p, f in zip(masters, new_m, fast):
        nu = _rownorm(w)
        torch.testing.assert_close(_rownorm(p), nu, rtol=1e-5, atol=1e-5)
        assert f.dtype == torch.bfloat16 and torch.equal(f, p.to(torch.bfloat16))


def test_moe_write_zero_and_parallel_steps():
    w = _rand(1, 1, 4, 16, seed=1)
    nu = w.norm(dim=-1, keepdim=True)
    zero = torch.zeros_like(w)
    _, (p0, _, _), _ = OW.moe_write((zero, zero, zero), (w, w, w), lr_scale=3.0)
    torch.testing.assert_close(p0, w * (nu / (nu + OW.EPS)), rtol=1e-6, atol=1e-7)
    _, (pc, _, _), _ = OW.moe_write((2.0 * w, zero, zero), (w, w, w), lr_scale=0.25)
    cos = (pc * w).sum(-1) / (pc.norm(dim=-1) * nu.squeeze(-1))
    torch.testing.assert_close(cos, torch.ones_like(cos), rtol=0, atol=1e-6)


@pytest.mark.parametrize("s", [0.5, 2.0])
def test_moe_write_orthogonal_step_angle(s):
    w = torch.zeros(1, 1, 2, 6)
    w[..., 0, 0] = 3.0
    w[..., 1, 2] = 1.5
    g = torch.zeros_like(w)
    g[..., 0, 1] = 4.0   # orthogonal to row 0
    g[..., 1, 5] = -2.0  # orthogonal to row 1
    _, (p, _, _), _ = OW.moe_write((g, g, g), (w, w, w), lr_scale=s)
    for row in range(2):
        wr, gr, pr = w[0, 0, row], g[0, 0, row], p[0, 0, row]
        ang = math.atan2((pr @ gr).item() / gr.norm().item(), (pr @ wr).item() / wr.norm().item())
        assert abs(ang - math.atan(s * gr.norm().item() / wr.norm().item())) < 1e-6


def test_moe_write_momentum_is_a_preadded_gradient():
    B, E, R, C = 2, 2, 3, 8
    masters = tuple(_rand(B, E, R, C, seed=i) for i in range(3))
    grads = tuple(_rand(B, E, R, C, seed=10 + i) for i in range(3))
    moms = tuple(_rand(B, E, R, C, seed=20 + i) for i in range(3))
    m = torch.tensor([0.3, -0.8]).view(B, 1, 1, 1)
    f1, p1, mom1 = OW.moe_write(grads, masters, moms, m, lr_scale=0.5)
    pre = tuple(g + mo * m for g, mo in zip(grads, moms))
    f2, p2, _ = OW.moe_write(pre, masters, lr_scale=0.5)
    for a, b_, c in zip(p1, p2, mom1):
        assert torch.equal(a, b_)
    for c, p in zip(mom1, pre):
        assert torch.equal(c, p)


def test_dense_slices_are_column_blocks():
    b, h, d, r = 2, 3, 4, 3
    w1 = _rand(b, h, d, r * d, seed=3)
    sl = OW.wide_to_slices(w1, "w1", r).reshape(b, h, r, d, d)
    for s in range(r):
        assert torch.equal(sl[:, :, s], w1[..., s * d:(s + 1) * d])
    w0 = _rand(b, h, r * d, d, seed=4)
    sl0 = OW.wide_to_slices(w0, "w0", r).reshape(b, h, r, d, d)
    for s in range(r):
        assert torch.equal(sl0[:, :, s], w0[:, :, s * d:(s + 1) * d])
    for name, w in (("w0", w0), ("w1", w1)):
        assert torch.equal(OW.slices_to_wide(OW.wide_to_slices(w, name, r), name, b, h, r), w)


@pytest.mark.parametrize("master_renorm", [False, True])
def test_dense_write_segment_norms(master_renorm):
    b, h, d, r = 1, 2, 8, 2
    master = (_rand(b, h, r * d, d, seed=1), _rand(b, h, d, r * d, seed=2), _rand(b, h, r * d, d, seed=3))
    fast = tuple((w * 1.01).to(torch.bfloat16) for w in master)
    grads = tuple(_rand(*w.shape, seed=5 + i) * 0.2 for i, w in enumerate(master))
    nf, nm, _ = OW.dense_write(grads, fast, master, r, lr_scale=0.9, master_renorm=master_renorm)
    src = master if master_renorm else tuple(f.float() for f in fast)
    for i, name in enumerate(("w0", "w1", "w2")):
        seg_old = OW.wide_to_slices(src[i].float(), name, r).norm(dim=2)
        # the fast weight is the step U = master + s G projected onto the old
        # segment norms: same direction as U, segment norms restored
        u = OW.wide_to_slices(master[i] + grads[i] * 0.9, name, r)
        pf = OW.wide_to_slices(nf[i].float(), name, r)
        torch.testing.assert_close(pf.norm(dim=2), seg_old, rtol=1e-2, atol=0)
        cos = (pf * u).sum(2) / (pf.norm(dim=2) * u.norm(dim=2))
        torch.testing.assert_close(cos, torch.ones_like(cos), rtol=0, atol=1e-4)
        if master_renorm:
            torch.testing.assert_close(OW.wide_to_slices(nm[i], name, r).norm(dim=2), seg_old,
                                       rtol=1e-5, atol=1e-5)
            assert torch.equal(nf[i], nm[i].to(torch.bfloat16))
        else:
            assert torch.equal(nm[i], master[i] + grads[i] * 0.9)


# ---- NVS unit-row write (oracle/write.nvs_write) ----

def _nvs_inputs(b=2, e=3, I=8, D=12, seed=0):
    ms = (_rand(b, e, I, D, seed=seed), _rand(b, e, D, I, seed=seed + 1),
          _rand(b, e, I, D, seed=seed + 2))
    g02 = _rand(b, e, 2 * I, D, seed=seed + 3) * 0.1
    g1 = _rand(b, e, D, I, seed=seed + 4) * 0.1
    return ms, g02, g1


def test_nvs_write_unit_rows_and_unprojected_master():
    ms, g02, g1 = _nvs_inputs()
    I = 8
    (f02, f1), (m0, m1, m2) = OW.nvs_write((g02, g1), ms, I)
    # the masters keep the plain sum: (master' - master) is the gradient
    torch.testing.assert_close(m0 - ms[0], g02[:, :, :I], rtol=0, atol=1e-6)
    torch.testing.assert_close(m2 - ms[2], g02[:, :, I:], rtol=0, atol=1e-6)
    torch.testing.assert_close(m1 - ms[1], g1, rtol=0, atol=1e-6)
    # fast rows: unit length along the last dim, parallel to the masters
    for f in (f02, f1):
        n = _rownorm(f.float())
        assert ((n - 1).abs() < 8e-3).all()
    torch.testing.assert_close(f02[:, :, :I].float(), (m0 / _rownorm(m0)[..., None]).float(),
                               rtol=8e-3, atol=1e-6)
    torch.testing.assert_close(f02[:, :, I:].float(), (m2 / _rownorm(m2)[..., None]).float(),
                               rtol=8e-3, atol=1e-6)
    # the library routine the reference calls
    ref = torch.nn.functional.normalize(m1, dim=3, eps=1e-5).to(torch.bfloat16)
    assert (f1.float() - ref.float()).abs().max() <= 8e-3


def test_nvs_write_clamps_tiny_rows():
    """F.normalize divides by max(|u|, eps): a row of norm 3e-6 comes out with
    norm 0.3 (a "+ eps" form would give 0.23), a zero row stays zero."""
    ms, g02, g1 = _nvs_inputs(b=1, e=1, I=4, D=8)
    w0 = ms[0].clone()
    w0[0, 0, 0] = 0.0
    w0[0, 0, 1] = 0.0
    g02 = g02.clone()
    g02[0, 0, 0] = 0.0
    v = torch.randn(8, generator=torch.Generator().manual_seed(9))
    g02[0, 0, 1] = v / v.norm() * 3e-6
    (f02, _), _ = OW.nvs_write((g02, g1), (w0, ms[1], ms[2]), 4)
    assert torch.equal(f02[0, 0, 0].float(), torch.zeros(8))
    assert abs(float(f02[0, 0, 1].float().norm()) - 0.3) < 3e-3


def test_nvs_write_packed_equals_three_matrices():
    ms, g02, g1 = _nvs_inputs(seed=4)
    I = 8
    (f02, f1), m = OW.nvs_write((g02, g1), ms, I)
    f3, m3 = OW.nvs_write((g02[:, :, :I], g1, g02[:, :, I:]), ms, I)
    assert torch.equal(f02, torch.cat([f3[0], f3[2]], dim=2)) and torch.equal(f1, f3[1])
    for a, b in zip(m, m3):
        assert torch.equal(a, b)


def test_nvs_write_muon_step_is_orthogonalised():
    """With Muon the masters move by NS5 of each expert matrix: the step's
    singular values sit near 1 (the quintic's band), so its Frobenius norm
    is about sqrt(min(R, C))."""
    ms, g02, g1 = _nvs_inputs(b=1, e=2, I=16, D=32, seed=6)
    _, m = OW.nvs_write((g02, g1), ms, 16, use_muon=True)
    step = m[0] - ms[0]
    sv = torch.linalg.svdvals(step[0, 0].double())
    assert (sv > 0.5).all() and (sv < 1.3).all()

"""GPU parity of the WRITE step (csrc/write_step.hip through
uttt_amd.fast_weight_write) against oracle/write.py on the same seeded
inputs.

Bar: the fp32 masters within rtol 1e-5 (the norms are reduced in a different
order than the oracle's fp64 sums); the momentum buffer and, without master
renorm, the unprojected master are bit-exact (same fp32 operations in the
same order); the bf16 fast weights within rtol 8e-3 (two bf16 ulps: an fp32
difference in the last place can move a value across a bf16 rounding
boundary).
"""
import pytest
import torch

from oracle import write as OW
from uttt_amd import _lib as L
from uttt_amd import fast_weight_write as FWW

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def _close_master(ours, ref):
    torch.testing.assert_close(ours.cpu(), ref, rtol=1e-5, atol=1e-6)


def _close_fast(ours, ref):
    assert ours.dtype == torch.bfloat16
    torch.testing.assert_close(ours.cpu().float(), ref.float(), rtol=8e-3, atol=1e-6)


@pytest.mark.parametrize("B,E,I,D,grad_dtype,mom", [
    (1, 4, 40, 96, torch.float32, False),       # w1 rows of 40: a partly filled wave
    (2, 3, 384, 192, torch.bfloat16, True),
    (1, 2, 3072, 1536, torch.bfloat16, False),  # the 760M expert shapes (rows of 1536 / 3072)
    (1, 2, 768, 4096, torch.float32, True),     # the longest segment one wave holds
])
def test_moe_write_matches_oracle(B, E, I, D, grad_dtype, mom):
    shapes = [(B, E, I, D), (B, E, D, I), (B, E, I, D)]
    masters = [_rand(s, i) / D ** 0.5 for i, s in enumerate(shapes)]
    grads = [_rand(s, 10 + i, 0.05).to(grad_dtype) for i, s in enumerate(shapes)]
    moms = [_rand(s, 20 + i, 0.05) for i, s in enumerate(shapes)] if mom else None
    m = torch.rand(B, 1, 1, 1, generator=torch.Generator().manual_seed(5)) if mom else None
    rf, rm, rmom = OW.moe_write(tuple(g.float() for g in grads), masters, moms, m, lr_scale=0.8)
    fast = tuple(w.to(torch.bfloat16).to(DEV) for w in masters)
    of, om, omom = FWW.apply_moe_update_dense(
        tuple(g.to(DEV) for g in grads), fast, tuple(w.to(DEV) for w in masters),
        tuple(x.to(DEV) for x in moms) if mom else None, m.to(DEV) if mom else None, lr_scale=0.8)
    for i in range(3):
        _close_master(om[i], rm[i])
        _close_fast(of[i], rf[i])
        if mom:
            assert torch.equal(omom[i].cpu(), rmom[i])
    if not mom:
        assert omom is None


@pytest.mark.parametrize("master_renorm,mom", [(False, False), (True, False), (False, True)])
def test_dense_write_matches_oracle(master_renorm, mom):
    b, h, d, r = 1, 4, 96, 2   # configs[0] head shape: d = 96, d_h = 192
    shapes = [(b, h, r * d, d), (b, h, d, r * d), (b, h, r * d, d)]
    masters = [_rand(s, i) / d ** 0.5 for i, s in enumerate(shapes)]
    # fast weights 3-6% off their masters, row by row: a write that took the
    # norms from the masters instead of the fast weights fails the bar below
    gap = torch.Generator().manual_seed(31)
    fast = [(w * (1.03 + 0.03 * torch.rand(w.shape[:-1] + (1,), generator=gap)))
            .to(torch.bfloat16) for w in masters]
    grads = [_rand(s, 10 + i, 0.02) for i, s in enumerate(shapes)]
    moms = [_rand(s, 20 + i, 0.02) for i, s in enumerate(shapes)] if mom else None
    coeffs = [torch.full((b, 1, 1, 1), 0.4), torch.full((b, 1, 1, 1), 0.6)] if mom else None
    coeff = torch.stack(coeffs).mean(0) if mom else None
    rf, rm, rmom = OW.dense_write(grads, fast, masters, r, moms, coeff, lr_scale=0.5,
                                  master_renorm=master_renorm)
    of, om, omom = FWW.apply_shared_update(
        tuple(g.to(DEV) for g in grads), tuple(f.to(DEV) for f in fast),
        tuple(w.to(DEV) for w in masters), tuple(x.to(DEV) for x in moms) if mom else None,
        [c.to(DEV) for c in coeffs] if mom else None, r=r, lr_scale=0.5,
        master_renorm=master_renorm)
    for i in range(3):
        _close_fast(of[i], rf[i])
        if master_renorm:
            _close_master(om[i], rm[i])
        else:
            assert torch.equal(om[i].cpu(), rm[i])
        if mom:
            assert torch.equal(omom[i].cpu(), rmom[i])
    if not master_renorm:
        # planted mistake: the same write with the norms of the masters (the
        # master-renorm mode's source) is off the kernel's result by more
        # than the fast-weight bar
        wf, _, _ = OW.dense_write(grads, [w.to(torch.bfloat16) for w in masters], masters, r,
                                  moms, coeff, lr_scale=0.5, master_renorm=False)
        assert max(((of[i].cpu().float() - wf[i].float()).abs()
                    / (wf[i].float().abs() + 1e-6)).max().item() for i in range(3)) > 2e-2


def test_write_in_place_equals_out_of_place():
    B, E, R, C = 1, 3, 64, 1536
    w = (_rand((B, E, R, C), 1) / C ** 0.5).to(DEV)
    g = _rand((B, E, R, C), 2, 0.05).to(torch.bfloat16).to(DEV)
    mom = _rand((B, E, R, C), 3, 0.05).to(DEV)
    mc = torch.tensor([0.7], device=DEV)
    outs = []
    for in_place in (False, True):
        master = w.clone()
        mo = mom.clone()
        m_out = master if in_place else torch.empty_like(master)
        mo_out = mo if in_place else torch.empty_like(mo)
        f_out = torch.empty(w.shape, dtype=torch.bfloat16, device=DEV)
        L.call("uttt_write_step", L.ptr(master), None, L.ptr(g), L.BF16, L.ptr(mo), L.ptr(mc), 0.3,
               B, E * R, C, C, 0, 1, L.ptr(m_out), L.ptr(f_out), L.ptr(mo_out), L.stream_of(w))
        outs.append((m_out, f_out, mo_out))
    for a, b_ in zip(*outs):
        assert torch.equal(a, b_)


def test_muon_write_rejects_unaligned_shapes():
    """The Newton-Schulz entry point needs rows and cols that are multiples
    of 8 (16-byte bf16 rows); anything else is refused before any launch."""
    w = torch.zeros(1, 1, 4, 8, device=DEV)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        FWW.apply_moe_update_dense((w, w, w), (w, w, w), (w, w, w), use_moun=True)


@pytest.mark.parametrize("use_moun,mom", [(False, False), (False, True), (True, True)])
def test_packed_pool_write_equals_three_matrix_write(use_moun, mom):
    """apply_moe_update_packed on W0_W2 / W1 (w0 rows then w2 rows per
    expert) gives bit for bit the three-matrix write (same row kernel, the
    same Newton-Schulz per [I, D] matrix), in place when given outputs."""
    from uttt_amd import fast_weight_write as FWW

    B, E, I, D = 2, 3, 64, 48
    g = torch.Generator().manual_seed(21)
    rn = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DEV)
    M0, M2, M1 = rn(B, E, I, D, sc=0.2), rn(B, E, I, D, sc=0.2), rn(B, E, D, I, sc=0.2)
    G0, G2, G1 = (rn(*t.shape, sc=0.05).to(torch.bfloat16) for t in (M0, M2, M1))
    moms = (rn(B, E, I, D, sc=0.05), rn(B, E, D, I, sc=0.05), rn(B, E, I, D, sc=0.05)) if mom else None
    coeff = torch.full((B, 1, 1, 1), 0.9, device=DEV) if mom else None
    ref = FWW.apply_moe_update_dense((G0, G1, G2), None, (M0, M1, M2), moms, coeff, lr_scale=0.7,
                                     use_moun=use_moun)
    M02 = torch.cat([M0, M2], dim=2).contiguous()
    G02 = torch.cat([G0, G2], dim=2).contiguous()
    mom_p = (torch.cat([moms[0], moms[2]], dim=2).contiguous(), moms[1]) if mom else None
    F02 = torch.empty(M02.shape, dtype=torch.bfloat16, device=DEV)
    F1 = torch.empty(M1.shape, dtype=torch.bfloat16, device=DEV)
    M1c = M1.clone()
    fast, master, new_mom = FWW.apply_moe_update_packed(
        G02, G1, M02, M1c, mom_p, coeff, lr_scale=0.7, use_moun=use_moun,
        out=((F02, F1), (M02, M1c)))
    torch.cuda.synchronize()
    assert fast[0] is F02 and master[0] is M02 and master[1] is M1c
    assert torch.equal(F02, torch.cat([ref[0][0], ref[0][2]], dim=2))
    assert torch.equal(F1, ref[0][1])
    assert torch.equal(M02, torch.cat([ref[1][0], ref[1][2]], dim=2))
    assert torch.equal(M1c, ref[1][1])
    if mom:
        assert torch.equal(new_mom[0], torch.cat([ref[2][0], ref[2][2]], dim=2))
        assert torch.equal(new_mom[1], ref[2][1])


@pytest.mark.parametrize("packed,grad_dtype,b,e,I,D", [
    (True, torch.float32, 2, 3, 40, 96),       # rows of 40: a partly filled wave
    (True, torch.bfloat16, 1, 4, 3072, 1536),  # the 760M expert shapes
    (False, torch.float32, 1, 2, 384, 192),
])
def test_nvs_unit_row_write_matches_oracle(packed, grad_dtype, b, e, I, D):
    """apply_raw_update (uttt_nvs/models/uttt_moe_block.py:665-714): masters
    bit-exact (one fp32 add), fast weights within two bf16 ulps; a zero row
    and a row of norm 3e-6 cover the clamp of F.normalize."""
    ms = [_rand(s, 30 + i) / D ** 0.5 for i, s in enumerate([(b, e, I, D), (b, e, D, I), (b, e, I, D)])]
    g02 = _rand((b, e, 2 * I, D), 40, 0.05).to(grad_dtype)
    g1 = _rand((b, e, D, I), 41, 0.05).to(grad_dtype)
    ms[0][0, 0, 0] = 0.0
    g02[0, 0, 0] = 0.0
    ms[0][0, 0, 1] = 0.0
    g02[0, 0, 1] = (torch.ones(D) * (3e-6 / D ** 0.5)).to(grad_dtype)
    grads = (g02, g1) if packed else (g02[:, :, :I].contiguous(), g1, g02[:, :, I:].contiguous())
    rf, rm = OW.nvs_write(tuple(g.float() for g in grads), ms, I)
    of, om = FWW.apply_raw_update(tuple(g.to(DEV) for g in grads), tuple(w.to(DEV) for w in ms),
                                  inter_dim=I)
    assert len(of) == len(rf)
    for a, r in zip(om, rm):
        assert torch.equal(a.cpu(), r)
    for a, r in zip(of, rf):
        assert a.shape == r.shape
        _close_fast(a, r)
    assert torch.equal(of[0][0, 0, 0].cpu().float(), torch.zeros(D))


def test_nvs_unit_row_write_muon():
    """With Muon the step is this library's Newton-Schulz (checked on its own
    in the Muon tests); the write after it matches the oracle's write of that
    same step, packed and as three matrices."""
    b, e, I, D = 1, 2, 64, 32
    ms = [_rand(s, 50 + i).to(DEV) for i, s in enumerate([(b, e, I, D), (b, e, D, I), (b, e, I, D)])]
    g02 = _rand((b, e, 2 * I, D), 60, 0.05).to(DEV)
    g1 = _rand((b, e, D, I), 61, 0.05).to(DEV)
    of, om = FWW.apply_raw_update((g02, g1), ms, inter_dim=I, use_muon=True)
    s02 = FWW.newton_schulz5(g02.reshape(b * e * 2, I, D)).reshape(g02.shape)
    s1 = FWW.newton_schulz5(g1.reshape(b * e, D, I)).reshape(g1.shape)
    rf, rm = OW.nvs_write((s02.float().cpu(), s1.float().cpu()), [w.cpu() for w in ms], I)
    for a, r in zip(om, rm):
        assert torch.equal(a.cpu(), r)
    for a, r in zip(of, rf):
        _close_fast(a, r)
    of3, om3 = FWW.apply_raw_update((g02[:, :, :I], g1, g02[:, :, I:]), ms, inter_dim=I,
                                    use_muon=True)
    assert torch.equal(torch.cat([of3[0], of3[2]], dim=2), of[0]) and torch.equal(of3[1], of[1])

"""GPU parity of the Muon write: the Newton-Schulz kernels (csrc/grouped_gemm.hip
through uttt_amd.fast_weight_write.newton_schulz5) and the momentum kernel
(csrc/write_step.hip) against oracle/write.py on the same seeded inputs.

Bar.  The momentum buffer bit-exact (same fp32 operations).  The written
fp32 masters and bf16 fast weights at the elementwise rtol 2e-2 against the
oracle's write fed the device's Newton-Schulz output for the oracle's own
input (this pins the momentum, scaling, add and norm-preserving projection
arithmetic), and against the pure oracle at the Newton-Schulz bar below,
applied to the update (new - old).  The Newton-Schulz output itself is bf16 tensor
arithmetic in the reference, and the iteration amplifies a perturbation
along a small singular direction by up to p'(0) = a (about 4) per step, so a
one-ulp difference of one product's rounding (the GEMMs accumulate in fp32
in another order than the CPU's) can reach tens of ulps in isolated
elements after five steps.  It is therefore held to: relative Frobenius
error to the oracle <= 1e-2; at most 1 element in 1000 outside the rtol 2e-2
elementwise bar; and, against the same iteration in fp64 without the bf16
roundings, an error no larger than 1.5x the oracle's own (both are bf16
realisations of the same map).
"""
import pytest
import torch

from oracle import write as OW
from tests.helpers import assert_bf16_close, assert_bf16_mostly_close
from uttt_amd import fast_weight_write as FWW

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


def _ns5_fp64(G):
    """The same iteration in fp64, no bf16 rounding (the map both realise)."""
    X = G.double()
    tr = X.shape[1] > X.shape[2]
    if tr:
        X = X.transpose(1, 2)
    X = X / (X.norm(dim=(1, 2), keepdim=True) + 1e-7)
    for a, b, c in OW.NS5_COEFFS:
        A = X @ X.transpose(1, 2)
        X = a * X + (b * A + c * A @ A) @ X
    return X.transpose(1, 2) if tr else X


def _rel(x, y):
    x, y = x.double().cpu(), y.double().cpu()
    return ((x - y).norm() / y.norm()).item()


@pytest.mark.parametrize("n,R,C,dtype,scale", [
    (3, 64, 128, torch.float32, 1.0),      # wide: X = G
    (2, 256, 128, torch.float32, 1.0),     # tall: X = G^T, transposed back
    (4, 96, 96, torch.bfloat16, 0.5),      # square, bf16 input, a step size
    (1, 40, 200, torch.float32, 1.0),      # partial tiles on both axes
    (2, 3072, 1536, torch.float32, 0.8),   # the 760M expert shape (w0 / w2)
])
def test_newton_schulz5_matches_oracle(n, R, C, dtype, scale):
    G = _rand((n, R, C), R + C).to(dtype)
    ref = OW.newton_schulz5(G)
    if scale != 1.0:
        ref = ref * scale                   # the reference's bf16 g * lr_scale
    ours = FWW.newton_schulz5(G.to(DEV), scale).cpu()
    assert ours.dtype == torch.bfloat16 and ours.shape == (n, R, C)
    assert torch.isfinite(ours.float()).all()
    assert _rel(ours, ref) <= 1e-2, _rel(ours, ref)
    o, r = ours.float(), ref.float()
    bound = 2e-2 * r.abs() + 2e-2 * r.pow(2).mean().sqrt()
    assert ((o - r).abs() > bound).float().mean().item() <= 1e-3
    exact = _ns5_fp64(G.float()) * scale
    assert _rel(ours, exact) <= 1.5 * _rel(ref, exact) + 1e-3, (_rel(ours, exact), _rel(ref, exact))


def _ns5_kernels(run):
    """Names of the device kernels that run() launches."""
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        run()
        torch.cuda.synchronize()
    return {e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA}


@pytest.mark.parametrize("n,R,C,dtype,scale", [
    (16, 192, 192, torch.float32, 1.0),    # the uTTT-Dense 124M w0 / w2 slices
    (8, 192, 192, torch.bfloat16, 0.5),
    (4, 96, 96, torch.float32, 1.0),       # configs[0]'s d = 96 slices
    (3, 64, 128, torch.float32, 1.0),      # wide
    (3, 192, 96, torch.float32, 0.7),      # tall: X = G^T
    (2, 32, 192, torch.bfloat16, 1.0),     # one row block
    (5, 160, 128, torch.float32, 1.0),     # tall, 5 x 4 blocks: uneven wave grid
    (2, 32, 32, torch.float32, 1.0),       # the smallest shape the one launch takes
])
def test_one_launch_newton_schulz_equals_multi_launch(n, R, C, dtype, scale):
    """Matrices with both sides multiples of 32 and at most 192 run the whole
    iteration in one launch (csrc/ns_small.hip); its result is the
    multi-launch path's bit for bit (same rounding points, same MFMA
    accumulation order), and the oracle's at the Newton-Schulz bar."""
    from uttt_amd import _lib as L

    G = _rand((n, R, C), 7 * R + C).to(dtype).to(DEV)
    prev = L.lib().uttt_debug_set_ns_path(1)
    try:
        multi = FWW.newton_schulz5(G, scale)
        names_multi = _ns5_kernels(lambda: FWW.newton_schulz5(G, scale))
    finally:
        L.lib().uttt_debug_set_ns_path(prev)
    L.lib().uttt_debug_set_ns_path(0)
    try:
        one = FWW.newton_schulz5(G, scale)
        names_one = _ns5_kernels(lambda: FWW.newton_schulz5(G, scale))
    finally:
        L.lib().uttt_debug_set_ns_path(prev)
    assert any("ns_small_kernel" in k for k in names_one), names_one
    assert not any("ns_small_kernel" in k for k in names_multi), names_multi
    assert torch.equal(one, multi), (one.float() - multi.float()).abs().max().item()
    ref = OW.newton_schulz5(G.cpu()) * scale
    assert _rel(one.cpu(), ref) <= 1e-2, _rel(one.cpu(), ref)


def test_newton_schulz5_zero_slice():
    """A zero slice orthogonalises to zero on both paths (the reference's
    X = G / (|G| + 1e-7) is 0 and every step keeps it 0), beside non-zero
    slices of the same call, whose norms are their own."""
    from uttt_amd import _lib as L

    G = _rand((3, 96, 96), 5)
    G[1] = 0.0
    outs = []
    for path in (0, 1):   # the one launch, then the multi-launch path
        prev = L.lib().uttt_debug_set_ns_path(path)
        try:
            outs.append(FWW.newton_schulz5(G.to(DEV), 1.0).cpu())
        finally:
            L.lib().uttt_debug_set_ns_path(prev)
    assert torch.equal(outs[0], outs[1])
    assert (outs[0][1] == 0).all()
    ref = OW.newton_schulz5(G)
    assert (ref[1] == 0).all()
    for i in (0, 2):
        assert _rel(outs[0][i], ref[i]) <= 1e-2, (i, _rel(outs[0][i], ref[i]))


def _gpu_ns5(G):
    """The device Newton-Schulz on the oracle's own input, for the oracle's
    write to consume: isolates the write arithmetic from the iteration's
    accumulation order."""
    return FWW.newton_schulz5(G.to(DEV), 1.0).cpu()


@pytest.mark.parametrize("mom", [False, True])
def test_moe_muon_write_matches_oracle(mom, monkeypatch):
    B, E, I, D = 1, 3, 192, 128
    shapes = [(B, E, I, D), (B, E, D, I), (B, E, I, D)]
    masters = [_rand(s, i) / D ** 0.5 for i, s in enumerate(shapes)]
    grads = [_rand(s, 10 + i, 0.05) for i, s in enumerate(shapes)]
    moms = [_rand(s, 20 + i, 0.05) for i, s in enumerate(shapes)] if mom else None
    m = torch.rand(B, 1, 1, 1, generator=torch.Generator().manual_seed(5)) if mom else None
    rf, rm, rmom = OW.moe_write(grads, masters, moms, m, lr_scale=0.7, use_moun=True)
    of, om, omom = FWW.apply_moe_update_dense(
        tuple(g.to(DEV) for g in grads), None, tuple(w.to(DEV) for w in masters),
        tuple(x.to(DEV) for x in moms) if mom else None, m.to(DEV) if mom else None,
        lr_scale=0.7, use_moun=True)
    monkeypatch.setattr(OW, "newton_schulz5", _gpu_ns5)
    cf, cm, _ = OW.moe_write(grads, masters, moms, m, lr_scale=0.7, use_moun=True)
    for i in range(3):
        assert_bf16_close(om[i], cm[i], name=f"master {i}")
        assert_bf16_close(of[i], cf[i], name=f"fast {i}")
        assert_bf16_mostly_close(om[i], rm[i], masters[i], name=f"master {i} (oracle NS5)")
        assert_bf16_mostly_close(of[i], rf[i], masters[i], name=f"fast {i} (oracle NS5)")
        if mom:
            assert torch.equal(omom[i].cpu(), rmom[i])


@pytest.mark.parametrize("master_renorm", [False, True])
def test_dense_muon_write_matches_oracle(master_renorm, monkeypatch):
    b, h, d, r = 1, 2, 64, 2
    shapes = [(b, h, r * d, d), (b, h, d, r * d), (b, h, r * d, d)]
    masters = [_rand(s, 30 + i) / d ** 0.5 for i, s in enumerate(shapes)]
    fast = [w.to(torch.bfloat16) for w in masters]
    grads = [_rand(s, 40 + i, 0.05) for i, s in enumerate(shapes)]
    moms = [_rand(s, 50 + i, 0.05) for i, s in enumerate(shapes)]
    coeff = torch.rand(b, 1, 1, 1, generator=torch.Generator().manual_seed(6))
    rf, rm, rmom = OW.dense_write(grads, fast, masters, r, moms, coeff, lr_scale=0.6,
                                  master_renorm=master_renorm, use_moun=True)
    of, om, omom = FWW.apply_shared_update(
        tuple(g.to(DEV) for g in grads), tuple(f.to(DEV) for f in fast),
        tuple(w.to(DEV) for w in masters), tuple(x.to(DEV) for x in moms), coeff.to(DEV),
        r=r, lr_scale=0.6, master_renorm=master_renorm, use_moun=True)
    monkeypatch.setattr(OW, "newton_schulz5", _gpu_ns5)
    cf, cm, _ = OW.dense_write(grads, fast, masters, r, moms, coeff, lr_scale=0.6,
                               master_renorm=master_renorm, use_moun=True)
    for i in range(3):
        assert_bf16_close(om[i], cm[i], name=f"master {i}")
        assert_bf16_close(of[i], cf[i], name=f"fast {i}")
        assert_bf16_mostly_close(om[i], rm[i], masters[i], name=f"master {i} (oracle NS5)")
        assert_bf16_mostly_close(of[i], rf[i], masters[i], name=f"fast {i} (oracle NS5)")
        assert torch.equal(omom[i].cpu(), rmom[i])

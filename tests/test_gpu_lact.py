"""GPU parity of the single-layer LaCT with the prenorm write
(uttt_amd/lact.py) against oracle/lact.py, and of its two write kernels
against their formulas.

Bars: the row norms and the prenorm write's fp32 main weights at rtol 1e-5,
its bf16 fast weights within one bf16 rounding; the loop's final weights at
rtol 2e-2 in bf16 (tests.helpers.assert_bf16_close).  The outputs: rtol 2e-2
against the oracle at the reference's rounding points on all but at most
1 element in 10^4; those few sit where the two rounding orders straddle a
cancellation (the kernels round each GEMM output once from fp32, the
reference's autocast bmm chain rounds y0 and y2 to bf16 before the SwiGLU),
and there the kernels' value must be as close to the exact fp64 result as
the reference's own rounding is, within the same bar.
"""
import pytest
import torch

from oracle import lact as OL
from tests.helpers import assert_bf16_close
from tests.test_oracle_lact import _case
from uttt_amd import lact

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("rows,C,gdt", [(300, 96, torch.bfloat16), (17, 1536, torch.float32),
                                        (64, 3072, torch.bfloat16)])
def test_prenorm_write_kernel(rows, C, gdt):
    g = torch.Generator().manual_seed(C)
    main = torch.randn(rows, C, generator=g) / C ** 0.5
    grad = (torch.randn(rows, C, generator=g) * 0.01).to(gdt)
    n0 = (torch.rand(rows, generator=g) + 0.5)
    norms = lact.row_norms(main.to(DEV))
    assert torch.allclose(norms.cpu(), main.double().norm(dim=1).float(), rtol=1e-5)
    md = main.to(DEV)
    fast = torch.empty(rows, C, dtype=torch.bfloat16, device=DEV)
    lact.write_prenorm(md, grad.to(DEV), n0.to(DEV), fast)
    u = main + grad.float()
    ref = u / (u.double().norm(dim=1, keepdim=True).float() + 1e-5) * n0[:, None]
    torch.testing.assert_close(md.cpu(), u, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(fast.cpu().float(), ref, rtol=8e-3, atol=1e-6)
    # bf16 rows also feed the norm kernel
    nb = lact.row_norms(main.to(torch.bfloat16).to(DEV))
    assert torch.allclose(nb.cpu(), main.to(torch.bfloat16).double().norm(dim=1).float(), rtol=1e-5)


def _close_ref_or_exact(ours, ref, exact, name):
    """rtol 2e-2 (+ 2e-2 rms) against the oracle at the reference's rounding
    points on all but 1 element in 10^4; those few (a cancellation the two
    rounding orders straddle) as close to the exact fp64 value as the
    reference's own rounding is, within the same bar."""
    o, r, x = ours.cpu().double(), ref.double(), exact.double()
    bound = 2e-2 * r.abs() + 2e-2 * r.pow(2).mean().sqrt()
    bad = (o - r).abs() > bound
    assert bad.double().mean() <= 1e-4, f"{name}: {int(bad.sum())} of {bad.numel()} off"
    assert ((o - x).abs()[bad] <= (r - x).abs()[bad] + bound[bad]).all(), name


def _check_muon_write(w0, w1, w2, q, k, v, lrs, momentum, c, out, rout, mains):
    """One Muon write (two chunks), stage by stage: the device's raw update of
    chunk 0 within the bf16 bar of the oracle's; its Newton-Schulz step (the
    new main minus the old, after the momentum) within the Newton-Schulz bar
    (relative Frobenius 1e-2) of the oracle's Newton-Schulz of that same raw
    update; chunk 0's output at the bf16 bar.  The oracle's own step, from
    its own raw update, differs by up to ~2% Frobenius: Newton-Schulz maps
    the update's singular values (condition ~10 here) toward 1 and so
    amplifies the 0.5% bf16-level difference between the two rounding
    orders; chunk 1's output is held to 3e-2 Frobenius against it."""
    from oracle import write as OW
    from uttt_amd.lact_moe_triton.lact_fw_grad import grouped_lact_swiglu_ffn_fast_weight_grads

    b, dh, d = w0.shape
    W02 = torch.cat([w0, w2], 1).to(torch.bfloat16).reshape(b, 1, 2 * dh, d).to(DEV)
    W1 = w1.to(torch.bfloat16).reshape(b, 1, d, dh).to(DEV)
    gs = torch.full((b, 1), c, dtype=torch.int32, device=DEV)
    d02, d1 = grouped_lact_swiglu_ffn_fast_weight_grads(
        W02, W1, k[:, :c].to(torch.bfloat16).contiguous().to(DEV),
        v[:, :c].to(torch.bfloat16).contiguous().to(DEV),
        *[x[:, :c].reshape(b, c).contiguous().to(DEV) for x in lrs], gs)
    ours = (d02[:, 0, :dh].cpu(), d1[:, 0].cpu(), d02[:, 0, dh:].cpu())
    args = (w0, w1, w2, k[:, :c], v[:, :c].transpose(1, 2), *[x[:, :c] for x in lrs])
    ref = OL.chunk_grads(*args)
    exact = OL.chunk_grads(*args, exact=True)
    for i, (g, r, x) in enumerate(zip(ours, ref, exact)):
        _close_ref_or_exact(g, r, x, f"raw update {i}")
        g = g.float()   # + the zero momentum buffer of the first write
        step = mains[i].cpu() - (w0, w1, w2)[i].float()
        ns = OW.newton_schulz5(g).float()
        assert (step - ns).norm() <= 1e-2 * ns.norm(), f"Newton-Schulz step {i}"
    assert_bf16_close(out[:, :c].cpu(), rout[:, :c], name="output chunk 0")
    o1, r1 = out[:, c:].cpu().float(), rout[:, c:].float()
    assert (o1 - r1).norm() <= 3e-2 * r1.norm(), "output chunk 1"


@pytest.mark.parametrize("kv_repeat,use_muon,with_mom", [
    (1, False, False), (2, False, False), (1, False, True), (1, True, False), (1, True, True)])
def test_prenorm_lact_loop_matches_oracle(kv_repeat, use_muon, with_mom):
    # Muon replaces each step by an orthogonal matrix of unit singular values,
    # an O(1) change of the weights per chunk whose Newton-Schulz iteration
    # amplifies bf16-level differences along small singular directions: the
    # trajectories of two correct roundings part after a few writes, so the
    # Muon cases check one write (two chunks) stage by stage
    b, dh, d, c = 2, 192, 96, 256                  # the configs[0] head shape
    seq = 2 * c if use_muon else 1024
    w0, w1, w2, q, k, v, lrs, mom = _case(b=b, dh=dh, d=d, seq=seq, kv_repeat=kv_repeat,
                                          seed=kv_repeat + 2 * use_muon + 4 * with_mom)
    momentum = mom if with_mom else None
    out, fast, mains = lact.prenorm_block_causal_lact_swiglu(
        *(t.to(DEV) for t in (w0, w1, w2, q, k, v)), *(x.to(DEV) for x in lrs), chunk_size=c,
        kv_repeat=kv_repeat, use_muon=use_muon,
        momentum=momentum.to(DEV) if with_mom else None, return_weights=True)
    torch.cuda.synchronize()
    rout, rfast, rmains = OL.prenorm_block_causal_lact_swiglu(
        w0, w1, w2, q, k, v, *lrs, chunk_size=c, kv_repeat=kv_repeat, use_muon=use_muon,
        momentum=momentum)
    assert out.dtype == torch.bfloat16 and out.shape == (b, seq, d)
    if use_muon:
        _check_muon_write(w0, w1, w2, q, k, v, lrs, momentum, c, out, rout, mains)
        return
    xout, _, _ = OL.prenorm_block_causal_lact_swiglu(
        w0, w1, w2, q, k, v, *lrs, chunk_size=c, kv_repeat=kv_repeat, use_muon=use_muon,
        momentum=momentum, exact=True)
    _close_ref_or_exact(out, rout, xout, "output")
    for i, nm in enumerate(("w0", "w1", "w2")):
        assert_bf16_close(fast[i].cpu(), rfast[i], name=f"fast {nm}")
        assert_bf16_close(mains[i].cpu(), rmains[i], name=f"main {nm}")
        # the prenorm invariant on the device result: the sequence-start norms
        n0 = (w0, w1, w2)[i].double().norm(dim=2)
        assert torch.allclose(fast[i].cpu().double().norm(dim=2), n0, rtol=8e-3)
    # chunk 0 is read with the initial weights: bit-equal to one grouped read
    from uttt_amd.lact_moe_triton.lact_swiglu_ffn import grouped_swiglu_ffn_fwd
    W02 = torch.cat([w0, w2], 1).to(torch.bfloat16).reshape(b, 1, 2 * dh, d).to(DEV)
    W1 = w1.to(torch.bfloat16).reshape(b, 1, d, dh).to(DEV)
    gs = torch.full((b, 1), c, dtype=torch.int32, device=DEV)
    first = grouped_swiglu_ffn_fwd(W02, W1, q[:, :c].to(torch.bfloat16).contiguous().to(DEV), gs)
    assert torch.equal(out[:, :c], first)

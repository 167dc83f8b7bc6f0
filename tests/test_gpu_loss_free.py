"""GPU parity of the loss-free balancing step (csrc/loss_free.hip through
uttt_amd.loss_free.LossFreeBalancer) and of the NVS router selection
(uttt_amd.nvs_routing) against oracle/routing.py.

Bars: counts, step counters and update counts bit-exact (sums of integers in
fp32); the bias within 1e-7 absolute (its mean is an fp32 sum whose order
differs from the oracle's); NVS mask and group sizes bit-exact, probabilities
and lb_loss within rtol 1e-5 (fp32).
"""
import pytest
import torch

from oracle import routing as OR
from uttt_amd import loss_free as LF
from uttt_amd import nvs_routing as NR

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("scope,L,B,E,warmup,interval", [
    ("layer", 24, 2, 32, 1, 1),
    ("pool", 24, 1, 96, 0, 2),
    ("layer", 3, 4, 300, 2, 3),     # E above one workgroup's width
])
def test_loss_free_sequence_matches_oracle(scope, L, B, E, warmup, interval):
    kw = dict(rate=1e-3, bias_max=0.01, warmup=warmup, interval=interval)
    ref = OR.LossFree(L, E, scope, **kw)
    ours = LF.LossFreeBalancer(L, E, lb_mode="loss_free", lb_scope=scope, update_rate=kw["rate"],
                               bias_max=kw["bias_max"], warmup_steps=warmup,
                               update_interval=interval)
    g = torch.Generator().manual_seed(E)
    zipf = 1.0 / torch.arange(1, E + 1).float() ** 1.1
    for step in range(12):
        a = torch.poisson(zipf.expand(L, B, E) * 400, generator=g)
        u = torch.poisson(zipf.flip(0).expand(L, B, E) * 100, generator=g)
        if step == 5:
            a.zero_(), u.zero_()
        ref.store(a, u)
        ours.store_loss_free_counts(a.to(DEV), u.to(DEV))
        ref.maybe_update()
        ours.maybe_update_loss_free_bias()
        torch.cuda.synchronize()
        assert torch.equal(ours.pending_counts.cpu(), ref.counts), step
        assert int(ours.steps) == ref.steps and int(ours.num_updates) == ref.num_updates, step
        torch.testing.assert_close(ours.bias.cpu(), ref.bias, rtol=0, atol=1e-7)
    assert ref.num_updates > 0
    rb = ours.get_router_bias(1)
    assert rb.shape == (1, E, 1)


def test_loss_free_disabled_paths():
    off = LF.LossFreeBalancer(2, 8, lb_mode="loss", update_rate=1e-3)
    assert off.get_router_bias(0) is None
    off.store_loss_free_counts(torch.ones(2, 1, 8, device=DEV), torch.ones(2, 1, 8, device=DEV))
    off.maybe_update_loss_free_bias()
    assert int(off.steps) == 0 and off.pending_counts.abs().sum() == 0
    with pytest.raises(ValueError, match="memory_lb_scope"):
        LF.LossFreeBalancer(2, 8, lb_scope="global")


@pytest.mark.parametrize("alpha,E,k", [(1.0, 32, 2), (2.5, 16, 1), (0.5, 96, 4)])
def test_nvs_router_matches_oracle(alpha, E, k):
    g = torch.Generator().manual_seed(E + k)
    logits = torch.randn(2, E, 257, generator=g)
    m, gs, p, lb = NR.create_router_mask_sizes_probs(logits.to(DEV), k, alpha)
    rm, rgs, rp, rlb = OR.nvs_create_router_mask_sizes_probs(logits, k, alpha)
    assert torch.equal(m.cpu(), rm) and torch.equal(gs.cpu(), rgs)
    torch.testing.assert_close(p.cpu(), rp, rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(lb.cpu(), rlb, rtol=1e-5, atol=1e-7)
    with pytest.raises(AssertionError):
        NR.create_router_mask_sizes_probs(logits.to(DEV), k, alpha, use_sigmoid=True)

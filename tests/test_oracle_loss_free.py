"""Pins of the router oracle's loss-free balancing state and NVS selection
(oracle/routing.py) by closed forms and invariants:

* one overloaded expert among E: after one step its bias is -2r(E-1)/E and
  every other expert's is 2r/E (sign step, then mean-centring), so the
  under-loaded experts gain score; equal counts leave the bias at zero;
* the clamp holds the bias inside [-bias_max, bias_max];
* warm-up passes drop their counts, an update interval holds them, a zero
  total does nothing;
* the pool scope sums the counts over layers and batches, the layer scope
  over batches only;
* the NVS selection is the uTTT-MoE selection with softmax scores, no bias and
  unmasked probabilities, its loss scaled by alpha; each token picks exactly
  top-k experts and the probabilities sum to alpha.
"""
import pytest
import torch

from oracle import routing as OR


def _lf(scope="layer", L=2, E=8, rate=1e-3, bias_max=2.0, warmup=0, interval=1):
    return OR.LossFree(L, E, scope, rate, bias_max, warmup, interval)


def _freqs(L, B, E, seed, hot=None):
    g = torch.Generator().manual_seed(seed)
    f = torch.randint(0, 50, (L, B, E), generator=g).float()
    if hot is not None:
        f[:, :, hot] += 1000
    return f


@pytest.mark.parametrize("E", [8, 96])
def test_one_overloaded_expert_closed_form(E):
    r = 1e-3
    s = _lf(scope="pool", L=1, E=E, rate=r)
    f = torch.full((1, 1, E), 10.0)
    f[0, 0, 3] = 10.0 + E * 5.0
    s.store(f, torch.zeros_like(f))
    s.maybe_update()
    want = torch.full((E,), 2 * r / E)
    want[3] = -2 * r * (E - 1) / E
    torch.testing.assert_close(s.bias, want, rtol=1e-5, atol=1e-9)
    assert abs(float(s.bias.double().sum())) < 1e-8
    assert s.num_updates == 1 and s.counts.abs().sum() == 0


def test_equal_counts_leave_bias():
    s = _lf()
    f = torch.full((2, 3, 8), 7.0)
    s.store(f, f)
    s.maybe_update()
    assert torch.equal(s.bias, torch.zeros(2, 8)) and s.num_updates == 1


def test_clamp_and_sign():
    s = _lf(E=4, L=1, rate=0.75, bias_max=1.0)
    for _ in range(4):
        f = torch.tensor([[[100.0, 0.0, 0.0, 0.0]]])
        s.store(f, torch.zeros_like(f))
        s.maybe_update()
        assert s.bias.abs().max() <= 1.0 + 1e-7
    assert s.bias[0, 0] < 0 and (s.bias[0, 1:] > 0).all()   # the loaded expert loses score


def test_warmup_interval_and_zero_total():
    s = _lf(warmup=2, interval=2)
    f = _freqs(2, 2, 8, 0, hot=1)
    for step in range(1, 8):
        s.store(f, f)
        before = s.counts.clone()
        s.maybe_update()
        if step <= 2:
            assert s.counts.abs().sum() == 0 and s.num_updates == 0     # warm-up drops counts
        elif (step - 2) % 2:
            assert torch.equal(s.counts, before)                         # held until the interval
        else:
            assert s.counts.abs().sum() == 0
    assert s.num_updates == 2
    z = _lf()
    z.store(torch.zeros(2, 1, 8), torch.zeros(2, 1, 8))
    z.maybe_update()
    assert z.num_updates == 0 and torch.equal(z.bias, torch.zeros(2, 8))


def test_scopes_sum_the_right_axes():
    a, u = _freqs(3, 2, 8, 1), _freqs(3, 2, 8, 2)
    p, l = _lf(scope="pool", L=3), _lf(scope="layer", L=3)
    p.store(a, u)
    l.store(a, u)
    assert torch.equal(p.counts, (a + u).sum(dim=(0, 1)))
    assert torch.equal(l.counts, (a + u).sum(dim=1))


@pytest.mark.parametrize("alpha,dtype", [(1.0, torch.float32), (2.5, torch.float32),
                                         (1.0, torch.bfloat16)])
def test_nvs_selection(alpha, dtype):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(2, 12, 50, generator=g).to(dtype)
    m, gs, p, lb = OR.nvs_create_router_mask_sizes_probs(logits, 3, alpha)
    assert (m.sum(dim=1) == 3).all() and torch.equal(gs, m.sum(-1).to(torch.int32))
    torch.testing.assert_close(p.float().sum(dim=1), torch.full((2, 50), alpha),
                               rtol=2e-2 if dtype == torch.bfloat16 else 1e-5, atol=0)
    m2, gs2, comb, bal, lb2 = OR.create_router_mask_sizes_probs(logits, 3, alpha)
    assert torch.equal(m, m2) and torch.equal(gs, gs2) and torch.equal(p, comb)
    torch.testing.assert_close(lb, lb2 * alpha, rtol=1e-2 if dtype == torch.bfloat16 else 1e-5,
                               atol=0)

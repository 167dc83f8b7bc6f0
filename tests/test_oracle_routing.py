"""Pins of the router oracle (oracle/routing.py) by facts independent of its
code path:

* the mask is the brute-force top-k: for each token, Python's sorted() over
  the (score + bias, expert) pairs picks the same k experts (continuous draws:
  no ties), and group_sizes are the mask's row sums;
* balance rows are probability vectors: softmax variants sum to 1; for
  norm_softmax the selection scores have norm `scale` so the balance equals
  softmax(scale * l / |l|); norm_relu with all-negative logits falls back to
  the uniform 1/E;
* topk_renorm combine weights sum to alpha over the selected experts and are
  zero elsewhere; selected_prob is alpha * balance;
* lb_loss is exactly 1 when the balance is uniform (sum_e freq_e = 1), and
  equals E * sum_e p_e f_e computed by brute force over a tiny case.
"""
import math

import pytest
import torch

from oracle import routing as R


def _logits(B, E, T, seed):
    return torch.randn(B, E, T, generator=torch.Generator().manual_seed(seed))


@pytest.mark.parametrize("rt", ["softmax", "norm_softmax", "norm_relu"])
def test_mask_is_brute_force_topk(rt):
    B, E, T, k = 2, 7, 50, 3
    l = _logits(B, E, T, 1)
    bias = torch.randn(1, E, 1, generator=torch.Generator().manual_seed(2)) * 0.3
    mask, gs, _, _, _ = R.create_router_mask_sizes_probs(l, k, router_type=rt, routing_bias=bias)
    scale = math.sqrt(E)
    for b in range(B):
        for t in range(T):
            col = l[b, :, t].tolist()
            n = math.sqrt(sum(v * v for v in col))
            if rt == "softmax":
                sel = col
            elif rt == "norm_softmax":
                sel = [v / n * scale for v in col]
            else:
                sel = [max(v / n, 0.0) * scale for v in col]
            sc = [(sel[e] + bias[0, e, 0].item(), e) for e in range(E)]
            top = {e for _, e in sorted(sc, reverse=True)[:k]}
            assert {e for e in range(E) if mask[b, e, t]} == top
    assert torch.equal(gs, mask.sum(-1).to(torch.int32))


def test_balance_rows_are_distributions():
    l = _logits(1, 6, 40, 3)
    _, _, _, bal, _ = R.create_router_mask_sizes_probs(l, 2)
    torch.testing.assert_close(bal.sum(1), torch.ones(1, 40))
    _, _, _, bal_n, _ = R.create_router_mask_sizes_probs(l, 2, router_type="norm_softmax",
                                                          router_scale=2.5)
    z = l / l.norm(dim=1, keepdim=True)
    torch.testing.assert_close(bal_n, torch.softmax(2.5 * z, dim=1))
    neg = -l.abs() - 0.1
    _, _, _, bal_r, _ = R.create_router_mask_sizes_probs(neg, 2, router_type="norm_relu")
    torch.testing.assert_close(bal_r, torch.full_like(bal_r, 1 / 6))


@pytest.mark.parametrize("alpha", [1.0, 0.7])
def test_combine_weights(alpha):
    l = _logits(2, 5, 30, 4)
    mask, _, comb, bal, _ = R.create_router_mask_sizes_probs(l, 2, alpha=alpha,
                                                             combine_mode="topk_renorm")
    torch.testing.assert_close(comb.sum(1), torch.full((2, 30), alpha))
    assert torch.all(comb[~mask] == 0)
    _, _, comb_s, bal_s, _ = R.create_router_mask_sizes_probs(l, 2, alpha=alpha)
    torch.testing.assert_close(comb_s, bal_s * alpha)


def test_lb_loss_uniform_and_brute_force():
    neg = -_logits(2, 4, 16, 5).abs() - 0.1
    *_, lb = R.create_router_mask_sizes_probs(neg, 2, router_type="norm_relu")
    assert abs(lb.item() - 1.0) < 1e-6
    l = _logits(2, 3, 5, 6)
    mask, gs, _, bal, lb = R.create_router_mask_sizes_probs(l, 1)
    B, E, T = l.shape
    p = [sum(bal[b, e, t].item() for b in range(B) for t in range(T)) / (B * T) for e in range(E)]
    g = [sum(int(mask[b, e, t]) for b in range(B) for t in range(T)) / B for e in range(E)]
    ref = E * sum(p[e] * g[e] / sum(g) for e in range(E))
    assert abs(lb.item() - ref) < 1e-6


def test_sigmoid_routing_refused():
    with pytest.raises(NotImplementedError):
        R.create_router_mask_sizes_probs(_logits(1, 4, 3, 0), 1, 1.0, True)


def test_router_logits_brute_force():
    """router_logits (modeling_recurrent_lact.py:153-157) is R x^T per batch:
    against explicit dot products, for shared [E, D] and per-batch [B, E, D]
    weights; a transposed operand (x R^T laid out [B, T, E]) is caught."""
    g = torch.Generator().manual_seed(9)
    B, T, E, D = 2, 5, 3, 7
    x = torch.randn(B, T, D, generator=g)
    for W in (torch.randn(E, D, generator=g), torch.randn(B, E, D, generator=g)):
        got = R.router_logits(x, W)
        assert got.shape == (B, E, T)
        for b in range(B):
            Wb = W if W.dim() == 2 else W[b]
            for e in range(E):
                for t in range(T):
                    ref = sum(float(Wb[e, d]) * float(x[b, t, d]) for d in range(D))
                    assert abs(float(got[b, e, t]) - ref) < 1e-9
    wrong = torch.matmul(x.double(), W.double().transpose(-1, -2))   # [B, T, E]
    assert wrong.shape != got.shape or not torch.allclose(wrong, got)

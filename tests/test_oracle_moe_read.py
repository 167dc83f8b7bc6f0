"""Pins of oracle/moe_read.py, the routed read (permute -> grouped SwiGLU ->
gate-weighted unpermute, modeling_recurrent_lact.py:330-349).

The composition of the pinned permute and apply oracles must equal the
per-token restatement (experts of a token in descending order, bf16 hidden
and expert outputs, fp32 merge) on ragged routings: tokens with fewer than k
experts and tokens with none.  Planted mistakes (swapped w0 / w2 halves,
gates of the wrong expert, a dropped expert) must break that equality.
"""
import pytest
import torch

from oracle import moe_read as MR
from tests.helpers import assert_bf16_close


def _case(B, T, E, k, D, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(torch.bfloat16)
    scores = torch.rand(B, E, T, generator=g)
    top = scores.topk(k, dim=1).indices
    mask = torch.zeros(B, E, T, dtype=torch.bool).scatter_(1, top, True)
    mask[:, :, 0] &= torch.arange(E).view(1, E) != top[:, 0, 0].view(B, 1)   # token 0: k-1 experts
    if T > 2:
        mask[:, :, 2] = False                                               # token 2: none
    probs = torch.rand(B, E, T, generator=g) * mask
    return x, W02, W1, mask, probs


@pytest.mark.parametrize("B,T,E,k,D,I", [(1, 1, 8, 2, 32, 48), (2, 5, 6, 3, 16, 24),
                                         (1, 9, 16, 2, 24, 40)])
def test_composition_equals_per_token(B, T, E, k, D, I):
    x, W02, W1, mask, probs = _case(B, T, E, k, D, I, seed=B * 100 + T)
    got = MR.apply_moe_grouped(x, W02, W1, mask, probs, k)
    ref = MR.apply_moe_direct(x, W02, W1, mask, probs)
    assert_bf16_close(got, ref, rtol=8e-3, name="routed read")
    if T > 2:
        assert (got[:, 2] == 0).all()                     # a token with no expert reads zero


def test_planted_mistakes_fail():
    B, T, E, k, D, I = 1, 4, 8, 2, 32, 48
    x, W02, W1, mask, probs = _case(B, T, E, k, D, I, seed=7)
    ref = MR.apply_moe_direct(x, W02, W1, mask, probs)
    swapped = torch.cat([W02[:, :, I:], W02[:, :, :I]], dim=2)
    wrong_gates = torch.roll(probs, 1, dims=1) * mask
    dropped = mask.clone()
    dropped[0, mask[0, :, 1].nonzero()[0, 0], 1] = False
    for bad in (MR.apply_moe_grouped(x, swapped, W1, mask, probs, k),
                MR.apply_moe_grouped(x, W02, W1, mask, wrong_gates, k),
                MR.apply_moe_grouped(x, W02, W1, dropped, probs, k)):
        with pytest.raises(AssertionError):
            assert_bf16_close(bad, ref, rtol=8e-3, name="planted")

"""Pins of the Newton-Schulz oracle (oracle/write.py newton_schulz5,
restating uttt_llm/flame/custom_models/uttt_moe/ttt_operation.py:19-46).

The reference ships no test or golden vector for it, so the restatement is
pinned by what the mathematics fixes:
  - NS5 maps each singular value s of the normalised G through
    p(s) = a s + b s^3 + c s^5 per step (X <- a X + (b A + c A^2) X with
    A = X X^T); for an orthogonal input every singular value is 1/sqrt(m)
    after the normalisation, so NS5(Q) = p5(...p1(1/sqrt(m))) Q exactly in
    real arithmetic, checked against that scalar recurrence in fp64;
  - on a random Gaussian G the result is close to orthogonal: every
    singular value lies in [0.6, 1.25] (the band these five steps reach);
  - the result does not depend on the scale of G (exactly, for powers of
    two, which bf16 represents without rounding) and commutes with the
    transpose (exactly: the transposed case is computed on X^T by
    construction).
Mutations of the oracle (coefficient columns swapped, the a X term dropped,
the steps reversed) must fail these checks, which the last test verifies.
"""
import math

import pytest
import torch

from oracle import write as OW


def _g(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def _orth(m, seed):
    q, _ = torch.linalg.qr(_g((m, m), seed).double())
    return q.float()


def _scalar_ns5(s0, coeffs):
    s = s0
    for a, b, c in coeffs:
        s = a * s + b * s ** 3 + c * s ** 5
    return s


def _band(X):
    sv = torch.linalg.svdvals(X.float())
    return sv.min().item(), sv.max().item()


@pytest.mark.parametrize("m", [32, 64, 96])
def test_orthogonal_input_follows_the_scalar_recurrence(m):
    Q = _orth(m, m)
    X = OW.newton_schulz5(Q.unsqueeze(0))[0].float()
    s = _scalar_ns5(1.0 / math.sqrt(m), OW.NS5_COEFFS)
    assert math.isfinite(s) and 0.5 < s < 1.5, s   # the five steps bring 1/sqrt(m) near 1
    err = (X - s * Q).abs().max().item()
    assert err <= 3e-2 * s, err


@pytest.mark.parametrize("shape", [(3, 64, 32), (2, 32, 96), (2, 48, 48), (1, 128, 256)])
def test_random_input_is_nearly_orthogonal(shape):
    lo, hi = _band(OW.newton_schulz5(_g(shape, 7)))
    assert 0.6 <= lo and hi <= 1.25, (lo, hi)


def test_scale_invariance_and_transpose():
    G = _g((2, 64, 96), 3)
    X = OW.newton_schulz5(G)
    assert torch.equal(OW.newton_schulz5(G * 4.0), X)
    assert torch.equal(OW.newton_schulz5(G * 0.125), X)
    assert torch.equal(OW.newton_schulz5(G.transpose(1, 2).contiguous()), X.transpose(1, 2))


def _checks_pass():
    try:
        test_orthogonal_input_follows_the_scalar_recurrence(64)
        test_random_input_is_nearly_orthogonal((2, 32, 96))
        # the recurrence above reads NS5_COEFFS; also pin the table against the
        # reference's first and last rows, which a reordering would move
        assert OW.NS5_COEFFS[0] == (4.0848, -6.8946, 2.9270)
        assert OW.NS5_COEFFS[-1] == (2.8366, -3.0525, 1.2012)
    except AssertionError:
        return False
    return True


def test_planted_mistakes_fail(monkeypatch):
    assert _checks_pass()
    good = OW.NS5_COEFFS
    for bad in (tuple((a, c, b) for a, b, c in good),        # b and c swapped
                tuple((0.0, b, c) for a, b, c in good),       # the a X term dropped
                tuple(reversed(good))):                       # steps in the wrong order
        monkeypatch.setattr(OW, "NS5_COEFFS", bad)
        assert not _checks_pass(), bad
    monkeypatch.setattr(OW, "NS5_COEFFS", good)

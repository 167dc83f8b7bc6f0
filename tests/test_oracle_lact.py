"""Pins of oracle/lact.py (CPU): the single-layer LaCT with the prenorm write
(uttt_nvs/models/kernels/ttt_operation.py:217-367).  Each check is one a
plausible mistake in the restatement fails: the chunk update against the
autograd-pinned grouped UPDATE oracle, the norm invariant of the prenorm
write, the read-before-write order, the last chunk never written, and the
zero-step and zero-momentum reductions."""
import pytest
import torch
import torch.nn.functional as F

from oracle import fastweight as FW
from oracle import lact as OL


def _case(b=2, dh=48, d=32, seq=96, kv_repeat=1, seed=0):
    g = torch.Generator().manual_seed(seed)
    w0 = torch.randn(b, dh, d, generator=g) / d ** 0.5
    w2 = torch.randn(b, dh, d, generator=g) / d ** 0.5
    w1 = torch.randn(b, d, dh, generator=g) / dh ** 0.5
    n = seq * kv_repeat
    q = F.normalize(torch.randn(b, seq, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(b, n, d, generator=g), dim=-1)
    v = F.normalize(torch.randn(b, n, d, generator=g), dim=-1)
    lrs = [torch.sigmoid(torch.randn(b, n, 1, generator=g)) * 0.1 for _ in range(3)]
    mom = torch.sigmoid(torch.randn(b, seq, 1, generator=g))
    return w0, w1, w2, q, k, v, lrs, mom


def test_chunk_grads_are_the_grouped_update():
    # the chunk update (lr applied to k / hidden, T:307-316) is the grouped
    # UPDATE of one expert (lr in the epilogue), whose oracle is pinned by
    # autograd: the same quantity in exact (fp64) arithmetic
    w0, w1, w2, q, k, v, (l0, l1, l2), _ = _case(seed=1)
    dw0, dw1, dw2 = OL.chunk_grads(w0, w1, w2, k, v.transpose(1, 2), l0, l1, l2, exact=True)
    b, dh, d = w0.shape
    W02 = torch.cat([w0, w2], dim=1).reshape(b, 1, 2 * dh, d)
    gs = torch.full((b, 1), k.shape[1], dtype=torch.int32)
    r02, r1 = FW.fast_weight_grads(W02, w1.reshape(b, 1, d, dh), k, v, l0[..., 0], l1[..., 0],
                                   l2[..., 0], gs, exact=True)
    assert torch.allclose(dw0, r02[:, 0, :dh].double(), rtol=1e-9, atol=1e-15)
    assert torch.allclose(dw2, r02[:, 0, dh:].double(), rtol=1e-9, atol=1e-15)
    assert torch.allclose(dw1, r1[:, 0].double(), rtol=1e-9, atol=1e-15)
    # the bf16 path stays within the bf16 bar of it
    bf = OL.chunk_grads(w0, w1, w2, k, v.transpose(1, 2), l0, l1, l2)
    for a, r in zip(bf, (dw0, dw1, dw2)):
        err = (a.double() - r).abs()
        assert (err <= 2e-2 * r.abs() + 2e-2 * r.pow(2).mean().sqrt()).all()


@pytest.mark.parametrize("use_muon,with_mom", [(False, False), (True, False), (False, True)])
def test_prenorm_write_keeps_the_sequence_start_norms(use_muon, with_mom):
    w0, w1, w2, q, k, v, lrs, mom = _case(seed=2)
    out, ws, mains = OL.prenorm_block_causal_lact_swiglu(
        w0, w1, w2, q, k, v, *lrs, chunk_size=32, use_muon=use_muon,
        momentum=mom if with_mom else None, exact=True)
    for w, w_init, m in zip(ws, (w0, w1, w2), mains):
        n0 = w_init.double().norm(dim=2)
        nm = m.norm(dim=2)
        # |fast row| = n0 * |main| / (|main| + 1e-5): the start norms up to the eps
        assert torch.allclose(w.norm(dim=2), n0 * nm / (nm + 1e-5), rtol=1e-12)
        assert torch.allclose(w.norm(dim=2), n0, rtol=1e-4)
        # and the main weights moved (the write is not a no-op)
        assert (m - w_init.double()).abs().max() > 1e-3


def test_read_before_write_and_last_chunk_unwritten():
    w0, w1, w2, q, k, v, lrs, _ = _case(seed=3)
    c = 32
    out, ws, _ = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *lrs, chunk_size=c,
                                                    exact=True)
    # chunk 0 is read with the initial weights
    first = OL._read(w0.double(), w1.double(), w2.double(), q[:, :c].transpose(1, 2).double(),
                     True).transpose(1, 2)
    assert torch.allclose(out[:, :c], first, rtol=1e-12, atol=1e-14)
    # the last chunk is read and never written: the weights after a sequence of
    # 3 chunks equal those after 2 chunks and one token
    _, ws2, _ = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q[:, :2 * c + 1], k[:, :2 * c + 1],
                                                   v[:, :2 * c + 1],
                                                   *[x[:, :2 * c + 1] for x in lrs],
                                                   chunk_size=c, exact=True)
    for a, b_ in zip(ws, ws2):
        assert torch.equal(a, b_)
    # and the chunk 1 read sees the weights after one write, not the initial ones
    assert not torch.allclose(out[:, c:2 * c], OL._read(w0.double(), w1.double(), w2.double(),
                                                        q[:, c:2 * c].transpose(1, 2).double(),
                                                        True).transpose(1, 2), rtol=1e-6)


def test_zero_step_and_zero_momentum_reductions():
    w0, w1, w2, q, k, v, lrs, mom = _case(seed=4)
    zero = [torch.zeros_like(x) for x in lrs]
    out, ws, mains = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *zero, chunk_size=32,
                                                        exact=True)
    for w, w_init, m in zip(ws, (w0, w1, w2), mains):
        assert torch.equal(m, w_init.double())            # main + 0
        n0 = w_init.double().norm(dim=2, keepdim=True)
        assert torch.allclose(w, w_init.double() * n0 / (n0 + 1e-5), rtol=1e-12)
    # momentum coefficients of zero give the momentum-free run
    a = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *lrs, chunk_size=32,
                                            momentum=torch.zeros_like(mom), exact=True)
    b_ = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *lrs, chunk_size=32, exact=True)
    assert torch.equal(a[0], b_[0])
    # and nonzero momentum changes the result from the second write on
    c = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *lrs, chunk_size=32,
                                            momentum=mom, exact=True)
    assert torch.equal(c[0][:, :64], b_[0][:, :64])
    assert not torch.allclose(c[0][:, 64:], b_[0][:, 64:], rtol=1e-6)


def test_kv_repeat_reads_k_and_v_at_the_repeated_rate():
    # kv_repeat = 2: chunk i updates from k / v rows [2 i c, 2 (i + 1) c)
    w0, w1, w2, q, k, v, lrs, _ = _case(seq=64, kv_repeat=2, seed=5)
    c = 32
    _, ws, mains = OL.prenorm_block_causal_lact_swiglu(w0, w1, w2, q, k, v, *lrs, chunk_size=c,
                                                      kv_repeat=2, exact=True)
    dws = OL.chunk_grads(w0.double(), w1.double(), w2.double(), k[:, :2 * c],
                         v[:, :2 * c].transpose(1, 2), *[x[:, :2 * c] for x in lrs], exact=True)
    for m, w_init, dw in zip(mains, (w0, w1, w2), dws):
        assert torch.allclose(m, w_init.double() + dw, rtol=1e-12)

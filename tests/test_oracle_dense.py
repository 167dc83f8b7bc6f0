"""Pins of the uTTT-Dense oracle (oracle/dense.py):

* the head split: read / compute_update equal the grouped oracle applied to
  each head's column block x[..., h*d:(h+1)*d] taken by plain slicing
  (fastweight's apply and update are pinned by autograd in
  test_oracle_fastweight.py), for lr shared by the heads and per head;
* the sweep's schedule: chunk 0 is read with the initial weights; a sequence
  of one chunk is never written; two layers with identical inputs under the
  mean reduce give the one-layer result; with lr = 0 every write only
  rescales each slice by nu / (nu + 1e-5).
"""
import torch

from oracle import dense as OD
from oracle import fastweight as FW


def _weights(b, H, d, r, seed=0):
    g = torch.Generator().manual_seed(seed)
    w0 = torch.randn(b, H, r * d, d, generator=g) / d ** 0.5
    w1 = torch.randn(b, H, d, r * d, generator=g) / d ** 0.5
    w2 = torch.randn(b, H, r * d, d, generator=g) / d ** 0.5
    return w0, w1, w2


def _qkv(b, S, H, d, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.nn.functional.normalize(torch.randn(b, S, H, d, generator=g), dim=-1)
               .reshape(b, S, H * d) for _ in range(3))
    return q, k, v


def test_read_is_per_head_apply():
    b, H, d, r, l = 2, 3, 8, 2, 11
    w0, w1, w2 = _weights(b, H, d, r)
    x, _, _ = _qkv(b, l, H, d, 1)
    out = OD.read(x, w0, w1, w2, exact=True)
    gs = torch.tensor([[l]], dtype=torch.int32)
    for bi in range(b):
        for h in range(H):
            xh = x[bi:bi + 1, :, h * d:(h + 1) * d]
            W02 = torch.cat([w0[bi, h], w2[bi, h]], 0)[None, None]
            ref = FW.swiglu_ffn_fwd(W02, w1[bi, h][None, None], xh, gs, exact=True)
            assert torch.allclose(out[bi, :, h * d:(h + 1) * d].double(), ref[0], atol=1e-12)


def test_update_is_per_head_update():
    b, H, d, r, l = 1, 3, 8, 2, 9
    w = _weights(b, H, d, r)
    _, k, v = _qkv(b, l, H, d, 2)
    g = torch.Generator().manual_seed(3)
    for lr in (torch.rand(b, l, 3, generator=g), torch.rand(b, l, H * 3, generator=g)):
        dw0, dw1, dw2 = OD.compute_update(k, v, lr, w, exact=True)
        gs = torch.tensor([[l]], dtype=torch.int32)
        for h in range(H):
            sl = slice(h * d, (h + 1) * d)
            lh = lr[0] if lr.shape[2] == 3 else lr[0, :, 3 * h:3 * h + 3]
            W02 = torch.cat([w[0][0, h], w[2][0, h]], 0)[None, None]
            r02, r1 = FW.fast_weight_grads(W02, w[1][0, h][None, None], k[:, :, sl], v[:, :, sl],
                                           lh[None, :, 0], lh[None, :, 1], lh[None, :, 2], gs,
                                           exact=True)
            assert torch.allclose(dw0[0, h].double(), r02[0, 0, :r * d], atol=1e-10)
            assert torch.allclose(dw2[0, h].double(), r02[0, 0, r * d:], atol=1e-10)
            assert torch.allclose(dw1[0, h].double(), r1[0, 0], atol=1e-10)


def _sweep_inputs(L, S, b=1, H=2, d=8, seed=10):
    qs, ks, vs, lrs = [], [], [], []
    for li in range(L):
        q, k, v = _qkv(b, S, H, d, seed + li)
        qs.append(q), ks.append(k), vs.append(v)
        lrs.append(torch.rand(b, S, 3, generator=torch.Generator().manual_seed(seed + 50 + li)) * 0.1)
    return qs, ks, vs, lrs


def test_sweep_schedule():
    H, d, r, S, c = 2, 8, 2, 40, 16
    w = _weights(1, H, d, r)
    fast = tuple(x.to(torch.bfloat16) for x in w)
    qs, ks, vs, lrs = _sweep_inputs(1, S, H=H, d=d)
    outs, f1, m1 = OD.sweep(qs, ks, vs, lrs, fast, w, r, c, exact=True)
    first = OD.read(qs[0][:, :c], *fast, exact=True)
    assert torch.allclose(outs[0][:, :c].double(), first.double())
    # one chunk: read only, no write
    o1, f_one, _ = OD.sweep([q[:, :c] for q in qs], [k[:, :c] for k in ks],
                            [x[:, :c] for x in vs], [x[:, :c] for x in lrs], fast, w, r, c)
    for a, b_ in zip(f_one, fast):
        assert torch.equal(a, b_)
    # two identical layers, mean reduce == one layer
    o2, f2, m2 = OD.sweep(qs * 2, ks * 2, vs * 2, lrs * 2, fast, w, r, c, exact=True)
    for a, b_ in zip(m2, m1):
        assert torch.allclose(a, b_, rtol=1e-6, atol=1e-7)
    assert torch.allclose(o2[1].double(), outs[0].double(), rtol=1e-6, atol=1e-7)


def test_sweep_zero_lr_only_rescales():
    H, d, r, S, c = 2, 8, 2, 48, 16
    w = _weights(1, H, d, r, seed=4)
    qs, ks, vs, lrs = _sweep_inputs(1, S, H=H, d=d, seed=20)
    zero = [torch.zeros_like(x) for x in lrs]
    fast = tuple(x.double() for x in w)
    _, f, m = OD.sweep(qs, ks, vs, zero, fast, w, r, c, exact=True, master_renorm=True)
    writes = (S + c - 1) // c - 1
    for name, a, w0 in zip(("w0", "w1", "w2"), m, w):
        sl = OD.OW.wide_to_slices(w0.double(), name, r)
        nu = sl.norm(dim=2, keepdim=True)
        ref = sl * (nu / (nu + 1e-5)) ** writes
        assert torch.allclose(OD.OW.wide_to_slices(a.double(), name, r), ref, rtol=1e-6, atol=1e-9)

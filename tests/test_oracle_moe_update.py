"""Pins of oracle/moe_update.py (CPU): closed forms and invariants that a
plausible mistake in the preprocessing, the per-writer gradient glue or the
aggregate sum would fail."""
import pytest
import torch

from oracle import fastweight as FW
from oracle import moe_update as MU


def _pre(x, silu=False, norm=None, rows_of=None, rope=None):
    """preprocess_rows on [rows, F] or [B, L, F]."""
    y = x if x.dim() == 3 else x.unsqueeze(0)
    out = MU.preprocess_rows(y, silu=silu, norm=norm, rows_of=rows_of, rope=rope)
    return out if x.dim() == 3 else out[0]


def test_l2_norm_rows_unit_norm_and_eps_placement():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(64, 96, generator=g) * 3).to(torch.bfloat16)
    y = _pre(x, norm="l2")
    n = y.double().norm(dim=-1)
    assert (n - 1).abs().max() < 2e-2
    # eps outside the norm and added, not max(|x|, eps) (F.normalize) or
    # inside the square root: |x| = 1e-5 gives 1e-5 / (1e-5 + 1e-5) = 0.5
    t = torch.zeros(1, 8)
    t[0, 3] = 1e-5
    y = _pre(t, norm="l2")
    assert abs(float(y[0, 3]) - 0.5) < 1e-6
    assert abs(float(torch.nn.functional.normalize(t, dim=-1)[0, 3]) - 0.5) > 0.4


def test_norms_round_once_in_fp32():
    # torch.compile'd l2_norm / rms_norm (ref_base.py:181-195) keep the norm in
    # fp32 and round only the quotient: the result equals the exact value
    # rounded to bf16 once (not the bf16-rounded norm of eager arithmetic)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(256, 384, generator=g) * 2).to(torch.bfloat16)
    xd = x.double()
    exact_l2 = xd / (xd.norm(dim=-1, keepdim=True) + 1e-5)
    exact_rms = xd / (xd.pow(2).mean(-1, keepdim=True) + 1e-5).sqrt()
    for norm, exact in (("l2", exact_l2), ("rms", exact_rms)):
        y = _pre(x, norm=norm)
        once = exact.to(torch.bfloat16)
        # at most one bf16 ulp from the once-rounded exact value, nearly always equal
        diff = (y.float() - once.float()).abs()
        assert (diff <= once.float().abs() * 2 ** -8 + 1e-30).all(), norm
        assert (diff > 0).float().mean() < 0.01, norm
    # rms: unit mean square; l2 and rms differ by sqrt(D)
    y = _pre(x.float(), norm="rms")
    assert (y.double().pow(2).mean(-1) - 1).abs().max() < 1e-5
    assert torch.allclose(_pre(x.float(), norm="l2") * 384 ** 0.5, y, rtol=1e-4, atol=1e-6)


def test_l2_norm_rows_scale_invariance_and_rows():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(4, 6, 4 * 32, generator=g) + 0.5).to(torch.bfloat16)
    # powers of two scale exactly in bf16 and the eps is below the norm's ulp
    assert torch.equal(_pre(2 * x, norm="l2"), _pre(x, norm="l2"))
    # per-head rows equal the norm of each head taken alone
    per_head = _pre(x, norm="l2", rows_of=32)
    for h in range(4):
        sl = slice(32 * h, 32 * h + 32)
        assert torch.equal(per_head[..., sl], _pre(x[..., sl].contiguous(), norm="l2"))
    assert not torch.equal(per_head, _pre(x, norm="l2"))


def test_silu_closed_forms():
    x = torch.tensor([[0.0, 1.0, 20.0, -20.0, -1.0, 2.0, 0.5, -0.5]])
    y = _pre(x, silu=True)
    assert float(y[0, 0]) == 0.0
    assert abs(float(y[0, 1]) - 0.7310585786) < 1e-6
    assert abs(float(y[0, 2]) - 20.0) < 1e-6
    assert abs(float(y[0, 3])) < 1e-6
    assert abs(float(y[0, 4]) + 0.2689414214) < 1e-6
    # bf16 input: silu rounds to bf16 before the norm
    yb = _pre(x.to(torch.bfloat16), silu=True)
    assert yb.dtype == torch.bfloat16
    assert torch.equal(yb, y.to(torch.bfloat16))


def _rope_complex(y, dim, base, offset):
    """The rotary as complex multiplication, angles in fp64 from the formula
    theta_i(p) = p / base^(2i/dim): pair (j, j + dim/2) of each block is the
    complex number y_j + i y_(j+dim/2), multiplied by exp(i theta_j(p))."""
    B, Lx, F = y.shape
    R = dim // 2
    blk = y.double().reshape(B, Lx, F // dim, 2, R)
    z = torch.complex(blk[..., 0, :], blk[..., 1, :])
    p = torch.arange(offset, offset + Lx, dtype=torch.float64).view(1, Lx, 1, 1)
    theta = p / (float(base) ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    w = z * torch.exp(1j * theta)
    return torch.stack([w.real, w.imag], dim=3).reshape(B, Lx, F)


@pytest.mark.parametrize("dim,base,offset", [(64, 1e6, 0), (64, 1e4, 37), (128, 500.0, 5)])
def test_rope_is_the_complex_rotation(dim, base, offset):
    g = torch.Generator().manual_seed(dim + offset)
    B, Lx, F = 2, 21, 3 * dim
    x = torch.randn(B, Lx, F, generator=g).to(torch.bfloat16)
    cos, sin = MU.rope_tables(dim, base, offset + Lx)
    assert cos.dtype == torch.bfloat16 and cos.shape == (offset + Lx, dim // 2)
    y = MU.preprocess_rows(x, rope=(cos, sin, offset))
    ref = _rope_complex(x.float(), dim, base, offset)
    # cos / sin are bf16 table values: a few bf16 ulps of |x|
    assert (y.double() - ref).abs().max() < 3 * 2 ** -8 * x.float().abs().max()
    # pair norms are kept (a rotation), position 0 is the identity
    blk = y.float().reshape(B, Lx, F // dim, 2, dim // 2).pow(2).sum(3)
    bx = x.float().reshape(B, Lx, F // dim, 2, dim // 2).pow(2).sum(3)
    assert torch.allclose(blk, bx, rtol=2e-2, atol=1e-3)
    if offset == 0:
        assert torch.equal(y[:, 0], x[:, 0])
    # the conjugate rotation undoes it (in fp32, before any rounding)
    yf = MU._rope_fp32(x.float(), cos, sin, offset)
    back = MU._rope_fp32(yf, cos, sin, offset, conj=True)
    c2s2 = (cos.float() ** 2 + sin.float() ** 2)[offset:offset + Lx]  # bf16 tables: ~1
    assert torch.allclose(back, x.float() * torch.cat([c2s2, c2s2], -1).repeat(1, F // dim)
                          .unsqueeze(0), rtol=1e-5, atol=1e-6)
    # a planted mistake fails: pairs of neighbours (the interleaved layout)
    inter = x.float().reshape(B, Lx, F // 2, 2).transpose(2, 3).reshape(B, Lx, F)
    assert (MU._rope_fp32(inter, cos, sin, offset).double() - ref).abs().max() > 0.1


def _pre_fp64(x, silu, norm, rows_of, rope):
    """The same map in fp64 without any rounding (for autograd)."""
    B, Lx, F = x.shape
    D = F if rows_of is None else rows_of
    y = x * torch.sigmoid(x) if silu else x
    yr = y.reshape(B, Lx, F // D, D)
    if norm == "l2":
        yr = yr / (yr.pow(2).sum(-1, keepdim=True).sqrt() + 1e-5)
    elif norm == "rms":
        yr = yr * torch.rsqrt(yr.pow(2).mean(-1, keepdim=True) + 1e-5)
    y = yr.reshape(B, Lx, F)
    if rope is not None:
        cos, sin, off = rope
        R = cos.shape[-1]
        c = cos[off:off + Lx].double().view(1, Lx, 1, R)
        s = sin[off:off + Lx].double().view(1, Lx, 1, R)
        blk = y.reshape(B, Lx, F // (2 * R), 2 * R)
        x0, x1 = blk[..., :R], blk[..., R:]
        y = torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], -1).reshape(B, Lx, F)
    return y


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("norm", [None, "l2", "rms"])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_preprocess_backward_is_the_vjp(silu, norm, rope, dtype):
    g = torch.Generator().manual_seed(int(silu) + 2 * len(str(norm)) + int(rope))
    B, Lx, H, hd = 2, 9, 2, 64
    x = (torch.randn(B, Lx, H * hd, generator=g) * 1.5).to(dtype)
    gout = torch.randn(B, Lx, H * hd, generator=g).to(torch.bfloat16 if rope else dtype)
    rp = (*MU.rope_tables(32, 1e4, 20), 3) if rope else None
    ours = MU.preprocess_rows_bwd(x, gout, silu=silu, norm=norm, rows_of=hd, rope=rp)
    assert ours.dtype == dtype and ours.shape == x.shape
    xd = x.double().requires_grad_()
    _pre_fp64(xd, silu, norm, hd, rp).backward(gout.double())
    ref = xd.grad
    tol = 1e-5 if (dtype == torch.float32 and not rope) else 3e-2
    err = (ours.double() - ref).abs()
    assert (err <= tol * ref.abs() + tol * ref.pow(2).mean().sqrt()).all(), err.max()


def test_preprocess_backward_planted_mistake_fails():
    # dropping the projection term of the l2 backward (g / (n + e) alone)
    # fails the bar the backward passes against autograd
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 4, 64, generator=g)
    gout = torch.randn(1, 4, 64, generator=g)
    xd = x.double().requires_grad_()
    _pre_fp64(xd, False, "l2", None, None).backward(gout.double())
    ref = xd.grad

    def within(t):
        err = (t.double() - ref).abs()
        return bool((err <= 3e-2 * ref.abs() + 3e-2 * ref.pow(2).mean().sqrt()).all())

    good = MU.preprocess_rows_bwd(x, gout, norm="l2")
    wrong = gout / (x.norm(dim=-1, keepdim=True) + 1e-5)
    assert within(good) and not within(wrong)
    # the l2 backward is orthogonal to the row (up to the eps term)
    assert ((good * x).sum(-1).abs() < 1e-4 * (good.abs() * x.abs()).sum(-1)).all()


def test_head_tokens_and_lr_tokens_index_map():
    B, Lx, H, hd = 2, 3, 4, 5
    x = torch.arange(B * Lx * H * hd, dtype=torch.float32).reshape(B, Lx, H * hd)
    t = MU.head_tokens(x, H)
    for b in range(B):
        for l in range(Lx):
            for h in range(H):
                assert torch.equal(t[b, l * H + h], x[b, l, h * hd:(h + 1) * hd])
    lr = torch.arange(B * Lx * 3, dtype=torch.float32).reshape(B, Lx, 3)
    lt = MU.lr_tokens(lr, H)
    assert lt.shape == (B, Lx * H, 3)
    for h in range(H):
        assert torch.equal(lt[:, h::H], lr)
    lr3h = torch.arange(B * Lx * 3 * H, dtype=torch.float32).reshape(B, Lx, 3 * H)
    lt = MU.lr_tokens(lr3h, H)
    for h in range(H):
        assert torch.equal(lt[:, h::H], lr3h[:, :, 3 * h:3 * h + 3])


def _writer(T, E, D, k, seed, all_ones=False, p=None):
    g = torch.Generator().manual_seed(seed)
    kk = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1).to(torch.bfloat16)
    vv = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1).to(torch.bfloat16)
    lr = torch.sigmoid(torch.randn(1, T, 3, generator=g)) * 0.1
    if all_ones:
        mask = torch.ones(1, E, T, dtype=torch.bool)
        probs = torch.full((1, E, T), 1.0 if p is None else p)
    else:
        s = torch.randn(1, E, T, generator=g)
        idx = s.topk(k, dim=1).indices
        mask = torch.zeros(1, E, T, dtype=torch.bool).scatter_(1, idx, True)
        probs = torch.softmax(s, dim=1) * mask
    return kk, vv, lr, mask, probs


def _weights(E, D, I, seed):
    g = torch.Generator().manual_seed(seed)
    W02 = (torch.randn(1, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(1, E, D, I, generator=g) / D ** 0.5).to(torch.bfloat16)
    return W02, W1


def test_writer_grads_identity_routing_is_the_update():
    """One expert, every token routed with gate 1: the permutation is the
    identity and v*p = v, so the glue reduces to the grouped UPDATE."""
    T, D, I = 40, 32, 48
    k, v, lr, mask, probs = _writer(T, 1, D, 1, 3, all_ones=True)
    W02, W1 = _weights(1, D, I, 4)
    got = MU.writer_grads(k, v, lr, mask, probs, 1, W02, W1)
    lrs = [lr[:, :, j].to(torch.bfloat16) for j in range(3)]
    ref = FW.fast_weight_grads(W02, W1, k, v, *lrs, torch.tensor([[T]], dtype=torch.int32))
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])


def test_writer_grads_scale_with_the_gate():
    """Gate 0.5 (exact in bf16) halves v, hence every dW exactly; a glue that
    dropped the v*p product would not."""
    T, D, I = 40, 32, 48
    W02, W1 = _weights(1, D, I, 5)
    a = MU.writer_grads(*_writer(T, 1, D, 1, 6, all_ones=True, p=1.0), 1, W02, W1)
    b = MU.writer_grads(*_writer(T, 1, D, 1, 6, all_ones=True, p=0.5), 1, W02, W1)
    assert torch.equal(b[0].double(), a[0].double() * 0.5)
    assert torch.equal(b[1].double(), a[1].double() * 0.5)


def test_writer_grads_per_expert_brute_force():
    """Top-2 of 4 experts: expert e's dW is the UPDATE over exactly the tokens
    that selected it, in token order, with v scaled by the token's gate."""
    T, E, D, I, k = 50, 4, 32, 40, 2
    kk, vv, lr, mask, probs = _writer(T, E, D, k, 7)
    W02, W1 = _weights(E, D, I, 8)
    d02, d1 = MU.writer_grads(kk, vv, lr, mask, probs, k, W02, W1)
    for e in range(E):
        sel = mask[0, e].nonzero().flatten()
        ke = kk[:, sel]
        ve = (vv[:, sel].float() * probs[0, e, sel].float()[None, :, None]).to(torch.bfloat16)
        lre = [lr[:, sel, j].to(torch.bfloat16) for j in range(3)]
        gs = torch.tensor([[len(sel)]], dtype=torch.int32)
        r02, r1 = FW.fast_weight_grads(W02[:, e:e + 1], W1[:, e:e + 1], ke, ve, *lre, gs)
        assert torch.equal(d02[:, e:e + 1], r02)
        assert torch.equal(d1[:, e:e + 1], r1)


def test_aggregate_is_the_sum_over_writers():
    T, E, D, I, k = 30, 4, 32, 40, 2
    W02, W1 = _weights(E, D, I, 9)
    ws = [_writer(T, E, D, k, 10 + i) for i in range(3)]
    s02, s1 = MU.aggregate_grads(ws, W02, W1, k)
    one = MU.aggregate_grads(ws[:1], W02, W1, k)
    d02, d1 = MU.writer_grads(*ws[0], k, W02, W1)
    assert torch.equal(one[0], d02.double()) and torch.equal(one[1], d1.double())
    # the same tokens as one writer: the per-expert segments hold all of them,
    # so the sum equals one UPDATE over the concatenation (up to bf16 rounding)
    cat = [torch.cat([w[i] for w in ws], dim=1 if i < 3 else 2) for i in range(5)]
    c02, c1 = MU.writer_grads(*cat, k, W02, W1)
    from tests.helpers import assert_bf16_close
    assert_bf16_close(c02, s02, name="dW0_W2 concat vs sum")
    assert_bf16_close(c1, s1, name="dW1 concat vs sum")
    # a sum that dropped a writer is far off
    s02b, _ = MU.aggregate_grads(ws[:2], W02, W1, k)
    with pytest.raises(AssertionError):
        assert_bf16_close(s02b, s02, name="dropped writer")


def test_writer_grads_bwd_identity_routing_and_gate():
    T, D, I = 24, 32, 40
    W02, W1 = _weights(1, D, I, 11)
    g = torch.Generator().manual_seed(12)
    G02 = (torch.randn(W02.shape, generator=g) * 0.02).to(torch.bfloat16)
    G1 = (torch.randn(W1.shape, generator=g) * 0.02).to(torch.bfloat16)
    k, v, lr, mask, probs = _writer(T, 1, D, 1, 13, all_ones=True)
    got = MU.writer_grads_bwd(k, v, lr, mask, probs, 1, W02, W1, G02, G1)
    lrs = [lr[:, :, j].to(torch.bfloat16) for j in range(3)]
    ref = FW.fast_weight_grads_bwd(W02, W1, k, v, *lrs, torch.tensor([[T]], dtype=torch.int32),
                                   G02, G1)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    assert torch.equal(got[2], ref[2]) and torch.equal(got[3], ref[3])
    assert torch.equal(got[4], torch.stack(ref[4:7], dim=-1))
    # d/dp of <grad_vp, v p> is <grad_vp, v>
    gp = (ref[3].double() * v.double()).sum(-1).float()
    assert torch.allclose(got[5][0, 0], gp[0], rtol=1e-6, atol=1e-9)
    # gate 0.5: grad_v is half of grad_vp
    k, v, lr, mask, probs = _writer(T, 1, D, 1, 13, all_ones=True, p=0.5)
    half = MU.writer_grads_bwd(k, v, lr, mask, probs, 1, W02, W1, G02, G1)
    vp = (v.float() * 0.5).to(torch.bfloat16)
    ref = FW.fast_weight_grads_bwd(W02, W1, k, vp, *lrs, torch.tensor([[T]], dtype=torch.int32),
                                   G02, G1)
    assert torch.equal(half[3].double(), (ref[3].double() * 0.5).to(torch.bfloat16).double())

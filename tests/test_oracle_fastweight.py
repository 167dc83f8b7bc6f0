"""Pins the grouped fast-weight oracle (oracle/fastweight.py) on the CPU.

Each check is chosen so a plausible slip fails it:
  - E=1 grouped ops equal one dense batched matmul of the whole token set
    (a wrong segment offset or a transposed operand breaks it);
  - in exact mode the UPDATE equals torch.autograd's gradient of the
    lr-weighted dot-product loss sum_n lr_j[n] <f(k_n), v_n> for each of the
    three matrices (a dropped SiLU' term, a wrong sign or a swapped lr fails);
  - a central finite difference of the same loss agrees with one dW entry;
  - an empty expert yields zero weight gradients and leaves its neighbours'
    segments unchanged (segment bookkeeping);
  - the APPLY equals W1 (silu(W0 x) * (W2 x)) built from torch.nn.functional.
"""
import torch
import torch.nn.functional as F

from oracle import fastweight as FW


def _inputs(B, E, D, I, gs, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    N = int(max(sum(r) for r in gs))
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(dtype)
    W1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(dtype)
    K = torch.randn(B, N, D, generator=g).to(dtype)
    V = torch.randn(B, N, D, generator=g).to(dtype)
    lr = [torch.sigmoid(torch.randn(B, N, generator=g)) * 0.1 for _ in range(3)]
    return W02, W1, K, V, lr, torch.tensor(gs, dtype=torch.int32)


def _f(t):
    return t.double()


def test_apply_e1_equals_dense_formula():
    W02, W1, X, _, _, gs = _inputs(2, 1, 24, 40, [[37], [37]])
    out = FW.swiglu_ffn_fwd(W02, W1, X, gs, exact=True)
    I = 40
    w0, w2, w1, x = _f(W02[:, 0, :I]), _f(W02[:, 0, I:]), _f(W1[:, 0]), _f(X)
    h = F.silu(torch.bmm(x, w0.transpose(1, 2))) * torch.bmm(x, w2.transpose(1, 2))
    ref = torch.bmm(h, w1.transpose(1, 2))
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_apply_grouped_equals_per_expert_dense():
    gs = [[5, 0, 17, 9], [1, 30, 0, 0]]
    W02, W1, X, _, _, gsz = _inputs(2, 4, 16, 24, gs, seed=1)
    out = FW.swiglu_ffn_fwd(W02, W1, X, gsz, exact=True)
    I = 24
    for b in range(2):
        s = 0
        for e, g in enumerate(gs[b]):
            x = _f(X[b, s:s + g])
            h = F.silu(x @ _f(W02[b, e, :I]).T) * (x @ _f(W02[b, e, I:]).T)
            assert torch.allclose(out[b, s:s + g], h @ _f(W1[b, e]).T, rtol=1e-12, atol=1e-12)
            s += g


def _loss_grads(W02, W1, K, V, lr, gs, b, e):
    """Autograd of sum_n lr_j[n] <f(k_n), v_n> over expert e's segment."""
    I = W02.shape[2] // 2
    s = int(gs[b, :e].sum())
    g = int(gs[b, e])
    k, v = _f(K[b, s:s + g]), _f(V[b, s:s + g])
    grads = []
    for j, wname in ((0, "w0"), (1, "w1"), (2, "w2")):
        w0 = _f(W02[b, e, :I]).clone().requires_grad_(wname == "w0")
        w2 = _f(W02[b, e, I:]).clone().requires_grad_(wname == "w2")
        w1 = _f(W1[b, e]).clone().requires_grad_(wname == "w1")
        f = (F.silu(k @ w0.T) * (k @ w2.T)) @ w1.T          # [g, D]
        loss = (lr[j][b, s:s + g].double() * (f * v).sum(-1)).sum()
        loss.backward()
        grads.append({"w0": w0, "w1": w1, "w2": w2}[wname].grad)
    return grads  # dW0 (lr0), dW1 (lr1), dW2 (lr2)


def test_update_is_gradient_of_dot_product_loss():
    gs = [[6, 0, 11], [3, 9, 5]]
    W02, W1, K, V, lr, gsz = _inputs(2, 3, 12, 20, gs, seed=2)
    dw02, dw1 = FW.fast_weight_grads(W02, W1, K, V, *lr, gsz, exact=True)
    I = 20
    for b in range(2):
        for e in range(3):
            if gs[b][e] == 0:
                assert torch.count_nonzero(dw02[b, e]) == 0 and torch.count_nonzero(dw1[b, e]) == 0
                continue
            g0, g1, g2 = _loss_grads(W02, W1, K, V, lr, gsz, b, e)
            assert torch.allclose(dw02[b, e, :I], g0, rtol=1e-10, atol=1e-12)
            assert torch.allclose(dw02[b, e, I:], g2, rtol=1e-10, atol=1e-12)
            assert torch.allclose(dw1[b, e], g1, rtol=1e-10, atol=1e-12)


def test_update_finite_difference():
    gs = [[7, 4]]
    W02, W1, K, V, lr, gsz = _inputs(1, 2, 8, 10, gs, seed=3)
    dw02, dw1 = FW.fast_weight_grads(W02, W1, K, V, *lr, gsz, exact=True)
    I, e, s, g = 10, 1, 7, 4
    k, v = _f(K[0, s:s + g]), _f(V[0, s:s + g])

    def loss(w0, w2, w1, lrv):
        f = (F.silu(k @ w0.T) * (k @ w2.T)) @ w1.T
        return (lrv * (f * v).sum(-1)).sum()

    w0, w2, w1 = _f(W02[0, e, :I]), _f(W02[0, e, I:]), _f(W1[0, e])
    h = 1e-6
    for (mat, i, j) in (("w0", 3, 5), ("w2", 7, 1), ("w1", 2, 9)):
        lrv = lr[{"w0": 0, "w1": 1, "w2": 2}[mat]][0, s:s + g].double()
        args = {"w0": w0.clone(), "w2": w2.clone(), "w1": w1.clone()}
        args[mat][i, j] += h
        lp = loss(args["w0"], args["w2"], args["w1"], lrv)
        args[mat][i, j] -= 2 * h
        lm = loss(args["w0"], args["w2"], args["w1"], lrv)
        fd = (lp - lm) / (2 * h)
        ana = {"w0": lambda: dw02[0, e, i, j], "w2": lambda: dw02[0, e, I + i, j],
               "w1": lambda: dw1[0, e, i, j]}[mat]()
        assert abs(fd - ana) < 1e-6 * max(1.0, abs(fd)), (mat, fd, ana)


def test_empty_expert_and_segment_independence():
    # removing an empty expert's slot must not change anyone else's result
    W02, W1, K, V, lr, gsz = _inputs(1, 3, 8, 12, [[5, 0, 6]], seed=4)
    a02, a1 = FW.fast_weight_grads(W02, W1, K, V, *lr, gsz)
    b02, b1 = FW.fast_weight_grads(W02[:, [0, 2]], W1[:, [0, 2]], K, V, *lr,
                                   torch.tensor([[5, 6]], dtype=torch.int32))
    assert torch.equal(a02[:, [0, 2]], b02) and torch.equal(a1[:, [0, 2]], b1)
    assert torch.count_nonzero(a02[0, 1]) == 0 and torch.count_nonzero(a1[0, 1]) == 0


def test_bf16_rounding_points_are_close_to_exact():
    # the rounded pipeline stays within the bf16 bar of the exact one
    W02, W1, K, V, lr, gsz = _inputs(1, 2, 64, 96, [[40, 24]], seed=5)
    r02, r1 = FW.fast_weight_grads(W02, W1, K, V, *lr, gsz)
    e02, e1 = FW.fast_weight_grads(W02, W1, K, V, *lr, gsz, exact=True)
    for r, e in ((r02, e02), (r1, e1)):
        err = (r.double() - e).abs().max()
        assert err <= 2e-2 * e.abs().max()


def test_apply_backward_is_autograd_of_apply():
    gs = [[9, 0, 14], [4, 4, 4]]
    W02, W1, X, G, _, gsz = _inputs(2, 3, 16, 20, gs, seed=6)
    gw02, gw1, gx = FW.swiglu_ffn_bwd(W02, W1, X, G, gsz, exact=True)
    I = 20
    for b in range(2):
        s = 0
        for e, g in enumerate(gs[b]):
            w0 = _f(W02[b, e, :I]).requires_grad_()
            w2 = _f(W02[b, e, I:]).requires_grad_()
            w1 = _f(W1[b, e]).requires_grad_()
            x = _f(X[b, s:s + g]).requires_grad_()
            f = (F.silu(x @ w0.T) * (x @ w2.T)) @ w1.T
            (f * _f(G[b, s:s + g])).sum().backward()
            assert torch.allclose(gw02[b, e, :I], w0.grad, rtol=1e-10, atol=1e-12)
            assert torch.allclose(gw02[b, e, I:], w2.grad, rtol=1e-10, atol=1e-12)
            assert torch.allclose(gw1[b, e], w1.grad, rtol=1e-10, atol=1e-12)
            assert torch.allclose(gx[b, s:s + g], x.grad, rtol=1e-10, atol=1e-12)
            s += g


def test_update_backward_is_autograd_of_update():
    """The exact-mode UPDATE backward equals torch.autograd through the exact
    UPDATE formula, for every input (W0, W2, W1, K, V, lr0, lr1, lr2)."""
    gs = [[5, 0, 9], [7, 3, 4]]
    W02, W1, K, V, lr, gsz = _inputs(2, 3, 10, 14, gs, seed=7)
    g = torch.Generator().manual_seed(8)
    GW02 = torch.randn(W02.shape, generator=g).to(torch.bfloat16)
    GW1 = torch.randn(W1.shape, generator=g).to(torch.bfloat16)
    out = FW.fast_weight_grads_bwd(W02, W1, K, V, *lr, gsz, GW02, GW1, exact=True)
    gw02, gw1, gk, gv, gl0, gl1, gl2 = out
    I = 14
    for b in range(2):
        s = 0
        for e, n in enumerate(gs[b]):
            w0 = _f(W02[b, e, :I]).requires_grad_()
            w2 = _f(W02[b, e, I:]).requires_grad_()
            w1 = _f(W1[b, e]).requires_grad_()
            k = _f(K[b, s:s + n]).requires_grad_()
            v = _f(V[b, s:s + n]).requires_grad_()
            l0, l1, l2 = (x[b, s:s + n].double().requires_grad_() for x in lr)
            y0, y2, dh = k @ w0.T, k @ w2.T, v @ w1
            sg = torch.sigmoid(y0)
            sw = sg * y0
            dy0 = l0[:, None] * sg * y2 * dh * (1 + y0 * (1 - sg))
            dy2 = l2[:, None] * sw * dh
            hl = l1[:, None] * sw * y2
            d_w0, d_w2, d_w1 = dy0.T @ k, dy2.T @ k, (hl.T @ v).T
            loss = ((d_w0 * _f(GW02[b, e, :I])).sum() + (d_w2 * _f(GW02[b, e, I:])).sum()
                    + (d_w1 * _f(GW1[b, e])).sum())
            loss.backward()
            tol = dict(rtol=1e-9, atol=1e-11)
            assert torch.allclose(gw02[b, e, :I], w0.grad, **tol)
            assert torch.allclose(gw02[b, e, I:], w2.grad, **tol)
            assert torch.allclose(gw1[b, e], w1.grad, **tol)
            if n:
                assert torch.allclose(gk[b, s:s + n], k.grad, **tol)
                assert torch.allclose(gv[b, s:s + n], v.grad, **tol)
                assert torch.allclose(gl0[b, s:s + n], l0.grad, **tol)
                assert torch.allclose(gl1[b, s:s + n], l1.grad, **tol)
                assert torch.allclose(gl2[b, s:s + n], l2.grad, **tol)
            s += n


def test_swiglu_bwd_bwd_is_vjp_of_first_order_map():
    """The pointwise pass (exact mode) returns the first-order values and the
    vector-Jacobian product of (dh, x0, x2, lr) -> (dx0, dx2, hidden_lr1)
    with the given cotangents, as torch.autograd computes it."""
    g = torch.Generator().manual_seed(21)
    B, I, L = 2, 5, 7
    dh = torch.randn(B, I, L, generator=g, dtype=torch.float64)
    x02 = torch.randn(B, 2 * I, L, generator=g, dtype=torch.float64)
    lr = [torch.rand(B, L, generator=g, dtype=torch.float64) for _ in range(3)]
    gdx = torch.randn(B, 2 * I, L, generator=g, dtype=torch.float64)
    ghl = torch.randn(B, I, L, generator=g, dtype=torch.float64)
    out = FW.swiglu_bwd_bwd(dh, x02, *lr, gdx, ghl, exact=True)
    h = dh.clone().requires_grad_()
    x = x02.clone().requires_grad_()
    ls = [t.clone().requires_grad_() for t in lr]
    x0, x2 = x[:, :I], x[:, I:]
    silu = F.silu(x0)
    dsilu = torch.autograd.grad(silu.sum(), x0, create_graph=True)[0]   # silu'(x0) by autograd
    dx0 = ls[0][:, None] * h * x2 * dsilu
    dx2 = ls[2][:, None] * h * silu
    hl1 = ls[1][:, None] * x2 * silu
    loss = (dx0 * gdx[:, :I]).sum() + (dx2 * gdx[:, I:]).sum() + (hl1 * ghl).sum()
    gh, gx, g0, g1, g2 = torch.autograd.grad(loss, [h, x, *ls])
    tol = dict(rtol=1e-10, atol=1e-12)
    assert torch.allclose(out[0], gh, **tol)
    assert torch.allclose(out[1], gx, **tol)
    for a, b_ in zip(out[2:5], (g0, g1, g2)):
        assert torch.allclose(a, b_, **tol)
    assert torch.allclose(out[5], torch.cat([dx0, dx2], 1).detach(), **tol)
    assert torch.allclose(out[6], hl1.detach(), **tol)


def test_backward_pieces_compose_to_update_backward():
    """four_grouped -> swiglu_bwd_bwd -> grad_kv -> two_gemm_fw_bwd, composed
    as the reference's backward does (L/lact_fw_grad.py:177-288), equals the
    autograd-pinned UPDATE backward in exact mode."""
    gs = [[4, 0, 6], [2, 5, 3]]
    W02, W1, K, V, lr, gsz = _inputs(2, 3, 8, 12, gs, seed=9)
    g = torch.Generator().manual_seed(10)
    GW02 = torch.randn(W02.shape, generator=g).to(torch.bfloat16)
    GW1 = torch.randn(W1.shape, generator=g).to(torch.bfloat16)
    ref = FW.fast_weight_grads_bwd(W02, W1, K, V, *lr, gsz, GW02, GW1, exact=True)
    y02, gy02, dh, gdh = FW.four_grouped(W02, GW02, W1, GW1, K, V, gsz, exact=True)
    lr64 = [x.double() for x in lr]
    g_dh, g_x02, gl0, gl1, gl2, dx02, hl1 = FW.swiglu_bwd_bwd(dh, y02, *lr64, gy02, gdh, exact=True)
    gk, gv = FW.grad_kv(GW02, W02, dx02, g_x02, W1, GW1, g_dh, hl1, gsz, exact=True)
    gw02, gw1 = FW.two_gemm_fw_bwd(g_x02, K, g_dh, V, gsz, exact=True)
    N = K.shape[1]
    cols = FW.written_columns(gsz, N)
    tol = dict(rtol=1e-10, atol=1e-12)
    assert torch.allclose(gw02, ref[0], **tol) and torch.allclose(gw1, ref[1], **tol)
    assert torch.allclose(gk[cols], ref[2][cols], **tol)
    assert torch.allclose(gv[cols], ref[3][cols], **tol)
    for a, b_ in zip((gl0, gl1, gl2), ref[4:]):
        assert torch.allclose(a[cols], b_[cols], **tol)

"""Oracle of the grouped SwiGLU fast-weight ops (checker only; see
oracle/__init__.py).  fp32 torch on the CPU, with the reference's bf16
rounding points.

Reference: uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/ (L/):
  two_mm_swiglu      triton_grouped_swiglu_kernels.py:204-270  (cited S:)
  gemm_transpose     triton_grouped_gemm.py:118-167            (cited G:)
  swiglu_ffn_fwd     lact_swiglu_ffn.py:37-61                  (cited F:)
  three_bmm_with_lr  triton_grouped_swiglu_bwd_with_lr_kernels.py:174-252 (cited U1:)
  two_gemm_fw_bwd    triton_lact_bwd_grouped_two_mm_grad_fw.py:117-225    (cited U2:)
  fast_weight_grads  lact_fw_grad.py:54-114                    (cited FG:)

Every GEMM takes bf16 operands, accumulates in fp32 (the oracle uses fp64
products summed in fp64, then rounds to fp32: a tighter statement of "fp32
accumulate" than any fixed order) and rounds the stored result to bf16 where
the reference stores bf16.  Columns of a batch beyond sum(group_sizes) are
never written by the reference (outputs come from torch.empty); the oracle
leaves them zero and the tests compare only written columns.

`exact=True` switches every bf16 rounding off (fp64 throughout): the
autograd and finite-difference checks in tests/test_oracle_fastweight.py use
it to pin the formulas themselves.
"""
from __future__ import annotations

import contextlib

import torch

# Accumulation dtype of the non-exact mode: fp64 for parity checks; the CPU
# baseline timing in bench.py switches it to fp32 (the reference's CPU path
# is fp32 PyTorch) with `fp32_accumulate()`.
_ACC = torch.float64


@contextlib.contextmanager
def fp32_accumulate():
    global _ACC
    old = _ACC
    _ACC = torch.float32
    try:
        yield
    finally:
        _ACC = old


def _r(x, exact):
    """Store point: bf16 in the reference, identity in exact mode."""
    return x if exact else x.to(torch.bfloat16)


def _f(x, exact):
    return x.double() if exact else x.float().to(_ACC)


def segments(group_sizes_row):
    """[(e, start, size)] of one batch: expert e owns [start, start+size)."""
    out, s = [], 0
    for e, g in enumerate(group_sizes_row.tolist()):
        out.append((e, s, int(g)))
        s += int(g)
    return out


def two_mm_swiglu(W0_W2, X, group_sizes, exact=False):
    """S:204-270.  Hidden[b, :, seg_e] = silu(w0 X_e^T) * (w2 X_e^T), bf16 [B, I, N]."""
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = X.shape[1]
    out = torch.zeros(B, I, N, dtype=torch.float64)
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            w = _f(W0_W2[b, e], exact)
            x = _f(X[b, s:s + g], exact)
            y0 = (w[:I] @ x.T)
            y2 = (w[I:] @ x.T)
            if not exact:
                y0, y2 = y0.float().to(_ACC), y2.float().to(_ACC)
            out[b, :, s:s + g] = y2 * (y0 * torch.sigmoid(y0))
    return _r(out, exact)


def gemm_transpose(W, X, group_sizes, exact=False):
    """G:118-167.  Y[b, seg_e, :] = (W[b,e] @ X[b, :, seg_e])^T, bf16 [B, N, M]."""
    B, E, M, K = W.shape
    N = X.shape[2]
    out = torch.zeros(B, N, M, dtype=torch.float64)
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            out[b, s:s + g] = (_f(W[b, e], exact) @ _f(X[b, :, s:s + g], exact)).T
    return _r(out, exact)


def swiglu_ffn_fwd(W0_W2, W1, X, group_sizes, exact=False):
    """F:37-61: the APPLY op.  Hidden is stored bf16 between the two GEMMs."""
    H = two_mm_swiglu(W0_W2, X, group_sizes, exact)
    return gemm_transpose(W1, H, group_sizes, exact)


def three_bmm_with_lr(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, exact=False):
    """U1:174-252.  Returns DY0_DY2 [B, 2I, N] and Hidden [B, I, N] (bf16):
      Y0 = w0 K^T, Y2 = w2 K^T, DH = w1^T V^T   (fp32 accumulate)
      DY0 = lr0 * sig*Y2*DH*(1 + Y0(1-sig)); DY2 = lr2 * silu(Y0)*DH;
      Hidden = lr1 * silu(Y0)*Y2     (lr loaded as stored, widened to fp32)."""
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = K.shape[1]
    dy = torch.zeros(B, I2, N, dtype=torch.float64)
    hid = torch.zeros(B, I, N, dtype=torch.float64)
    l0, l1, l2 = (_f(x.reshape(B, N), True) for x in (lr0, lr1, lr2))
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            w = _f(W0_W2[b, e], exact)
            k = _f(K[b, s:s + g], exact)
            v = _f(V[b, s:s + g], exact)
            y0 = w[:I] @ k.T
            y2 = w[I:] @ k.T
            dh = _f(W1[b, e], exact).T @ v.T
            if not exact:
                y0, y2, dh = (t.float().to(_ACC) for t in (y0, y2, dh))
            sig = torch.sigmoid(y0)
            sw = sig * y0
            dy[b, :I, s:s + g] = sig * y2 * dh * (1.0 + y0 * (1.0 - sig)) * l0[b, s:s + g]
            dy[b, I:, s:s + g] = sw * dh * l2[b, s:s + g]
            hid[b, :, s:s + g] = sw * y2 * l1[b, s:s + g]
    return _r(dy, exact), _r(hid, exact)


def two_gemm_fw_bwd(DY0_DY2, K, Hidden, V, group_sizes, exact=False):
    """U2:117-225.  dW0_W2[b,e] = DY0_DY2[:, seg] @ K[seg] ([B,E,2I,D]);
    dW1[b,e] = (Hidden[:, seg] @ V[seg])^T ([B,E,D,I]); bf16; an empty expert
    gets zeros."""
    B, I2, N = DY0_DY2.shape
    I = I2 // 2
    D = K.shape[2]
    E = group_sizes.shape[1]
    dw02 = torch.zeros(B, E, I2, D, dtype=torch.float64)
    dw1 = torch.zeros(B, E, D, I, dtype=torch.float64)
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            dw02[b, e] = _f(DY0_DY2[b, :, s:s + g], exact) @ _f(K[b, s:s + g], exact)
            dw1[b, e] = (_f(Hidden[b, :, s:s + g], exact) @ _f(V[b, s:s + g], exact)).T
    return _r(dw02, exact), _r(dw1, exact)


def fast_weight_grads(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, exact=False):
    """FG:54-114: the UPDATE op = U1 then U2 (DY0_DY2 and Hidden stored bf16)."""
    dy, hid = three_bmm_with_lr(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, exact)
    return two_gemm_fw_bwd(dy, K, hid, V, group_sizes, exact)


def written_columns(group_sizes, N):
    """[B, N] bool: token columns some expert segment covers."""
    B = group_sizes.shape[0]
    tot = group_sizes.sum(1)
    return torch.arange(N).unsqueeze(0) < tot.unsqueeze(1)


def swiglu_ffn_bwd(W0_W2, W1, X, grad_out, group_sizes, exact=False):
    """F:63-104: backward of the APPLY op.
      DY0_DY2, Hidden = three-GEMM pass with lr = 1 and V = grad_out (bf16),
      grad_W0_W2, grad_W1 = two_gemm_fw_bwd(DY0_DY2, X, Hidden, grad_out),
      grad_X[seg] = (W0_W2^T DY0_DY2[:, seg])^T   (bf16).
    Returns (grad_W0_W2, grad_W1, grad_X)."""
    B, N = X.shape[0], X.shape[1]
    ones = torch.ones(B, N)
    dy, hid = three_bmm_with_lr(W0_W2, W1, X, grad_out, ones, ones, ones, group_sizes, exact)
    gw02, gw1 = two_gemm_fw_bwd(dy, X, hid, grad_out, group_sizes, exact)
    gx = gemm_transpose(W0_W2.transpose(2, 3), dy, group_sizes, exact)
    return gw02, gw1, gx


def fast_weight_grads_bwd(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, G_W0_W2, G_W1,
                          exact=False):
    """FG:116-300: backward of the UPDATE op given the upstream gradients
    G_W0_W2 [B,E,2I,D] and G_W1 [B,E,D,I].  Rounding points as the reference:
      four GEMMs (L/triton_lact_bwd_grouped_four_mm.py:30-297) store bf16
        Y0_Y2 = W0_W2 K^T, GY = G_W0_W2 K^T, DH = W1^T V^T, GDH = G_W1^T V^T;
      the pointwise pass (L/triton_pointwise_kernels.py:354-436) computes in
        fp32 from those bf16 values and stores grad_dh, grad_x0_x2, dx0_x2,
        hidden_lr1 in bf16; grad_lr* = fp32 sums over the hidden rows, cast
        to the lr dtype;
      grad_K = G_W0_W2^T dx0_x2 + W0_W2^T grad_x0_x2 and
      grad_V = W1 grad_dh + G_W1 hidden_lr1 (L/triton_lact_bwd_grouped_grad_kv.py:29-224,
        bf16);
      grad_W0_W2, grad_W1 = two_gemm_fw_bwd(grad_x0_x2, K, grad_dh, V).
    Returns (grad_W0_W2, grad_W1, grad_K, grad_V, grad_lr0, grad_lr1, grad_lr2)."""
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = K.shape[1]
    lr_dtype = lr0.dtype
    l = [_f(x.reshape(B, N), True) for x in (lr0, lr1, lr2)]
    gdh = torch.zeros(B, I, N, dtype=torch.float64)
    gx02 = torch.zeros(B, I2, N, dtype=torch.float64)
    dx02 = torch.zeros(B, I2, N, dtype=torch.float64)
    hlr = torch.zeros(B, I, N, dtype=torch.float64)
    glr = [torch.zeros(B, N, dtype=torch.float64) for _ in range(3)]
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            k = _f(K[b, s:s + g], exact)
            v = _f(V[b, s:s + g], exact)

            def mm(w, a):
                y = _f(w, exact) @ a.T
                return y if exact else y.to(torch.bfloat16).to(_ACC)

            x02 = mm(W0_W2[b, e], k)
            gy = mm(G_W0_W2[b, e], k)
            dh = mm(W1[b, e].transpose(0, 1), v)
            gd = mm(G_W1[b, e].transpose(0, 1), v)
            x0, x2 = x02[:I], x02[I:]
            gdx0, gdx2 = gy[:I], gy[I:]
            L0, L1, L2 = (t[b, s:s + g] for t in l)
            sg = torch.sigmoid(x0)
            silu = sg * x0
            m = sg * (1 + x0 * (1 - sg))
            gdh[b, :, s:s + g] = gdx0 * L0 * x2 * m + gdx2 * L2 * silu
            gx2 = gdx0 * L0 * dh * m + gd * L1 * silu
            gsig = gdx0 * L0 * dh * x2 * (1 + x0 - 2 * sg * x0)
            gx0 = ((gdx2 * L2 * dh + gd * L1 * x2) * m + gdx0 * L0 * dh * x2 * sg * (1 - sg)
                   + gsig * sg * (1 - sg))
            gx02[b, :I, s:s + g] = gx0
            gx02[b, I:, s:s + g] = gx2
            glr[0][b, s:s + g] = (gdx0 * dh * x2 * m).sum(0)
            glr[1][b, s:s + g] = (gd * x2 * silu).sum(0)
            glr[2][b, s:s + g] = (gdx2 * dh * silu).sum(0)
            dx02[b, :I, s:s + g] = dh * x2 * m * L0
            dx02[b, I:, s:s + g] = silu * dh * L2
            hlr[b, :, s:s + g] = L1 * x2 * silu
    gdh, gx02, dx02, hlr = (_r(t, exact) for t in (gdh, gx02, dx02, hlr))
    gk = torch.zeros(B, N, D, dtype=torch.float64)
    gv = torch.zeros(B, N, D, dtype=torch.float64)
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            gk[b, s:s + g] = (_f(G_W0_W2[b, e], exact).T @ _f(dx02[b, :, s:s + g], exact)
                              + _f(W0_W2[b, e], exact).T @ _f(gx02[b, :, s:s + g], exact)).T
            gv[b, s:s + g] = (_f(W1[b, e], exact) @ _f(gdh[b, :, s:s + g], exact)
                              + _f(G_W1[b, e], exact) @ _f(hlr[b, :, s:s + g], exact)).T
    gw02, gw1 = two_gemm_fw_bwd(gx02, K, gdh, V, group_sizes, exact)
    glr = [t if exact else t.to(lr_dtype) for t in glr]
    return gw02, gw1, _r(gk, exact), _r(gv, exact), glr[0], glr[1], glr[2]


# ------------------------------------------------ kernel-level backward pieces
def four_grouped(W0_W2, G_W0_W2, W1, G_W1, K, V, group_sizes, exact=False):
    """L/triton_lact_bwd_grouped_four_mm.py:443-501 (reference_four_grouped):
    per segment Y0_Y2 = W0_W2 K^T, G_Y0_Y2 = G_W0_W2 K^T ([B,2I,N]),
    DHidden = W1^T V^T, G_DHidden = G_W1^T V^T ([B,I,N]); fp32 accumulate, bf16."""
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = K.shape[1]
    outs = [torch.zeros(B, r, N, dtype=torch.float64) for r in (I2, I2, I, I)]
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            k = _f(K[b, s:s + g], exact)
            v = _f(V[b, s:s + g], exact)
            outs[0][b, :, s:s + g] = _f(W0_W2[b, e], exact) @ k.T
            outs[1][b, :, s:s + g] = _f(G_W0_W2[b, e], exact) @ k.T
            outs[2][b, :, s:s + g] = _f(W1[b, e], exact).T @ v.T
            outs[3][b, :, s:s + g] = _f(G_W1[b, e], exact).T @ v.T
    return tuple(_r(o, exact) for o in outs)


def swiglu_bwd_bwd(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1, exact=False):
    """L/triton_pointwise_kernels.py:354-436.  Inputs [B,I,L] / [B,2I,L] /
    [B,L]; fp32 (fp64 when exact) arithmetic.  Returns (grad_dh, grad_x0_x2,
    grad_lr0, grad_lr1, grad_lr2, dx0_x2, hidden_lr1) with element outputs in
    the activations' dtype and the lr gradients in the lrs' dtype."""
    xd, ld = x0_x2.dtype, lr0.dtype
    acc = torch.float64 if exact else torch.float32
    h = dh.to(acc)
    x0, x2 = x0_x2.to(acc).chunk(2, dim=1)
    g0, g2 = grad_dx0_dx2.to(acc).chunk(2, dim=1)
    gh = grad_hidden_lr1.to(acc)
    l0, l1, l2 = (x.to(acc).unsqueeze(1) for x in (lr0, lr1, lr2))
    sg = torch.sigmoid(x0)
    silu = x0 * sg
    m = sg * (1 + x0 * (1 - sg))
    grad_dh = g0 * l0 * x2 * m + g2 * l2 * silu
    grad_x2 = g0 * l0 * h * m + gh * l1 * silu
    grad_sig = g0 * l0 * h * x2 * (1 + x0 - 2 * sg * x0)
    grad_x0 = (g2 * l2 * h + gh * l1 * x2) * m + g0 * l0 * h * x2 * sg * (1 - sg) \
        + grad_sig * sg * (1 - sg)
    glr0 = (g0 * h * x2 * m).sum(1)
    glr1 = (gh * x2 * silu).sum(1)
    glr2 = (g2 * h * silu).sum(1)
    dx02 = torch.cat([h * x2 * m * l0, silu * h * l2], dim=1)
    hl1 = l1 * x2 * silu
    cx = (lambda t: t) if exact else (lambda t: t.to(xd))
    cl = (lambda t: t) if exact else (lambda t: t.to(ld))
    return (cx(grad_dh), cx(torch.cat([grad_x0, grad_x2], dim=1)), cl(glr0), cl(glr1), cl(glr2),
            cx(dx02), cx(hl1))


def grad_kv(G_W0_W2, W0_W2, DY_lr, dY_02, W1, G_W1, dH, H_lr, group_sizes, exact=False):
    """L/triton_lact_bwd_grouped_grad_kv.py:344-396 (reference_grad_kv): per
    segment grad_K = G_W0_W2^T DY_lr + W0_W2^T dY_02 and
    grad_V = W1 dH + G_W1 H_lr, both [B,N,D]; fp32 accumulate, bf16."""
    B, E, I2, D = W0_W2.shape
    N = DY_lr.shape[2]
    gk = torch.zeros(B, N, D, dtype=torch.float64)
    gv = torch.zeros(B, N, D, dtype=torch.float64)
    for b in range(B):
        for e, s, g in segments(group_sizes[b]):
            if g == 0:
                continue
            sl = slice(s, s + g)
            gk[b, sl] = (_f(G_W0_W2[b, e], exact).T @ _f(DY_lr[b, :, sl], exact)
                         + _f(W0_W2[b, e], exact).T @ _f(dY_02[b, :, sl], exact)).T
            gv[b, sl] = (_f(W1[b, e], exact) @ _f(dH[b, :, sl], exact)
                         + _f(G_W1[b, e], exact) @ _f(H_lr[b, :, sl], exact)).T
    return _r(gk, exact), _r(gv, exact)

"""GPU parity of the uTTT-MoE caller glue (uttt_amd/moe.py) against the
oracle's compositions:
  - the routed prefill read (route -> row map -> permute -> grouped APPLY ->
    gate-weighted unpermute, modeling_recurrent_lact.py:296-349) at the
    configs[4] chunk (T = 2048, E = 32, D = 1536, I = 3072) and with four
    fast-weight heads, against oracle/moe_read.apply_moe_grouped on the
    router's own mask and gates;
  - one writer's gradients (M:453-518) and the aggregate of several writers
    (M:2428-2445), forward and backward, against oracle/moe_update.py;
  - the row preprocessing kernel (silu, l2 / rms norm per head or per row,
    the rotary embedding; forward and backward) against
    oracle/moe_update.preprocess_rows / preprocess_rows_bwd.
Bars: rtol 2e-2 in bf16 (tests.helpers.assert_bf16_close) for GEMM outputs;
the preprocessing within one bf16 rounding (rtol 8e-3) or 1e-5 in fp32, since
its fp32 sum of squares runs in another order than torch's and its sigmoid
uses the hardware exp (about 1 ulp of fp32).
"""
import pytest
import torch

from oracle import moe_read as MR
from oracle import moe_update as MU
from tests.helpers import assert_bf16_close
from uttt_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(ours, ref, rtol, name):
    o, r = ours.detach().float().cpu(), ref.float()
    bad = (o - r).abs() > rtol * r.abs() + 1e-6
    assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.numel()} elements off"


PREP_CASES = [
    # dtype, heads, hd, qk norm type, v norm type, rope (dim, base, offset) or None
    (torch.bfloat16, 4, 96, "l2", "rms", None),
    (torch.float32, 2, 64, "rms", "l2", None),
    (torch.bfloat16, 1, 1536, "l2", "l2", (64, 1e6, 0)),    # the 760M config: same_rope, l2
    (torch.bfloat16, 4, 384, "l2", "rms", (64, 1e6, 300)),  # four fast-weight heads, offset
    (torch.float32, 2, 256, "l2", "rms", (128, 1e4, 7)),
]


@pytest.mark.parametrize("dtype,heads,hd,qk_type,v_type,rope", PREP_CASES)
def test_preprocess_update_inputs(dtype, heads, hd, qk_type, v_type, rope):
    g = torch.Generator().manual_seed(heads + hd)
    B, Lx = 2, 37
    k = (torch.randn(B, Lx, heads * hd, generator=g) * 2).to(dtype)
    v = (torch.randn(B, Lx, heads * hd, generator=g) * 2).to(dtype)
    lr = torch.sigmoid(torch.randn(B, Lx, 3, generator=g)) * 0.1
    rp = orp = None
    if rope is not None:
        dim, base, off = rope
        cos, sin = MU.rope_tables(dim, base, off + Lx + 5)
        rp = moe.Rope(cos.to(DEV), sin.to(DEV), off)
        orp = (cos, sin, off)
    kd, vd = k.to(DEV).requires_grad_(), v.to(DEV).requires_grad_()
    kt, vt, lt = moe.preprocess_update_inputs(kd, vd, lr.to(DEV), heads, qkv_silu=True,
                                              v_norm=True, qk_norm=True, norm_type=v_type,
                                              qk_norm_type=qk_type, rope=rp)
    rk = MU.preprocess_rows(k, silu=True, norm=qk_type, rows_of=hd, rope=orp)
    rv = MU.preprocess_rows(v, silu=True, norm=v_type)
    # forward: within one rounding of the output dtype (the fp32 sums run in
    # another order than the oracle's; silu uses the hardware exp)
    out_bf16 = dtype == torch.bfloat16 or rope is not None
    _close(kt, MU.head_tokens(rk, heads), 8e-3 if out_bf16 else 1e-5, "k")
    _close(vt, MU.head_tokens(rv, heads), 8e-3 if dtype == torch.bfloat16 else 1e-5, "v")
    assert kt.dtype == (torch.bfloat16 if rope is not None else dtype) and vt.dtype == dtype
    assert torch.equal(lt.cpu(), MU.lr_tokens(lr, heads))
    # backward through the head tokens
    gk = torch.randn(kt.shape, generator=g).to(kt.dtype)
    gv = torch.randn(vt.shape, generator=g).to(vt.dtype)
    torch.autograd.backward([kt, vt], [gk.to(DEV), gv.to(DEV)])
    rgk = MU.preprocess_rows_bwd(k, gk.reshape(B, Lx, heads * hd), silu=True, norm=qk_type,
                                 rows_of=hd, rope=orp)
    rgv = MU.preprocess_rows_bwd(v, gv.reshape(B, Lx, heads * hd), silu=True, norm=v_type)
    assert kd.grad.dtype == dtype and vd.grad.dtype == dtype
    assert_bf16_close(kd.grad.cpu(), rgk, name="grad k")
    assert_bf16_close(vd.grad.cpu(), rgv, name="grad v")


@pytest.mark.parametrize("silu,norm,rows_of,rope", [
    (True, None, None, None), (False, "l2", 64, None), (False, "rms", None, None),
    (False, None, None, (32, 1e4, 2)), (True, None, 64, (64, 1e6, 0)),
])
def test_rows_preprocess_each_switch(silu, norm, rows_of, rope):
    g = torch.Generator().manual_seed(17)
    x = (torch.randn(3, 11, 256, generator=g) * 2).to(torch.bfloat16)
    rp = orp = None
    if rope is not None:
        dim, base, off = rope
        cos, sin = MU.rope_tables(dim, base, off + 11)
        rp, orp = moe.Rope(cos.to(DEV), sin.to(DEV), off), (cos, sin, off)
    xd = x.to(DEV).requires_grad_()
    y = moe.rows_preprocess(xd, silu=silu, norm=norm, rows_of=rows_of, rope=rp)
    _close(y, MU.preprocess_rows(x, silu=silu, norm=norm, rows_of=rows_of, rope=orp), 8e-3,
           "forward")
    gy = torch.randn(y.shape, generator=g).to(y.dtype)
    y.backward(gy.to(DEV))
    ref = MU.preprocess_rows_bwd(x, gy, silu=silu, norm=norm, rows_of=rows_of, rope=orp)
    assert_bf16_close(xd.grad.cpu(), ref, name="backward")


def test_read_query_path():
    # q -> silu -> l2 per head -> rotary, as the MoE read (M:588-601)
    g = torch.Generator().manual_seed(3)
    q = (torch.randn(1, 40, 4 * 96, generator=g) * 2).to(torch.bfloat16)
    cos, sin = MU.rope_tables(32, 1e4, 64)
    out = moe.preprocess_read_query(q.to(DEV), 4, qkv_silu=True, qk_norm=True,
                                    rope=moe.Rope(cos.to(DEV), sin.to(DEV), 9))
    ref = MU.preprocess_rows(q, silu=True, norm="l2", rows_of=96, rope=(cos, sin, 9))
    _close(out, ref, 8e-3, "q")
    assert moe.preprocess_read_query(q, 4) is q


@pytest.mark.parametrize("T,E,D,I,heads,topk,combine", [
    (2048, 32, 1536, 3072, 1, 2, "topk_renorm"),   # the configs[4] chunk read
    (256, 16, 4 * 96, 192, 4, 2, "selected_prob"),  # four fast-weight heads
])
def test_routed_read_matches_oracle(T, E, D, I, heads, topk, combine):
    g = torch.Generator().manual_seed(T + E)
    hd = D // heads
    x = torch.randn(1, T, D, generator=g).to(torch.bfloat16)
    W02 = (torch.randn(1, E, 2 * I, hd, generator=g) / hd ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(1, E, hd, I, generator=g) / I ** 0.5).to(torch.bfloat16)
    R = torch.randn(E, hd, generator=g) / hd ** 0.5
    bias = -1.1 * torch.log(torch.arange(E, dtype=torch.float32) + 1)
    cfg = moe.RouterConfig(topk=topk, combine_mode=combine)
    out, (bal_sum, gs) = moe.apply_moe_fast_weights_grouped(
        x.to(DEV), W02[:, :, :I].to(DEV), W1.to(DEV), W02[:, :, I:].to(DEV), R.to(DEV), cfg,
        heads, routing_bias=bias.to(DEV))
    assert out.shape == x.shape and out.dtype == x.dtype
    # the routing the read used (the router is deterministic)
    xt = moe.reshape_head_tokens(x.to(DEV), heads)
    mask, gs2, probs, bal = moe.route(xt, R.to(DEV), cfg, routing_bias=bias.to(DEV))
    assert torch.equal(gs, gs2) and torch.equal(gs2, mask.sum(-1, dtype=torch.int32))
    # the router's own balance sums: the same values added in another order
    torch.testing.assert_close(bal_sum, bal.sum(-1), rtol=1e-5, atol=1e-5)
    ref = MR.apply_moe_grouped(MU.head_tokens(x, heads), W02, W1, mask.cpu(), probs.cpu(), topk)
    ref = ref.reshape(1, T, D)
    assert_bf16_close(out, ref, name="routed read")
    # precomputed w0_w2 gives the same launches
    again, _ = moe.apply_moe_fast_weights_grouped(x.to(DEV), None, W1.to(DEV), None, R.to(DEV),
                                                  cfg, heads, routing_bias=bias.to(DEV),
                                                  precomputed_w0_w2=W02.to(DEV))
    assert torch.equal(again, out)


def _writer_inputs(T, E, D, k, seed):
    g = torch.Generator().manual_seed(seed)
    kk = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1).to(torch.bfloat16)
    vv = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1).to(torch.bfloat16)
    lr = torch.sigmoid(torch.randn(1, T, 3, generator=g)) * 0.1
    s = torch.randn(1, E, T, generator=g)
    idx = s.topk(k, dim=1).indices
    mask = torch.zeros(1, E, T, dtype=torch.bool).scatter_(1, idx, True)
    probs = (torch.softmax(s, dim=1) * mask).float()
    return kk, vv, lr, mask, probs


@pytest.mark.parametrize("n_writers", [1, 3])
def test_update_glue_and_aggregate(n_writers):
    E, D, I, k = 8, 128, 256, 2
    Ts = [300, 257, 512][:n_writers]
    g = torch.Generator().manual_seed(5)
    W02 = (torch.randn(1, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(1, E, D, I, generator=g) / D ** 0.5).to(torch.bfloat16)
    G02 = (torch.randn(1, E, 2 * I, D, generator=g) * 0.02).to(torch.bfloat16)
    G1 = (torch.randn(1, E, D, I, generator=g) * 0.02).to(torch.bfloat16)
    cpu = [_writer_inputs(T, E, D, k, 10 + i) for i, T in enumerate(Ts)]
    ws = [moe.WriterInputs(*(t.to(DEV).requires_grad_(t.is_floating_point()) if j != 3
                             else t.to(DEV) for j, t in enumerate(c))) for c in cpu]
    dw0, dw1, dw2 = moe.aggregate_moe_update_grads(ws, W02[:, :, :I].to(DEV), W1.to(DEV),
                                                   W02[:, :, I:].to(DEV), k)
    assert dw0.dtype == torch.float32 and dw0.shape == (1, E, I, D)
    s02, s1 = MU.aggregate_grads(cpu, W02, W1, k)
    assert_bf16_close(dw0, s02[:, :, :I], name="dW0")
    assert_bf16_close(dw2, s02[:, :, I:], name="dW2")
    assert_bf16_close(dw1, s1, name="dW1")
    if n_writers == 1:
        one = moe.compute_moe_update_grads_grouped(*(t.detach() for t in (ws[0].k_tokens,
                                                                           ws[0].v_tokens,
                                                                           ws[0].lr_tokens)),
                                                   W02[:, :, :I].to(DEV), W1.to(DEV),
                                                   W02[:, :, I:].to(DEV), ws[0].expert_mask,
                                                   ws[0].expert_mask.sum(-1, dtype=torch.int32),
                                                   ws[0].router_probs.detach(), k)
        for a, b in zip(one, (dw0, dw1, dw2)):
            assert torch.equal(a, b.detach())
    # backward: upstream gradients of (dW0, dW1, dW2) in the master dtype
    torch.autograd.backward([dw0, dw1, dw2], [G02[:, :, :I].float().to(DEV), G1.float().to(DEV),
                                              G02[:, :, I:].float().to(DEV)])
    torch.cuda.synchronize()
    for i, (c, w) in enumerate(zip(cpu, ws)):
        ref = MU.writer_grads_bwd(*c, k, W02, W1, G02, G1)
        nm = f"writer {i}"
        assert_bf16_close(w.k_tokens.grad, ref[2], name="grad_k " + nm)
        assert_bf16_close(w.v_tokens.grad, ref[3], name="grad_v " + nm)
        assert_bf16_close(w.lr_tokens.grad, ref[4].float(), name="grad_lr " + nm)
        assert_bf16_close(w.router_probs.grad, ref[5], name="grad_probs " + nm)


def test_compiled_read_and_update_equal_eager():
    """torch.compile (fullgraph, aot_eager: no generated kernels) over the
    routed read and the UPDATE with its backward runs the same registered
    ops as eager mode: bit-identical results."""
    E, D, I, T, k = 8, 128, 256, 300, 2
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, T, D, generator=g).to(torch.bfloat16).to(DEV)
    W02 = (torch.randn(1, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(DEV)
    W1 = (torch.randn(1, E, D, I, generator=g) / D ** 0.5).to(torch.bfloat16).to(DEV)
    R = (torch.randn(E, D, generator=g) / D ** 0.5).to(DEV)
    lr = (torch.sigmoid(torch.randn(1, T, 3, generator=g)) * 0.1).to(DEV)
    cfg = moe.RouterConfig(topk=k, combine_mode="topk_renorm")

    def read(x):
        return moe.apply_moe_fast_weights_grouped(x, None, W1, None, R, cfg, 1,
                                                  precomputed_w0_w2=W02)[0]

    def step(kk, vv, ll):
        m, gs, p, _ = moe.route(kk.detach(), R, cfg)
        d02, d1 = moe.moe_update_grads_packed(kk, vv, ll, W02, W1, m, gs, p, k)
        return (d02.float() * 1e-2).sum() + (d1.float() * 1e-2).sum(), d02, d1

    eager_out = read(x)
    comp_out = torch.compile(read, fullgraph=True, backend="aot_eager")(x)
    assert torch.equal(eager_out, comp_out)
    leaves = lambda: [t.clone().requires_grad_() for t in (x, x, lr)]
    a = leaves()
    loss_e, d02_e, d1_e = step(*a)
    loss_e.backward()
    b = leaves()
    loss_c, d02_c, d1_c = torch.compile(step, fullgraph=True, backend="aot_eager")(*b)
    loss_c.backward()
    assert torch.equal(d02_e, d02_c) and torch.equal(d1_e, d1_c)
    for ta, tb in zip(a, b):
        assert torch.equal(ta.grad, tb.grad)


def test_routed_read_without_gradient_equals_the_permuted_path():
    """The routed read under no_grad reads its token rows through the inverse
    row map (no permuted copy); with a gradient to track it permutes as the
    reference does.  Both give the same output bit for bit (configs[3] and
    configs[4] chunks)."""
    for E, D, I in ((16, 768, 1536), (32, 1536, 3072)):
        g = torch.Generator(device=DEV).manual_seed(E)
        W02 = (torch.randn(1, E, 2 * I, D, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16)
        W1 = (torch.randn(1, E, D, I, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16)
        x = torch.randn(1, 2048, D, generator=g, device=DEV)
        x = (x / x.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
        R = torch.randn(E, D, generator=g, device=DEV)
        rb = torch.randn(E, generator=g, device=DEV) * 0.5
        cfg = moe.RouterConfig(topk=2, combine_mode="topk_renorm")
        with torch.no_grad():
            fast, lb = moe.apply_moe_fast_weights_grouped(x, None, W1, None, R, cfg, 1,
                                                          routing_bias=rb, precomputed_w0_w2=W02)
        xg = x.clone().requires_grad_()
        slow, lb2 = moe.apply_moe_fast_weights_grouped(xg, None, W1, None, R, cfg, 1,
                                                       routing_bias=rb, precomputed_w0_w2=W02)
        torch.cuda.synchronize()
        assert torch.equal(fast, slow.detach()), f"E={E}: gathered read differs"
        assert torch.equal(lb[1], lb2[1])

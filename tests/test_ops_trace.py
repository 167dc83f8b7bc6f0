"""torch.compile over the drop-in ops on the CPU, with meta tensors: every
C-ABI call is a registered torch.ops.uttt_hip op whose fake implementation
gives its outputs' shapes, so the routed read and the UPDATE forward and
backward trace into one graph (fullgraph=True fails on any graph break).  No
kernel runs: meta tensors only carry shapes."""
import pytest
import torch

from uttt_amd import moe

DEV = "meta"
B, T, D, E, I = 1, 64, 32, 4, 48


def _t(*shape, dtype=torch.bfloat16, grad=False):
    return torch.empty(*shape, device=DEV, dtype=dtype, requires_grad=grad)


def test_routed_read_traces_as_one_graph():
    x, W02, W1 = _t(B, T, D), _t(B, E, 2 * I, D), _t(B, E, D, I)
    R = _t(E, D, dtype=torch.float32)
    cfg = moe.RouterConfig(topk=2)

    def read(x, W02, W1, R):
        out, (bal, gs) = moe.apply_moe_fast_weights_grouped(x, None, W1, None, R, cfg, 1,
                                                            precomputed_w0_w2=W02)
        return out, bal, gs

    out, bal, gs = torch.compile(read, fullgraph=True, backend="eager")(x, W02, W1, R)
    assert out.shape == (B, T, D) and out.dtype == torch.bfloat16
    assert bal.shape == (B, E) and gs.shape == (B, E) and gs.dtype == torch.int32


def test_update_forward_and_backward_trace_as_one_graph():
    W02, W1 = _t(B, E, 2 * I, D, grad=True), _t(B, E, D, I, grad=True)
    k, v = _t(B, T, D, grad=True), _t(B, T, D, grad=True)
    lr = _t(B, T, 3, dtype=torch.float32, grad=True)
    R = _t(E, D, dtype=torch.float32)
    cfg = moe.RouterConfig(topk=2, combine_mode="topk_renorm")

    def step(k, v, lr, W02, W1, R):
        m, gs, p, _ = moe.route(k.detach(), R, cfg)   # the router ops are forward only
        dW02, dW1 = moe.moe_update_grads_packed(k, v, lr, W02, W1, m, gs, p, 2)
        return (dW02.float().sum() + dW1.float().sum())

    loss = torch.compile(step, fullgraph=True, backend="aot_eager")(k, v, lr, W02, W1, R)
    loss.backward()
    for t in (k, v, lr, W02, W1):
        assert t.grad is not None and t.grad.shape == t.shape


@pytest.mark.parametrize("token_major", [True, False])
def test_fake_shapes(token_major):
    ops = torch.ops.uttt_hip
    gs = _t(B, E, dtype=torch.int32)
    W02, W1, X = _t(B, E, 2 * I, D), _t(B, E, D, I), _t(B, 2 * T, D)
    h = ops.grouped_gate_up(W02, X, gs, token_major)
    assert h.shape == ((B, 2 * T, I) if token_major else (B, I, 2 * T))
    assert ops.grouped_gemm_nt(W1, _t(B, 2 * T, I), gs).shape == (B, 2 * T, D)
    lr = _t(B, 2 * T)
    dy, hid, ys, dhs = ops.grouped_update_stage1(W02, W1, X, X, lr, lr, lr, gs, token_major, True)
    assert dy.shape == ((B, 2 * T, 2 * I) if token_major else (B, 2 * I, 2 * T))
    assert ys.shape == (B, 2 * T, 2 * I) and dhs.shape == (B, 2 * T, I)
    d02, d1 = ops.grouped_wgrad_pair(_t(B, 2 * T, 2 * I), X, _t(B, 2 * T, I), X, gs)
    assert d02.shape == W02.shape and d1.shape == W1.shape
    outs = ops.grouped_update_bwd(W02, W1, X, X, lr, lr, lr, gs, W02, W1, None, None)
    assert [o.shape for o in outs] == [W02.shape, W1.shape, X.shape, X.shape, lr.shape,
                                       lr.shape, lr.shape]
    mask = _t(B, E, T, dtype=torch.bool)
    rmap = ops.make_row_id_map(mask, B, T, E)
    assert rmap.shape == (B, T, 2 * E + 1) and rmap.dtype == torch.int32
    xp, pp = ops.permute_fwd(_t(B, T, D), rmap, _t(B, E, T, dtype=torch.float32), B, T, E, 2 * T, D)
    assert xp.shape == (B, 2 * T, D) and pp.shape == (B, 2 * T)
    assert ops.unpermute_fwd(xp, rmap, _t(B, E, T, dtype=torch.float32), B, T, E, D).shape == (B, T, D)
    r = ops.route_tokens(_t(B, T, D), _t(E, D, dtype=torch.float32), 2, 1.0, "softmax",
                         "selected_prob", 0.0, 1e-6, None, False)
    assert r[0].shape == (B, E, T) and r[0].dtype == torch.bool and r[4].numel() == 0
    assert r[5].shape == (B, E) and r[5].dtype == torch.float32

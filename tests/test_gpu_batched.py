"""GPU parity at the shapes bench.py times for configs[4] (uTTT-MoE 760M:
E=32, top-2, D=1536, I=3072, Zipf(1.1) routing prior), against the oracle.

The UPDATE runs through the product API, uttt_amd.moe.aggregate_moe_update_grads:
  - 24 writers of 2048 tokens concatenated, N = 98 304 routed rows: the
    batched UPDATE of the bench's sweep (XCD super-tile grids, every GEMM
    of the forward and of the 5-launch backward at its timed shape);
  - 1 writer, N = 4096: the per-layer UPDATE and its backward.
Forward and backward (autograd through the permute of k, v*p and lr) run on
the GPU at full size.  The oracle (oracle/fastweight.py, fp64 on the CPU)
checks what it can finish in seconds, exactly:
  - weight gradients of four experts (the largest, the smallest non-empty
    and two others) on a subset of 64 hidden units: hidden unit i's rows of
    dW0 / dW2 and column of dW1 (and of the backward's grad_W0_W2 / grad_W1)
    depend only on w0[i], w2[i], w1[:, i] and that expert's routed rows,
    which the oracle takes in the permuted order (writer-major, token-
    ascending; pinned by tests/test_oracle_moe_update.py);
  - per-token gradients (grad_k, grad_v, grad_lr, grad_probs) of sampled
    tokens: each depends only on that token's inputs and its experts'
    weights, so the oracle runs the token as a one-token writer
    (oracle/moe_update.writer_grads_bwd).
The batched call sums the writers' gradients in one fp32 accumulation; the
reference sums per-writer bf16 dW (the two agree to bf16 rounding, pinned in
tests/test_oracle_moe_update.py::test_aggregate_is_the_sum_over_writers).
Bar: rtol 2e-2 (tests.helpers.assert_bf16_close).
"""
import pytest
import torch

from oracle import fastweight as FW
from oracle import moe_update as MU
from tests.helpers import assert_bf16_close, routing_c2
from uttt_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"
E, D, I, TOPK, T = 32, 1536, 3072, 2, 2048


def _pool(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    W02 = (torch.randn(1, E, 2 * I, D, generator=g, device=DEV) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(1, E, D, I, generator=g, device=DEV) / D ** 0.5).to(torch.bfloat16)
    G02 = (torch.randn(1, E, 2 * I, D, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    G1 = (torch.randn(1, E, D, I, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    return W02, W1, G02, G1


def _writers(n, seed):
    """n writers' inputs as bench.py draws them: k, v ~ N(0,1) L2-normalised
    rows, lr = sigmoid(N(0,1)) * 0.1, routing top-2 of 32 with the Zipf(1.1)
    selection prior and topk_renorm gates."""
    out = []
    for l in range(n):
        g = torch.Generator().manual_seed(seed + l)
        k = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1)
        v = torch.nn.functional.normalize(torch.randn(1, T, D, generator=g), dim=-1)
        lr = torch.sigmoid(torch.randn(1, T, 3, generator=g)) * 0.1
        _, _, mask, _, probs = routing_c2(T=T, E=E, k=TOPK, seed=seed + 1000 + l, zipf=1.1)
        out.append(dict(k=k.to(torch.bfloat16), v=v.to(torch.bfloat16), lr=lr, mask=mask,
                        probs=probs.float()))
    return out


def _expert_rows(ws, e):
    """Expert e's permuted rows of the concatenated writers (writer-major,
    token-ascending): k, bf16(v * p), bf16 lr0/1/2."""
    ks, vs, ls = [], [], []
    for w in ws:
        sel = w["mask"][0, e].nonzero().flatten()
        ks.append(w["k"][0, sel])
        vs.append((w["v"][0, sel].float() * w["probs"][0, e, sel][:, None]).to(torch.bfloat16))
        ls.append(w["lr"][0, sel].to(torch.bfloat16))
    return torch.cat(ks)[None], torch.cat(vs)[None], torch.cat(ls)[None]


def _hidden_subset(n=64):
    idx = torch.linspace(0, I - 1, n).round().long()
    return torch.unique(idx)


def _sampled_experts(gs):
    sizes = gs.tolist()
    nonempty = [e for e in range(E) if sizes[e] > 0]
    pick = {max(range(E), key=lambda e: sizes[e]), min(nonempty, key=lambda e: sizes[e]), 3, 17}
    return sorted(pick)


@pytest.mark.parametrize("writers", [24, 1])
def test_update_fwd_bwd_at_760m_shape(writers):
    W02, W1, G02, G1 = _pool(seed=writers)
    ws = _writers(writers, seed=100 * writers)
    dev_ws = [moe.WriterInputs(w["k"].to(DEV).requires_grad_(), w["v"].to(DEV).requires_grad_(),
                               w["lr"].to(DEV).requires_grad_(), w["mask"].to(DEV),
                               w["probs"].to(DEV).requires_grad_()) for w in ws]
    Wl = [W02.clone().requires_grad_(), W1.clone().requires_grad_()]
    dW02, dW1 = moe.aggregate_moe_update_grads(dev_ws, None, Wl[1], None, TOPK,
                                               precomputed_w0_w2=Wl[0], packed=True)
    torch.autograd.backward([dW02, dW1], [G02, G1])
    torch.cuda.synchronize()
    gs = sum(w["mask"].sum(-1) for w in ws)[0]
    assert int(gs.sum()) == TOPK * T * writers
    S = _hidden_subset()
    SS = torch.cat([S, S + I])
    for e in _sampled_experts(gs):
        ke, ve, le = _expert_rows(ws, e)
        n = ke.shape[1]
        w02 = W02[0, e].cpu()[SS][None, None]
        w1 = W1[0, e].cpu()[:, S][None, None]
        g02 = G02[0, e].cpu()[SS][None, None]
        g1 = G1[0, e].cpu()[:, S][None, None]
        gsn = torch.tensor([[n]], dtype=torch.int32)
        lrs = [le[..., j] for j in range(3)]
        r02, r1 = FW.fast_weight_grads(w02, w1, ke, ve, *lrs, gsn)
        nm = f"e{e} (n={n})"
        assert_bf16_close(dW02[0, e].detach().cpu()[SS], r02[0, 0], name="dW0_W2 " + nm)
        assert_bf16_close(dW1[0, e].detach().cpu()[:, S], r1[0, 0], name="dW1 " + nm)
        ref = FW.fast_weight_grads_bwd(w02, w1, ke, ve, *lrs, gsn, g02, g1)
        assert_bf16_close(Wl[0].grad[0, e].cpu()[SS], ref[0][0, 0], name="grad_W0_W2 " + nm)
        assert_bf16_close(Wl[1].grad[0, e].cpu()[:, S], ref[1][0, 0], name="grad_W1 " + nm)
    # an expert no writer routed to gets exact zeros
    for e in (gs == 0).nonzero().flatten().tolist():
        assert torch.count_nonzero(dW02[0, e]) == 0 and torch.count_nonzero(dW1[0, e]) == 0

    # per-token gradients of sampled tokens, each as a one-token writer
    small = min((e for e in range(E) if int(gs[e]) > 0), key=lambda e: int(gs[e]))
    W02c = {}
    for li in sorted({0, writers // 2, writers - 1}):
        w, dw = ws[li], dev_ws[li]
        toks = list(range(8)) + list(range(T - 8, T))
        toks += w["mask"][0, small].nonzero().flatten()[:4].tolist()
        for t in sorted(set(toks)):
            sel = w["mask"][0, :, t].nonzero().flatten().tolist()
            for e in sel:
                if e not in W02c:
                    W02c[e] = (W02[0, e].cpu(), W1[0, e].cpu(), G02[0, e].cpu(), G1[0, e].cpu())
            # the token's experts only (others hold no rows of it)
            sub = torch.tensor(sel)
            w02 = torch.stack([W02c[e][0] for e in sel])[None]
            w1 = torch.stack([W02c[e][1] for e in sel])[None]
            g02 = torch.stack([W02c[e][2] for e in sel])[None]
            g1 = torch.stack([W02c[e][3] for e in sel])[None]
            mt = w["mask"][:, sub, t:t + 1]
            pt = w["probs"][:, sub, t:t + 1]
            ref = MU.writer_grads_bwd(w["k"][:, t:t + 1], w["v"][:, t:t + 1],
                                      w["lr"][:, t:t + 1], mt, pt, TOPK, w02, w1, g02, g1)
            nm = f"writer {li} token {t} experts {sel}"
            assert_bf16_close(dw.k_tokens.grad[0, t].cpu(), ref[2][0, 0], name="grad_k " + nm)
            assert_bf16_close(dw.v_tokens.grad[0, t].cpu(), ref[3][0, 0], name="grad_v " + nm)
            assert_bf16_close(dw.lr_tokens.grad[0, t].cpu(), ref[4][0, 0].float(),
                              name="grad_lr " + nm)
            assert_bf16_close(dw.router_probs.grad[0, sub, t].cpu(), ref[5][0, :, 0],
                              name="grad_probs " + nm)


def _close_dev(ours, ref, rtol=2e-2, name="", spread=None):
    """tests.helpers.assert_bf16_close's bar (|ours - ref| <= rtol*|ref| +
    rtol*rms(ref)) evaluated on the device, for whole pool-sized tensors.
    spread: sum of the magnitudes of the bf16-rounded terms that make up ref;
    each term carries up to 2^-9 of its own magnitude of rounding, so 2^-8 *
    spread is added to the bound (it matters only where the terms cancel)."""
    o, r = ours.detach().float(), ref.detach().float()
    assert o.shape == r.shape, (name, o.shape, r.shape)
    assert bool(torch.isfinite(o).all()), f"{name}: non-finite output"
    atol = rtol * r.pow(2).mean().sqrt()
    err = (o - r).abs()
    bound = rtol * r.abs() + atol
    if spread is not None:
        bound = bound + spread * 2.0 ** -8
    nbad = int((err > bound).sum())
    assert nbad == 0, (f"{name}: {nbad}/{o.numel()} elements out of tolerance; "
                       f"max err {err.max().item():.3e}, atol {atol.item():.3e}")


def test_batched_update_is_the_sum_over_writers():
    """Linearity at full size, over every expert and hidden unit: the batched
    UPDATE of 24 writers (N = 98 304) equals the sum of the 24 one-writer
    UPDATEs (each checked against the oracle above), the weight gradients of
    its backward the sum of theirs, and each token's gradients (k, v, lr,
    router probs) the ones its own writer's call gives.  The batched call
    accumulates all writers' rows in fp32 and rounds once; the sum adds 24
    bf16-rounded terms (the reference's own aggregate), so the bar is the
    bf16 one."""
    n = 24
    W02, W1, G02, G1 = _pool(seed=7)
    ws = _writers(n, seed=4242)

    def run(group):
        dws = [moe.WriterInputs(w["k"].to(DEV).requires_grad_(), w["v"].to(DEV).requires_grad_(),
                                w["lr"].to(DEV).requires_grad_(), w["mask"].to(DEV),
                                w["probs"].to(DEV).requires_grad_()) for w in group]
        Wl = [W02.clone().requires_grad_(), W1.clone().requires_grad_()]
        d02, d1 = moe.aggregate_moe_update_grads(dws, None, Wl[1], None, TOPK,
                                                 precomputed_w0_w2=Wl[0], packed=True)
        torch.autograd.backward([d02, d1], [G02, G1])
        return d02.detach(), d1.detach(), Wl[0].grad, Wl[1].grad, dws

    B02, B1, BG02, BG1, bdws = run(ws)
    sums = [torch.zeros(t.shape, dtype=torch.float32, device=DEV) for t in (B02, B1, BG02, BG1)]
    spreads = [torch.zeros_like(t) for t in sums]
    for li, w in enumerate(ws):
        d02, d1, g02, g1, dws = run([w])
        for s_, a_, t in zip(sums, spreads, (d02, d1, g02, g1)):
            s_ += t.float()
            a_ += t.float().abs()
        for attr in ("k_tokens", "v_tokens", "lr_tokens", "router_probs"):
            _close_dev(getattr(bdws[li], attr).grad, getattr(dws[0], attr).grad,
                       name=f"writer {li} grad {attr}")
    torch.cuda.synchronize()
    for t, s_, a_, nm in zip((B02, B1, BG02, BG1), sums, spreads,
                             ("dW0_W2", "dW1", "grad_W0_W2", "grad_W1")):
        _close_dev(t, s_, name=f"{nm} (batched) vs sum of writers", spread=a_)

"""GPU parity of the router (csrc/router.hip via uttt_amd.routing) against
oracle/routing.py on the same seeded logits.

Bar: mask and group_sizes bit-exact.  For the softmax router the routing
scores are the logits themselves, so the selection must match exactly; the
norm variants divide by a norm whose fp32 rounding can differ by an ulp from
torch's, and norm_relu clamps negative scores to exactly 0 (true ties, whose
order torch.topk leaves unspecified), so a token may only differ where its
k-th and (k+1)-th routing scores are within 1e-5; lb_loss is then checked
against the value implied by the kernel's own group sizes.  combine,
balance and lb_loss within rtol 1e-5 (fp32; exp and the sums round
differently).  The fused route (logits = R x^T in fp32) is compared with the
fp64 product within 1e-4 relative to |R||x|, and its selection with the
oracle's on the kernel's own logits.
"""
import pytest
import torch

from oracle import routing as OR
from uttt_amd import _lib as L
from uttt_amd import routing as RT

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cmp(ours, ref, k, logits_for_ties, bias=None):
    mask, gs, comb, bal, lb = ours
    rmask, rgs, rcomb, rbal, rlb = ref
    mask = mask.cpu()
    diff = (mask != rmask).any(1)                       # [B, T] tokens that differ
    if diff.any():
        sc = logits_for_ties if bias is None else logits_for_ties + bias
        top = sc.topk(k + 1, dim=1).values
        gap = (top[:, k - 1] - top[:, k])[diff]
        assert (gap.abs() < 1e-5).all(), f"selection differs away from a near tie: {gap}"
    else:
        assert torch.equal(gs.cpu(), rgs)
    torch.testing.assert_close(bal.cpu(), rbal, rtol=1e-5, atol=1e-7)
    ok = ~diff.unsqueeze(1).expand_as(rcomb)
    torch.testing.assert_close(comb.cpu()[ok], rcomb[ok], rtol=1e-5, atol=1e-7)
    if diff.any():
        # the counts differ at tied tokens: lb_loss from our group sizes
        E = rbal.shape[1]
        gm = gs.cpu().float().mean(0)
        rlb = (rbal.mean(0).mean(-1) * (gm / gm.sum())).sum() * E
    torch.testing.assert_close(lb.cpu(), rlb, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("E,k", [(16, 2), (32, 2), (7, 3), (128, 4)])
@pytest.mark.parametrize("rt", ["softmax", "norm_softmax", "norm_relu"])
@pytest.mark.parametrize("cm", ["selected_prob", "topk_renorm"])
def test_router_select(E, k, rt, cm):
    B, T = 2, 3001
    g = torch.Generator().manual_seed(E * 7 + k)
    logits = torch.randn(B, E, T, generator=g)
    bias = (torch.randn(1, E, 1, generator=g) * 0.5) if E != 7 else None
    kw = dict(alpha=0.8, router_type=rt, combine_mode=cm, routing_bias=bias)
    ours = RT.create_router_mask_sizes_probs(logits.to(DEV), k,
                                             **{**kw, "routing_bias": None if bias is None else bias.to(DEV)})
    ref = OR.create_router_mask_sizes_probs(logits, k, **kw)
    sel = logits if rt == "softmax" else None
    if rt != "softmax":
        n = logits.norm(dim=1, keepdim=True).clamp_min(1e-6)
        z = logits / n * (E ** 0.5)
        sel = z if rt == "norm_softmax" else z.clamp_min(0)
    if rt == "softmax":
        assert torch.equal(ours[0].cpu(), ref[0]) and torch.equal(ours[1].cpu(), ref[1])
    _cmp(ours, ref, k, sel, bias)


def test_router_select_strided_logits_and_batch_bias():
    # logits given as a [B, T, E] tensor viewed [B, E, T]; a per-batch bias
    B, T, E, k = 3, 700, 12, 2
    g = torch.Generator().manual_seed(3)
    lt = torch.randn(B, T, E, generator=g)
    bias = torch.randn(B, E, 1, generator=g)
    ours = RT.create_router_mask_sizes_probs(lt.to(DEV).transpose(1, 2), k, routing_bias=bias.to(DEV),
                                             combine_mode="topk_renorm")
    ref = OR.create_router_mask_sizes_probs(lt.transpose(1, 2), k, routing_bias=bias,
                                            combine_mode="topk_renorm")
    assert torch.equal(ours[0].cpu(), ref[0]) and torch.equal(ours[1].cpu(), ref[1])
    _cmp(ours, ref, k, lt.transpose(1, 2), bias)


@pytest.mark.parametrize("dtype,D,E,T", [(torch.bfloat16, 768, 16, 2048), (torch.bfloat16, 1536, 32, 1000),
                                         (torch.float32, 100, 5, 333)])
def test_route_tokens_fused(dtype, D, E, T):
    B, k = 1, 2
    g = torch.Generator().manual_seed(D + E)
    x = torch.randn(B, T, D, generator=g)
    x = (x / x.norm(dim=-1, keepdim=True)).to(dtype)
    Rw = torch.randn(E, D, generator=g)
    bias = torch.randn(1, E, 1, generator=g) * 0.5
    mask, gs, comb, bal, lg = RT.route_tokens(x.to(DEV), Rw.to(DEV), k, routing_bias=bias.to(DEV),
                                              combine_mode="topk_renorm", return_logits=True)
    ref_lg = OR.router_logits(x, Rw)
    scale = Rw.norm(dim=1).max().item() * x.float().norm(dim=-1).max().item()
    assert (lg.cpu().double() - ref_lg).abs().max().item() < 1e-4 * scale
    # the selection on the kernel's own logits is bit-exact
    ref = OR.create_router_mask_sizes_probs(lg.cpu(), k, routing_bias=bias, combine_mode="topk_renorm")
    assert torch.equal(mask.cpu(), ref[0]) and torch.equal(gs.cpu(), ref[1])
    torch.testing.assert_close(comb.cpu(), ref[2], rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(bal.cpu(), ref[3], rtol=1e-5, atol=1e-7)
    # and the fp64 logits select the same experts except at near ties
    ref64 = OR.create_router_mask_sizes_probs(ref_lg.float(), k, routing_bias=bias,
                                              combine_mode="topk_renorm")
    diff = (mask.cpu() != ref64[0]).any(1)
    if diff.any():
        top = (ref_lg + bias).topk(k + 1, dim=1).values
        assert ((top[:, k - 1] - top[:, k])[diff].abs() < 1e-4 * scale).all()
    _check_balance_sums(x, Rw, k, bias, mask, bal)


def _check_balance_sums(x, Rw, k, bias, mask, bal, **kw):
    """route_tokens_lb: the same routing plus the per-expert balance sums
    (the router's fixed-order reductions against torch's sum)."""
    m2, _, _, bal2, bsum = RT.route_tokens_lb(x.to(DEV), Rw.to(DEV), k, routing_bias=bias.to(DEV),
                                              combine_mode="topk_renorm", **kw)
    assert torch.equal(m2, mask) and torch.equal(bal2, bal)
    torch.testing.assert_close(bsum.cpu(), bal.cpu().sum(-1), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("B,T,D,E,k,dtype", [
    (8, 1, 1536, 32, 2, torch.bfloat16),   # the 760M decode step
    (3, 5, 768, 16, 2, torch.bfloat16),
    (4, 4, 768, 16, 2, torch.bfloat16),    # grouped loads, three chunks a group
    (1, 8, 1536, 32, 2, torch.bfloat16),   # grouped loads, two chunks, the most tokens
    (2, 3, 100, 64, 4, torch.float32),     # two experts per lane, ragged D
    (2, 7, 256, 128, 3, torch.bfloat16),   # matrix-core logits for E > 64
    (2, 40, 128, 7, 2, torch.bfloat16),    # two blocks per batch
])
@pytest.mark.parametrize("rt", ["softmax", "norm_softmax", "norm_relu"])
def test_route_tokens_few_tokens(B, T, D, E, k, dtype, rt):
    """Generation-sized batches (the vector-ALU logits) and every router type:
    the selection on the kernel's own logits against the oracle's."""
    g = torch.Generator().manual_seed(B * 1000 + T * 10 + E)
    x = torch.randn(B, T, D, generator=g)
    x = (x / x.norm(dim=-1, keepdim=True)).to(dtype)
    Rw = torch.randn(E, D, generator=g)
    bias = torch.randn(B, E, 1, generator=g) * 0.5
    mask, gs, comb, bal, lg = RT.route_tokens(x.to(DEV), Rw.to(DEV), k, routing_bias=bias.to(DEV),
                                              router_type=rt, combine_mode="topk_renorm",
                                              return_logits=True)
    ref_lg = OR.router_logits(x, Rw)
    scale = Rw.norm(dim=1).max().item() * x.float().norm(dim=-1).max().item()
    assert (lg.cpu().double() - ref_lg).abs().max().item() < 1e-4 * scale
    _check_balance_sums(x, Rw, k, bias, mask, bal, router_type=rt)
    own = lg.cpu()
    ref = OR.create_router_mask_sizes_probs(own, k, router_type=rt, routing_bias=bias,
                                            combine_mode="topk_renorm")
    # lb_loss of the same selection through the given-logits entry (one block per batch)
    lb = RT.create_router_mask_sizes_probs(lg, k, router_type=rt, routing_bias=bias.to(DEV),
                                           combine_mode="topk_renorm")[4]
    sel = own
    if rt != "softmax":
        z = own / own.norm(dim=1, keepdim=True).clamp_min(1e-6) * (E ** 0.5)
        sel = z if rt == "norm_softmax" else z.clamp_min(0)
    else:
        assert torch.equal(mask.cpu(), ref[0]) and torch.equal(gs.cpu(), ref[1])
    _cmp((mask, gs, comb, bal, lb), ref, k, sel, bias)


def test_router_errors():
    l = torch.randn(1, 4, 8, device=DEV)
    with pytest.raises(NotImplementedError):
        RT.create_router_mask_sizes_probs(l, 1, 1.0, True)
    with pytest.raises(ValueError):
        RT.create_router_mask_sizes_probs(l, 1, router_type="sigmoid")
    with pytest.raises(RuntimeError, match="topk"):
        RT.create_router_mask_sizes_probs(l, 5)


@pytest.mark.parametrize("B,T,D,E,k", [
    (1, 2048, 1536, 32, 2),   # one routed read at the 760M shape: two launches
    (2, 512, 768, 16, 2),
    (1, 20, 64, 8, 2),        # one selection block: the router's sums are final
    (1, 5000, 256, 16, 2),    # T > 4096: the general row map after the reduce
    (1, 1030, 128, 70, 3),    # E > 64 and T % 16 != 0
])
def test_route_tokens_map_equals_route_then_row_map(B, T, D, E, k):
    from uttt_amd.lact_moe_triton import triton_permute as TPM
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16).to(DEV)
    Rw = (torch.randn(E, D, generator=g) * D ** -0.5).to(DEV)
    bias = (torch.randn(E, generator=g) * 0.5).to(DEV)
    got = RT.route_tokens_map(x, Rw, k, routing_bias=bias, combine_mode="topk_renorm")
    ref = RT.route_tokens_lb(x, Rw, k, routing_bias=bias, combine_mode="topk_renorm")
    for a, b_ in zip(got[:4], ref[:4]):   # mask, group sizes, gates, balances
        assert torch.equal(a, b_)
    # the balance sums: the same partials added in another fixed order
    torch.testing.assert_close(got[4], ref[4], rtol=1e-6, atol=1e-6)
    rmap = TPM.make_row_id_map(ref[0], B, T, E)
    assert torch.equal(got[5], rmap)
    # deterministic
    again = RT.route_tokens_map(x, Rw, k, routing_bias=bias, combine_mode="topk_renorm")
    assert all(torch.equal(a, b_) for a, b_ in zip(again, got))


@pytest.mark.parametrize("B,T,D,E,k", [
    (1, 2048, 1536, 32, 2),   # the 760M routed read
    (2, 512, 768, 16, 2),
    (1, 4096, 256, 64, 4),    # the largest one-launch row map
    (1, 16, 64, 8, 2),
])
def test_route_tokens_map_src_rows_invert_the_row_map(B, T, D, E, k):
    """The inverse map: every routed (token, expert) row r of the row map has
    src_rows[b, r] == token, and the rows of a batch are T * k exactly."""
    assert RT.src_rows_supported(T, E) == bool(L.lib().uttt_route_tokens_map_src_rows(T, E))
    g = torch.Generator().manual_seed(3 * T + E)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16).to(DEV)
    Rw = (torch.randn(E, D, generator=g) * D ** -0.5).to(DEV)
    got = RT.route_tokens_map(x, Rw, k, combine_mode="topk_renorm", with_src_rows=True)
    plain = RT.route_tokens_map(x, Rw, k, combine_mode="topk_renorm")
    assert all(torch.equal(a, b_) for a, b_ in zip(got[:4], plain[:4]))
    assert torch.equal(got[5], plain[5])
    rmap, src = got[5].cpu(), got[6].cpu()
    assert src.shape == (B, T * k)
    n = rmap[:, :, 2 * E]                      # routed experts per token
    assert bool((n == k).all())
    rows = rmap[:, :, :k].long()               # each token's k rows
    tok = torch.arange(T)[None, :, None].expand(B, T, k)
    inv = torch.full((B, T * k), -1, dtype=torch.int32)
    inv.scatter_(1, rows.reshape(B, -1), tok.reshape(B, -1).to(torch.int32))
    assert torch.equal(src, inv)


def test_route_tokens_map_src_rows_refused_where_the_row_map_takes_more_launches():
    x = torch.randn(1, 5000, 64).to(torch.bfloat16).to(DEV)
    Rw = torch.randn(16, 64).to(DEV)
    assert not RT.src_rows_supported(5000, 16)
    with pytest.raises(RuntimeError, match="src_rows"):
        RT.route_tokens_map(x, Rw, 2, with_src_rows=True)

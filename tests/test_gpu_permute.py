"""GPU parity of the permute path: HIP kernels (through the C ABI via the
drop-in wrappers) against the C/torch oracle on the same seeded inputs.

Bar: bit-exact for the row map, group sizes, permuted payload bytes, permuted
probs, permute_kv_and_lrs outputs and the unpermute (fp32 fma accumulation in
slot order, one rounding); fp32 rtol/atol 1e-5 for the backward reductions
whose summation order the reference leaves to the compiler.
"""
import pytest
import torch

from oracle import permute as OP
from tests.helpers import load_golden, routing_c2, topk_mask_like_reference_test
from uttt_amd.lact_moe_triton import triton_permute as TP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bits(t):
    t = t.detach().cpu()
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def test_row_id_map_kat_on_gpu():
    kat = load_golden("row_id_map_kat.json")
    m = torch.tensor(kat["routing_map_token_major"], dtype=torch.int32).t().unsqueeze(0)
    rm = TP.make_row_id_map(m.to(DEV), 1, 5, 3).cpu()
    assert rm[0].tolist() == kat["expected_full"]


@pytest.mark.parametrize(
    "B,T,E,k,mask_dtype,ragged",
    [
        (1, 65536, 16, 2, torch.bool, False),   # the permute microbench shape
        (2, 4097, 32, 2, torch.int32, True),
        (3, 255, 7, 3, torch.bool, True),
        (1, 1, 1, 1, torch.bool, False),
        (1, 1000, 128, 4, torch.int32, True),
        (2, 300, 5, 5, torch.bool, False),      # every expert selected
        # one-launch row map (contiguous bool mask, T % 16 == 0, T <= 4096, E <= 64)
        (1, 2048, 32, 2, torch.bool, False),    # one apply's routing at the 760M shape
        (2, 2048, 32, 2, torch.bool, True),
        (1, 2048, 16, 2, torch.bool, True),     # the 124M shape
        (2, 4096, 64, 3, torch.bool, True),     # largest one-launch case: 16 tiles, E = 64
        (1, 1040, 7, 2, torch.bool, True),      # partial last tile and 64-token segment
        (1, 16, 3, 1, torch.bool, False),
        (1, 4096, 65, 2, torch.bool, False),    # E = 65 and T = 4112 take the three launches
        (1, 4112, 8, 2, torch.bool, True),
        # expert counts below their kernel's compile-time bucket
        (1, 2048, 20, 2, torch.bool, True),     # one launch, 32-expert bucket
        (1, 4096, 40, 3, torch.bool, True),     # one launch, 64-expert bucket
        (2, 5000, 20, 2, torch.bool, True),     # two launches, count rows padded to 32
        (1, 70000, 24, 4, torch.int32, False),  # two launches, E = 24, two count-table chunks
    ],
)
def test_row_id_map_bit_exact(B, T, E, k, mask_dtype, ragged):
    g = torch.Generator().manual_seed(B + T + E)
    scores = torch.rand(B, E, T, generator=g)
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, scores.topk(k, 1).indices, 1)
    if ragged:
        m = m * (torch.rand(B, E, T, generator=g) > 0.3).to(torch.int32)
        m[:, E // 2] = 0  # an empty expert
    gs = torch.empty(B, E, dtype=torch.int32, device=DEV)
    rm = TP.make_row_id_map(m.to(mask_dtype).to(DEV), B, T, E, group_sizes=gs)
    ref = OP.make_row_id_map(m)
    assert torch.equal(rm.cpu(), ref)
    assert torch.equal(gs.cpu(), m.sum(-1).to(torch.int32))


def test_row_id_map_strided_mask():
    # a [B, T, E] tensor viewed as [B, E, T]: the kernel honours strides
    g = torch.Generator().manual_seed(3)
    B, T, E = 2, 1500, 12
    m = torch.zeros(B, T, E, dtype=torch.int32).scatter_(2, torch.rand(B, T, E, generator=g).topk(2, 2).indices, 1)
    view = m.to(DEV).transpose(1, 2)
    assert not view.is_contiguous()
    rm = TP.make_row_id_map(view, B, T, E)
    assert torch.equal(rm.cpu(), OP.make_row_id_map(m.transpose(1, 2).contiguous()))


def test_row_id_map_deterministic():
    _, _, mask, _, _ = routing_c2(T=65536, E=16, k=2, seed=1)
    md = mask.to(DEV)
    a = TP.make_row_id_map(md, 1, 65536, 16)
    b = TP.make_row_id_map(md, 1, 65536, 16)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 768), (torch.float32, 16), (torch.bfloat16, 900), (torch.float16, 130)])
def test_permute_fwd_bit_exact(dtype, H):
    T, E, k = (65536, 16, 2) if H == 768 else (2000, 6, 2)
    _, _, mask, gs, comb = routing_c2(T=T, E=E, k=k, seed=2)
    comb = comb.clone()
    comb[0, :, 5] = 0.0  # padding slots -> zero rows
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, T, H, generator=g).to(dtype)
    out, pp, rm = TP.permute_with_expert_mask(x.to(DEV), mask.to(DEV), comb.to(DEV), k)
    ref_rm = OP.make_row_id_map(mask)
    assert torch.equal(rm.cpu(), ref_rm)
    ref_out, ref_pp = OP.permute(x, ref_rm, comb, k * T)
    wr = OP.written_rows(ref_rm, k * T)
    assert torch.equal(bits(out)[wr], bits(ref_out)[wr])
    assert torch.equal(pp.cpu()[wr], ref_pp[wr])


def test_permute_without_probs_and_few_slots():
    # the reference test's mask keeps k-1 experts: tail rows stay unwritten
    g = torch.Generator().manual_seed(321)
    B, T, E, H, k = 2, 32, 4, 16, 2
    mask = topk_mask_like_reference_test(B, T, E, k, g)
    x = torch.randn(B, T, H, generator=g)
    out, pp, rm = TP.permute_with_expert_mask(x.to(DEV), mask.to(DEV), None, k)
    assert pp is None
    ref_rm = OP.make_row_id_map(mask)
    ref_out, _ = OP.permute(x, ref_rm, None, k * T)
    wr = OP.written_rows(ref_rm, k * T)
    assert torch.equal(out.cpu()[wr], ref_out[wr])


def test_unpermute_reference_invariant():
    # uttt_nvs/tests/test_triton_permute.py:32-53 on our kernels
    g = torch.Generator().manual_seed(321)
    B, T, E, H, k = 2, 32, 4, 16, 2
    mask = topk_mask_like_reference_test(B, T, E, k, g)
    x = torch.randn(B, T, H, generator=g)
    probs = torch.rand(B, E, T, generator=g) * mask
    xp, _, rm = TP.permute_with_expert_mask(x.to(DEV), mask.to(DEV), probs.to(DEV), k)
    merged = TP.unpermute_and_merge_with_probs(xp, rm, probs.to(DEV))
    ref = x * (probs * mask).sum(dim=1).unsqueeze(-1)
    torch.testing.assert_close(merged.cpu(), ref, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("dtype,H,T,E", [(torch.bfloat16, 768, 65536, 16), (torch.float32, 48, 3000, 9)])
def test_unpermute_fwd_bit_exact(dtype, H, T, E):
    k = 2
    _, _, mask, gs, comb = routing_c2(T=T, E=E, k=k, seed=4)
    g = torch.Generator().manual_seed(9)
    rm = OP.make_row_id_map(mask)
    y = torch.randn(1, k * T, H, generator=g).to(dtype)
    out = TP.unpermute_and_merge_with_probs(y.to(DEV), rm.to(DEV), comb.to(DEV))
    ref = OP.unpermute(y, rm, comb, T)
    assert torch.equal(bits(out), bits(ref))


@pytest.mark.parametrize("dtype,H", [(torch.bfloat16, 256), (torch.float32, 36)])
def test_permute_unpermute_topk4_ragged(dtype, H):
    # top-4 with dropped slots: slots past the first two take the kernels'
    # general loop, tokens with 0..4 slots mix within one wave
    B, T, E, k = 2, 1537, 12, 4
    g = torch.Generator().manual_seed(17)
    scores = torch.rand(B, E, T, generator=g)
    mask = torch.zeros(B, E, T, dtype=torch.bool).scatter_(1, scores.topk(k, 1).indices, True)
    mask &= torch.rand(B, E, T, generator=g) > 0.25
    probs = torch.rand(B, E, T, generator=g) * mask
    probs[:, :, 3] = 0.0  # a token whose every gate is zero
    x = torch.randn(B, T, H, generator=g).to(dtype)
    out, pp, rm = TP.permute_with_expert_mask(x.to(DEV), mask.to(DEV), probs.to(DEV), k)
    ref_rm = OP.make_row_id_map(mask)
    assert torch.equal(rm.cpu(), ref_rm)
    ref_out, ref_pp = OP.permute(x, ref_rm, probs, k * T)
    wr = OP.written_rows(ref_rm, k * T)
    assert torch.equal(bits(out)[wr], bits(ref_out)[wr])
    assert torch.equal(pp.cpu()[wr], ref_pp[wr])
    y = torch.randn(B, k * T, H, generator=g).to(dtype)
    merged = TP.unpermute_and_merge_with_probs(y.to(DEV), rm, probs.to(DEV))
    assert torch.equal(bits(merged), bits(OP.unpermute(y, ref_rm, probs, T)))


def test_unpermute_strided_probs():
    # probs given as a [B, T, E] tensor viewed [B, E, T] (P:835-839)
    T, E, H, k = 1000, 8, 64, 2
    _, _, mask, _, comb = routing_c2(T=T, E=E, k=k, seed=5)
    g = torch.Generator().manual_seed(10)
    rm = OP.make_row_id_map(mask)
    y = torch.randn(1, k * T, H, generator=g).to(torch.bfloat16)
    pv = comb.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    out = TP.unpermute_and_merge_with_probs(y.to(DEV), rm.to(DEV), pv)
    assert torch.equal(bits(out), bits(OP.unpermute(y, rm, comb, T)))


def test_permute_unpermute_backward():
    T, E, H, k = 3000, 8, 96, 2
    _, _, mask, _, comb = routing_c2(T=T, E=E, k=k, seed=6)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, T, H, generator=g)
    xd = x.to(DEV).requires_grad_(True)
    pd = comb.to(DEV).requires_grad_(True)
    xp, pp, rm = TP.permute_with_expert_mask(xd, mask.to(DEV), pd, k)
    gy = torch.randn(1, k * T, H, generator=g)
    gpp = torch.randn(1, k * T, generator=g)
    (xp * gy.to(DEV)).sum().add((pp * gpp.to(DEV)).sum()).backward()
    rm_c = rm.cpu()
    gi, gp = OP.permute_bwd(gy, rm_c, gpp, T)
    torch.testing.assert_close(xd.grad.cpu(), gi, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(pd.grad.cpu(), gp, rtol=1e-5, atol=1e-5)

    y = torch.randn(1, k * T, H, generator=g)
    yd = y.to(DEV).requires_grad_(True)
    pd2 = comb.to(DEV).requires_grad_(True)
    out = TP.unpermute_and_merge_with_probs(yd, rm, pd2)
    go = torch.randn(1, T, H, generator=g)
    (out * go.to(DEV)).sum().backward()
    ag, gp2 = OP.unpermute_bwd(go, rm_c, y, comb)
    wr = OP.written_rows(rm_c, k * T)
    torch.testing.assert_close(yd.grad.cpu()[wr], ag[wr], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(pd2.grad.cpu(), gp2, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("kd,vd,lrd,H,T,E", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16, 768, 2048, 16),
    (torch.bfloat16, torch.float32, torch.float32, 1536, 2048, 32),
    (torch.float32, torch.float32, torch.float32, 50, 777, 5),
])
def test_permute_kv_and_lrs_bit_exact(kd, vd, lrd, H, T, E):
    k = 2
    _, _, mask, _, comb = routing_c2(T=T, E=E, k=k, seed=8)
    g = torch.Generator().manual_seed(12)
    kx = torch.randn(1, T, H, generator=g).to(kd)
    vx = torch.randn(1, T, H, generator=g).to(vd)
    lrs = [torch.sigmoid(torch.randn(1, T, generator=g)).mul(0.1).to(lrd) for _ in range(3)]
    outs = TP.permute_kv_and_lrs(kx.to(DEV), vx.to(DEV), *(l.to(DEV) for l in lrs),
                                 mask.to(torch.int32).to(DEV), comb.to(DEV), k)
    rm = OP.make_row_id_map(mask)
    refs = OP.permute_kv_lrs(kx, vx, *lrs, rm, comb, k * T)
    wr = OP.written_rows(rm, k * T)
    for o, r in zip(outs, refs):
        assert torch.equal(bits(o)[wr], bits(r)[wr])


def test_permute_kv_and_lrs_3d_lr_and_backward():
    T, E, H, k = 1500, 8, 64, 2
    _, _, mask, _, comb = routing_c2(T=T, E=E, k=k, seed=9)
    comb = comb.clone()
    comb[0, :, 11] = 0.0
    g = torch.Generator().manual_seed(13)
    kx = torch.randn(1, T, H, generator=g)
    vx = torch.randn(1, T, H, generator=g)
    lrs = [torch.rand(1, T, 1, generator=g) for _ in range(3)]
    kd, vd = kx.to(DEV).requires_grad_(True), vx.to(DEV).requires_grad_(True)
    lds = [l.to(DEV).requires_grad_(True) for l in lrs]
    pd = comb.to(DEV).requires_grad_(True)
    outs = TP.permute_kv_and_lrs(kd, vd, *lds, mask.to(DEV), pd, k)
    assert outs[2].shape == (1, k * T)
    grads = [torch.randn(o.shape, generator=g) for o in outs]
    sum((o * gg.to(DEV)).sum() for o, gg in zip(outs, grads)).backward()
    rm = OP.make_row_id_map(mask)
    grad_k, grad_v, grad_lr, gp = OP.permute_kv_lrs_bwd(grads[0], grads[1], grads[2:], rm, vx, comb, T)
    torch.testing.assert_close(kd.grad.cpu(), grad_k, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(vd.grad.cpu(), grad_v, rtol=1e-5, atol=1e-5)
    for ld, gr in zip(lds, grad_lr):
        assert ld.grad.shape == (1, T, 1)
        torch.testing.assert_close(ld.grad.cpu().squeeze(-1), gr, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(pd.grad.cpu(), gp, rtol=1e-5, atol=1e-4)


def test_permute_roundtrip_full_size_property():
    # full-size property check: unpermute(permute(x)) with unit-sum gates
    # reproduces x up to one bf16 rounding of sum_j x*p_j
    T, E, k, H = 65536, 16, 2, 768
    _, _, mask, _, comb = routing_c2(T=T, E=E, k=k, seed=10)
    g = torch.Generator().manual_seed(14)
    x = torch.randn(1, T, H, generator=g).to(torch.bfloat16).to(DEV)
    xp, _, rm = TP.permute_with_expert_mask(x, mask.to(DEV), comb.to(DEV), k)
    back = TP.unpermute_and_merge_with_probs(xp, rm, comb.to(DEV))
    torch.testing.assert_close(back.float(), x.float(), rtol=1e-2, atol=1e-2)

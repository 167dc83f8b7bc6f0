"""CPU checks that pin the permute oracle before it is trusted as the checker.

- row map: the reference's worked example (golden vector) and a brute-force
  statement of the closed form (expert-major, token-ascending destinations);
- permute/unpermute: the reference's own invariant
  unpermute(permute(x), p) == x * sum_e p_e m_e (uttt_nvs/tests/
  test_triton_permute.py:32-53) and byte equality of the copies;
- backward passes: torch autograd through an explicit 0/1 permutation matrix;
- permute_kv_and_lrs: the reference's composition route
  (_reference_permute_kv_and_lrs, triton_permute.py:2039-2080).
"""
import numpy as np
import pytest
import torch

from oracle import permute as OP
from tests.helpers import load_golden, topk_mask_like_reference_test


def brute_row_id_map(mask):
    """Closed form: row(e,t) = sum of counts of experts < e + rank of t in e.
    Column layout as left by the reference's passes 2 and 3."""
    B, E, T = mask.shape
    W = 2 * E + 1
    out = np.zeros((B, T, W), dtype=np.int64)
    for b in range(B):
        m = mask[b].numpy().astype(bool)
        cnt = m.sum(1)
        off = np.concatenate([[0], np.cumsum(cnt)[:-1]])
        row = np.full((E, T), -1)
        for e in range(E):
            ts = np.nonzero(m[e])[0]
            row[e, ts] = off[e] + np.arange(len(ts))
        for t in range(T):
            routed = [e for e in range(E) if m[e, t]]
            n = len(routed)
            out[b, t, :E] = row[:, t]
            for j, e in enumerate(sorted(routed, reverse=True)):
                out[b, t, j] = row[e, t]
                out[b, t, E + j] = e
            out[b, t, 2 * E] = n
    return torch.from_numpy(out.astype(np.int32))


def test_row_id_map_golden_kat():
    kat = load_golden("row_id_map_kat.json")
    m = torch.tensor(kat["routing_map_token_major"], dtype=torch.int32).t().unsqueeze(0)
    got = OP.make_row_id_map(m)[0]
    for t, row in enumerate(kat["expected_defined"]):
        for c, v in enumerate(row):
            if v is not None:
                assert got[t, c].item() == v, (t, c, got[t].tolist())
    assert got.tolist() == kat["expected_full"]


def test_row_id_map_second_kat_batch_matches_closed_form():
    kat = load_golden("row_id_map_kat.json")
    rows = [kat["routing_map_token_major"], kat["second_batch_token_major_from_P:1143-1158"]]
    m = torch.tensor(rows, dtype=torch.int32).transpose(1, 2).contiguous()
    assert torch.equal(OP.make_row_id_map(m), brute_row_id_map(m))


@pytest.mark.parametrize("B,T,E,k", [(1, 7, 1, 1), (2, 513, 3, 2), (3, 1100, 8, 2), (1, 600, 5, 4)])
def test_row_id_map_matches_closed_form(B, T, E, k):
    g = torch.Generator().manual_seed(B * 1000 + T + E)
    scores = torch.rand(B, E, T, generator=g)
    idx = scores.topk(k, dim=1).indices
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, idx, 1)
    # ragged: drop some selections so tokens have 0..k experts
    m = m * (torch.rand(B, E, T, generator=g) > 0.2).to(torch.int32)
    assert torch.equal(OP.make_row_id_map(m), brute_row_id_map(m))


def test_permute_unpermute_invariant_like_reference_test():
    # uttt_nvs/tests/test_triton_permute.py:32-53 (B=2, T=32, E=4, H=16, k=2, fp32)
    g = torch.Generator().manual_seed(321)
    B, T, E, H, k = 2, 32, 4, 16, 2
    mask = topk_mask_like_reference_test(B, T, E, k, g)
    x = torch.randn(B, T, H, generator=g)
    probs = torch.rand(B, E, T, generator=g) * mask
    rm = OP.make_row_id_map(mask)
    xp, pp = OP.permute(x, rm, probs, k * T)
    merged = OP.unpermute(xp, rm, probs, T)
    ref = x * (probs * mask).sum(dim=1).unsqueeze(-1)
    torch.testing.assert_close(merged, ref, atol=1e-3, rtol=1e-3)


def test_permute_copies_bytes_and_zero_rows():
    g = torch.Generator().manual_seed(5)
    B, T, E, H, k = 2, 300, 6, 40, 2
    scores = torch.rand(B, E, T, generator=g)
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, scores.topk(k, 1).indices, 1)
    probs = torch.rand(B, E, T, generator=g) * m
    probs[0, :, 7] = 0.0  # a token whose slots are padding: rows must be zero
    x = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    rm = OP.make_row_id_map(m)
    xp, pp = OP.permute(x, rm, probs, k * T)
    E_ = E
    for b in range(B):
        for t in range(T):
            n = rm[b, t, 2 * E_].item()
            for j in range(n):
                row, e = rm[b, t, j].item(), rm[b, t, E_ + j].item()
                assert pp[b, row].item() == probs[b, e, t].item()
                want = torch.zeros_like(x[b, t]) if probs[b, e, t] == 0 else x[b, t]
                assert torch.equal(xp[b, row].view(torch.int16), want.view(torch.int16))


def _perm_matrix(rm, num_out, T):
    """Dense 0/1 matrices P[b] (num_out x T) and the (row, expert, token) list."""
    B, _, W = rm.shape
    E = (W - 1) // 2
    P = torch.zeros(B, num_out, T, dtype=torch.float64)
    ent = []
    for b in range(B):
        for t in range(T):
            for j in range(rm[b, t, 2 * E].item()):
                r, e = rm[b, t, j].item(), rm[b, t, E + j].item()
                P[b, r, t] = 1.0
                ent.append((b, r, e, t))
    return P, ent


def test_permute_bwd_matches_autograd():
    g = torch.Generator().manual_seed(11)
    B, T, E, H, k = 2, 40, 5, 12, 2
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, torch.rand(B, E, T, generator=g).topk(k, 1).indices, 1)
    rm = OP.make_row_id_map(m)
    num_out = k * T
    P, ent = _perm_matrix(rm, num_out, T)
    gout = torch.randn(B, num_out, H, generator=g, dtype=torch.float64)
    gpp = torch.randn(B, num_out, generator=g, dtype=torch.float64)
    x = torch.zeros(B, T, H, dtype=torch.float64, requires_grad=True)
    probs = torch.rand(B, E, T, generator=g, dtype=torch.float64).requires_grad_(True)
    out = torch.bmm(P, x)
    pp = torch.zeros(B, num_out, dtype=torch.float64)
    for (b, r, e, t) in ent:
        pp = pp.index_put((torch.tensor([b]), torch.tensor([r])), probs[b, e, t].reshape(1))
    (out * gout).sum().add((pp * gpp).sum()).backward()
    gi, gp = OP.permute_bwd(gout.float(), rm, gpp.float(), T)
    torch.testing.assert_close(gi, x.grad.float(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gp, probs.grad.float(), rtol=1e-5, atol=1e-5)


def test_unpermute_bwd_matches_autograd():
    g = torch.Generator().manual_seed(12)
    B, T, E, H, k = 2, 40, 5, 12, 2
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, torch.rand(B, E, T, generator=g).topk(k, 1).indices, 1)
    rm = OP.make_row_id_map(m)
    num_out = k * T
    _, ent = _perm_matrix(rm, num_out, T)
    y = torch.randn(B, num_out, H, generator=g, dtype=torch.float64, requires_grad=True)
    probs = torch.rand(B, E, T, generator=g, dtype=torch.float64).requires_grad_(True)
    out = torch.zeros(B, T, H, dtype=torch.float64)
    for (b, r, e, t) in ent:
        out = out.index_put((torch.tensor([b]), torch.tensor([t])),
                            (y[b, r] * probs[b, e, t]).unsqueeze(0), accumulate=True)
    gout = torch.randn(B, T, H, generator=g, dtype=torch.float64)
    (out * gout).sum().backward()
    ag, gp = OP.unpermute_bwd(gout.float(), rm, y.detach().float(), probs.detach().float())
    wr = OP.written_rows(rm, num_out)
    torch.testing.assert_close(ag[wr], y.grad.float()[wr], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gp, probs.grad.float(), rtol=1e-5, atol=1e-5)


def test_permute_kv_lrs_matches_reference_composition():
    # _reference_permute_kv_and_lrs: permute k and v with the same map, then
    # v_p * permuted_probs rounded to k's dtype; lrs permuted as [B,T,1].
    g = torch.Generator().manual_seed(13)
    B, T, E, H, k = 2, 64, 4, 24, 2
    probs = torch.rand(B, E, T, generator=g)
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, probs.topk(k, 1).indices, 1)
    kx = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    vx = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    lrs = [torch.rand(B, T, generator=g).to(torch.bfloat16) for _ in range(3)]
    rm = OP.make_row_id_map(m)
    num_out = k * T
    ko, vo, l0, l1, l2 = OP.permute_kv_lrs(kx, vx, *lrs, rm, probs, num_out)
    kp, pp = OP.permute(kx, rm, probs, num_out)
    vp, _ = OP.permute(vx, rm, probs, num_out)
    vref = (vp * pp.unsqueeze(-1)).to(torch.bfloat16)
    wr = OP.written_rows(rm, num_out)
    assert torch.equal(ko[wr].view(torch.int16), kp[wr].view(torch.int16))
    assert torch.equal(vo[wr].view(torch.int16), vref[wr].view(torch.int16))
    for lo, li in zip((l0, l1, l2), lrs):
        lp, _ = OP.permute(li.unsqueeze(-1), rm, None, num_out)
        assert torch.equal(lo[wr].view(torch.int16), lp.squeeze(-1)[wr].view(torch.int16))


def test_permute_kv_lrs_bwd_matches_autograd():
    g = torch.Generator().manual_seed(14)
    B, T, E, H, k = 1, 30, 4, 10, 2
    probs = torch.rand(B, E, T, generator=g, dtype=torch.float64)
    m = torch.zeros(B, E, T, dtype=torch.int32).scatter_(1, probs.topk(k, 1).indices, 1)
    probs = (probs * m)
    probs[0, :, 3] = 0.0  # padding slots: prob grad must be zero there
    probs.requires_grad_(True)
    rm = OP.make_row_id_map(m)
    num_out = k * T
    _, ent = _perm_matrix(rm, num_out, T)
    kx = torch.randn(B, T, H, generator=g, dtype=torch.float64, requires_grad=True)
    vx = torch.randn(B, T, H, generator=g, dtype=torch.float64, requires_grad=True)
    lr = [torch.rand(B, T, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3)]
    gk = torch.randn(B, num_out, H, generator=g, dtype=torch.float64)
    gv = torch.randn(B, num_out, H, generator=g, dtype=torch.float64)
    glr = [torch.randn(B, num_out, generator=g, dtype=torch.float64) for _ in range(3)]
    loss = 0
    for (b, r, e, t) in ent:
        loss = loss + (kx[b, t] * gk[b, r]).sum() + (vx[b, t] * probs[b, e, t] * gv[b, r]).sum()
        for i in range(3):
            loss = loss + lr[i][b, t] * glr[i][b, r]
    loss.backward()
    grad_k, grad_v, grad_lr, gp = OP.permute_kv_lrs_bwd(
        gk.float(), gv.float(), [x.float() for x in glr], rm, vx.detach().float(),
        probs.detach().float(), T)
    torch.testing.assert_close(grad_k, kx.grad.float(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(grad_v, vx.grad.float(), rtol=1e-5, atol=1e-5)
    for a, x in zip(grad_lr, lr):
        torch.testing.assert_close(a, x.grad.float(), rtol=1e-5, atol=1e-5)
    # the reference zeroes the prob grad of padding slots (p == 0): autograd
    # would not, so compare the non-padding entries and check the zeros
    pad = probs.detach() == 0
    torch.testing.assert_close(gp[~pad], probs.grad.float()[~pad], rtol=1e-5, atol=1e-5)
    assert (gp[pad] == 0).all()

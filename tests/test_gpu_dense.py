"""GPU parity of the uTTT-Dense path (uttt_amd.dense) against oracle/dense.py
on the same seeded inputs at the configs[0] head shape (H = 4, d = 96,
d_h = 192, chunks of 512) and the configs[1] shape (d = 192, d_h = 384).

Bar: bf16 outputs and weights within rtol 2e-2 (tests.helpers.assert_bf16_close)
of the oracle run with the reference's bf16 storage points; raw updates
(bf16 stored, widened) the same; the fp32 masters of a multi-chunk sweep
within rtol 2e-2 as well (each write consumes bf16 updates).
"""
import pytest
import torch

from oracle import dense as OD
from tests.helpers import assert_bf16_close
from uttt_amd import dense as DN

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weights(b, H, d, r, seed=0):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(*s, generator=g) / d ** 0.5
                 for s in ((b, H, r * d, d), (b, H, d, r * d), (b, H, r * d, d)))


def _layer(b, S, H, d, seed, per_head_lr=False):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.nn.functional.normalize(torch.randn(b, S, H, d, generator=g), dim=-1)
               .reshape(b, S, H * d).to(torch.bfloat16) for _ in range(3))
    lr = torch.sigmoid(torch.randn(b, S, 3 * H if per_head_lr else 3, generator=g)) * 0.1
    return q, k, v, lr


@pytest.mark.parametrize("H,d,r,l", [(4, 96, 2, 512), (4, 192, 2, 2048), (2, 64, 3, 300)])
def test_dense_read_and_update(H, d, r, l):
    b = 1
    w = _weights(b, H, d, r)
    fast = tuple(x.to(torch.bfloat16) for x in w)
    q, k, v, lr = _layer(b, l, H, d, 1, per_head_lr=(r == 3))
    out = DN.apply_fast_weights(q.to(DEV), *(x.to(DEV) for x in fast))
    assert_bf16_close(out.cpu(), OD.read(q, *fast), name="read")
    dws = DN.compute_update(k.to(DEV), v.to(DEV), lr.to(DEV), tuple(x.to(DEV) for x in fast))
    refs = OD.compute_update(k, v, lr, fast)
    for o, rr, n in zip(dws, refs, ("dw0", "dw1", "dw2")):
        assert o.dtype == torch.float32
        assert_bf16_close(o.cpu(), rr, name=n)


@pytest.mark.parametrize("H,d,r,l", [(4, 192, 2, 1), (4, 96, 2, 8), (2, 64, 3, 3)])
def test_dense_read_few_tokens(H, d, r, l):
    """Generation-sized reads take the decode kernels: against the oracle and
    against the grouped path (one token more than the decode limit)."""
    b = 2
    fast = tuple(x.to(torch.bfloat16) for x in _weights(b, H, d, r, seed=3))
    q = _layer(b, l, H, d, 4)[0]
    out = DN.apply_fast_weights(q.to(DEV), *(x.to(DEV) for x in fast))
    assert out.shape == (b, l, H * d)
    assert_bf16_close(out.cpu(), OD.read(q, *fast), name="decode-size read")
    q9 = _layer(b, DN.DECODE_TOKENS + 1, H, d, 5)[0]
    q9[:, :l] = q
    grouped = DN.apply_fast_weights(q9.to(DEV), *(x.to(DEV) for x in fast))[:, :l]
    assert_bf16_close(out, grouped, name="decode kernels vs grouped path")


@pytest.mark.parametrize("L,S,chunk,H,d,r,master_renorm", [
    (1, 4096, 512, 4, 96, 2, False),     # configs[0]: one layer, 8 chunks
    (3, 1536, 512, 4, 96, 2, True),      # aggregate over layers, master renorm
])
def test_dense_sweep(L, S, chunk, H, d, r, master_renorm):
    b = 1
    w = _weights(b, H, d, r, seed=5)
    fast = tuple(x.to(torch.bfloat16) for x in w)
    layers = [_layer(b, S, H, d, 100 + i) for i in range(L)]
    qs, ks, vs, lrs = (list(t) for t in zip(*layers))
    ref_out, ref_fast, ref_master = OD.sweep(qs, ks, vs, lrs, fast, w, r, chunk,
                                             master_renorm=master_renorm)
    bank = DN.SharedFastWeights(*(x.to(DEV) for x in fast), r=r,
                                masters=tuple(x.to(DEV) for x in w), master_renorm=master_renorm)
    outs = [[] for _ in range(L)]
    for c0 in range(0, S, chunk):
        c1 = min(S, c0 + chunk)
        for li in range(L):
            outs[li].append(bank.read(qs[li][:, c0:c1].to(DEV)))
        if c1 < S:
            bank.write([k[:, c0:c1].to(DEV) for k in ks], [v[:, c0:c1].to(DEV) for v in vs],
                       [x[:, c0:c1].to(DEV) for x in lrs])
    torch.cuda.synchronize()
    for li in range(L):
        assert_bf16_close(torch.cat(outs[li], 1).cpu(), ref_out[li], name=f"out{li}")
    f, m = bank.weights()
    for a, rr, n in zip(f, ref_fast, ("w0", "w1", "w2")):
        assert_bf16_close(a.cpu(), rr, name="fast " + n)
    for a, rr, n in zip(m, ref_master, ("w0", "w1", "w2")):
        assert_bf16_close(a.cpu(), rr, name="master " + n)


@pytest.mark.parametrize("b,l,H,d,per_head,lr_dtype", [
    (2, 37, 4, 24, False, torch.float32),   # ragged token count, shared lr
    (1, 2048, 4, 192, True, torch.bfloat16),  # the 124M head shape, per-head lr
])
def test_gather_and_scatter_heads_are_exact(b, l, H, d, per_head, lr_dtype):
    """The head layout kernels move bytes: equal to torch's rearranges
    (D:251, :261, :370-398) bit for bit, three layers gathered at once."""
    g = torch.Generator().manual_seed(l)
    ks = [torch.randn(b, l, H * d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    vs = [torch.randn(b, l, H * d, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    lrs = [torch.rand(b, l, 3 * H if per_head else 3, generator=g).to(lr_dtype).to(DEV)
           for _ in range(3)]
    kh, vh, lr3 = DN._gather_heads(ks, vs, lrs, H)
    split = lambda x: x.reshape(b, l, H, d).permute(0, 2, 1, 3).reshape(b * H, l, d)
    assert torch.equal(kh, torch.cat([split(k) for k in ks], dim=1))
    assert torch.equal(vh, torch.cat([split(v) for v in vs], dim=1))
    for j in range(3):
        cols = [(lr.reshape(b, l, H, 3)[..., j] if per_head else
                 lr[..., j:j + 1].expand(b, l, H)).permute(0, 2, 1).reshape(b * H, l).float()
                for lr in lrs]
        assert torch.equal(lr3[j], torch.cat(cols, dim=1))
    y = torch.randn(b * H, l, d, generator=g).to(torch.bfloat16).to(DEV)
    out = DN._unheads(y, b, H)
    assert torch.equal(out, y.reshape(b, H, l, d).permute(0, 2, 1, 3).reshape(b, l, H * d))


@pytest.mark.parametrize("b,H,d,dh,l", [
    (1, 4, 192, 384, 2048),   # 124M: 12 hidden blocks, 3 per wave
    (2, 3, 128, 96, 77),      # 3 hidden blocks (one wave idle), ragged token tile
    (1, 2, 256, 512, 64),     # 4 blocks per wave, the largest head
    (3, 1, 64, 32, 9),        # one hidden block, one partial tile
])
def test_fused_dense_read(b, H, d, dh, l):
    """csrc/dense_read.hip (fused read for small heads) against the oracle
    and against the grouped route (head split, grouped APPLY, merge)."""
    from uttt_amd import _lib as L
    from uttt_amd.lact_moe_triton import _grouped as G

    assert L.lib().uttt_dense_read_supported(d, dh)
    g = torch.Generator().manual_seed(l + d)
    w0, w2 = ((torch.randn(b, H, dh, d, generator=g) / d ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    w1 = (torch.randn(b, H, d, dh, generator=g) / dh ** 0.5).to(torch.bfloat16)
    q = torch.randn(b, l, H * d, generator=g).to(torch.bfloat16)
    out = DN.apply_fast_weights(q.to(DEV), w0.to(DEV), w1.to(DEV), w2.to(DEV))
    assert out.shape == (b, l, H * d) and out.dtype == torch.bfloat16
    assert_bf16_close(out.cpu(), OD.read(q, w0, w1, w2), name="fused read")
    W02 = torch.cat([w0, w2], dim=2).reshape(b * H, 1, 2 * dh, d).to(DEV)
    W1 = w1.reshape(b * H, 1, d, dh).to(DEV)
    xh = DN._heads(q.to(DEV), H)
    gs = DN._gs(b * H, l, DEV)
    grouped = DN._unheads(G.gemm_nt(W1, G.gate_up(W02, xh, gs, token_major=True), gs), b, H)
    assert_bf16_close(out, grouped, name="fused read vs grouped route")


@pytest.mark.parametrize("b,H,d,dh,l", [
    (1, 4, 96, 192, 512),     # configs[0]
    (1, 4, 192, 384, 2048),   # configs[1]
    (2, 3, 128, 96, 77),
    (1, 2, 256, 512, 64),
    (3, 1, 64, 32, 9),
])
def test_packed_dense_read_is_bit_identical(b, H, d, dh, l):
    """The read from the fragment-ordered weight copy (uttt_dense_pack_weights
    + uttt_dense_read_packed) against the read from the weights as stored:
    the same operands in the same MFMAs, so the same bits; and the shared
    bank's reads after a write (the copy is rebuilt) against a fresh read."""
    g = torch.Generator().manual_seed(3 * l + d)
    w0, w2 = ((torch.randn(b, H, dh, d, generator=g) / d ** 0.5).to(torch.bfloat16)
              for _ in range(2))
    w1 = (torch.randn(b, H, d, dh, generator=g) / dh ** 0.5).to(torch.bfloat16)
    q = torch.randn(b, l, H * d, generator=g).to(torch.bfloat16).to(DEV)
    W02 = torch.cat([w0, w2], dim=2).reshape(b * H, 1, 2 * dh, d).contiguous().to(DEV)
    W1 = w1.reshape(b * H, 1, d, dh).contiguous().to(DEV)
    ref = DN._read(q, W02, W1, b, H)
    P = DN._pack(W02, W1)
    assert P is not None and P.numel() == b * H * 3 * dh * d
    got = DN._read_packed(q, P, W02, W1, b, H)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if dh % d == 0:
        # one-layer write: the first read uses W02/W1, the second the copy
        # packed then; two-layer write: the copy is packed at the write
        bank = DN.SharedFastWeights(w0.to(DEV), w1.to(DEV), w2.to(DEV), dh // d)
        for n_layers in (1, 2, 1):
            lay = [_layer(b, l, H, d, 5 + i) for i in range(n_layers)]
            bank.write([x[1].to(DEV) for x in lay], [x[2].to(DEV) for x in lay],
                       [x[3].to(DEV) for x in lay])
            ref2 = DN._read(q, bank.W02, bank.W1, b, H)
            for _ in range(2):
                got2 = bank.read(q)
                torch.cuda.synchronize()
                assert torch.equal(got2.view(torch.int16), ref2.view(torch.int16)), n_layers


@pytest.mark.parametrize("BH,N,d,dh,with_lr", [
    (4, 3000, 192, 384, True),   # configs[1] head, ragged token tiles
    (4, 1024, 96, 192, True),    # configs[0] head
    (2, 77, 128, 96, True),      # one partial tile
    (3, 128, 64, 32, False),     # one hidden block, lr = 1
    (1, 513, 256, 512, True),    # the largest head
])
def test_fused_dense_update_stage1(BH, N, d, dh, with_lr):
    """csrc/dense_update.hip (fused stage 1 for small heads: Y0, Y2, DH on
    MFMA, the SwiGLU-derivative epilogue in registers) against the grouped
    stage 1 with one expert (the same rounding points: fp32 Y and DH, one
    bf16 rounding of each output)."""
    from uttt_amd import _lib as L
    from uttt_amd.lact_moe_triton import _grouped as G

    assert L.lib().uttt_dense_update_supported(d, dh)
    g = torch.Generator().manual_seed(N + d)
    W02 = (torch.randn(BH, 1, 2 * dh, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(DEV)
    W1 = (torch.randn(BH, 1, d, dh, generator=g) / dh ** 0.5).to(torch.bfloat16).to(DEV)
    kh, vh = (torch.nn.functional.normalize(torch.randn(BH, N, d, generator=g), dim=-1)
              .to(torch.bfloat16).to(DEV) for _ in range(2))
    lr3 = ([(torch.sigmoid(torch.randn(BH, N, generator=g)) * 0.1).to(DEV) for _ in range(3)]
           if with_lr else None)
    gs = DN._gs(BH, N, DEV)
    dy, hl = DN._update_stage1(W02, W1, kh, vh, lr3, gs)
    ref_dy, ref_hl = G.update_stage1(W02, W1, kh, vh, *(lr3 or (None,) * 3), gs,
                                     token_major=True)
    torch.cuda.synchronize()
    assert dy.shape == (BH, N, 2 * dh) and hl.shape == (BH, N, dh)
    assert_bf16_close(dy.cpu(), ref_dy.cpu(), name="DY0_DY2")
    assert_bf16_close(hl.cpu(), ref_hl.cpu(), name="Hid")
    # same products in the same k order on the same MFMA, same epilogue: the
    # two routes agree bit for bit (measured at the configs[0] and [1] heads)
    if (d, dh) in ((192, 384), (96, 192)):
        assert torch.equal(dy.view(torch.int16), ref_dy.view(torch.int16))
        assert torch.equal(hl.view(torch.int16), ref_hl.view(torch.int16))
    # a second call into the same weight copy: same bits
    dy2, hl2 = DN._update_stage1(W02, W1, kh, vh, lr3, gs, DN._pack_update(W02, W1))
    torch.cuda.synchronize()
    assert torch.equal(dy2, dy) and torch.equal(hl2, hl)


@pytest.mark.parametrize("BH,N,d,dh", [
    (4, 3000, 192, 384),   # configs[1] head, ragged token tiles
    (4, 1024, 96, 192),    # configs[0] head
    (2, 77, 128, 96),      # one partial tile, odd block count (3 blocks: a lone last block)
    (3, 128, 64, 32),      # one hidden block
])
def test_staged_stage1_equals_four_wave_kernel(BH, N, d, dh):
    """The two kernels of the fused stage 1 for D <= 192 -- eight waves with
    the weight fragments staged through LDS (taken for grids of >= 256
    workgroups) and four waves with register prefetch (smaller grids) --
    compute every output with the same MFMA chain and epilogue, so they agree
    bit for bit; both forced on the same inputs, with and without lr."""
    from uttt_amd import _lib as L

    g = torch.Generator().manual_seed(7 * N + d)
    W02 = (torch.randn(BH, 1, 2 * dh, d, generator=g) / d ** 0.5).to(torch.bfloat16).to(DEV)
    W1 = (torch.randn(BH, 1, d, dh, generator=g) / dh ** 0.5).to(torch.bfloat16).to(DEV)
    kh, vh = (torch.nn.functional.normalize(torch.randn(BH, N, d, generator=g), dim=-1)
              .to(torch.bfloat16).to(DEV) for _ in range(2))
    lr3 = [(torch.sigmoid(torch.randn(BH, N, generator=g)) * 0.1).to(DEV) for _ in range(3)]
    gs = DN._gs(BH, N, DEV)
    for lr in (lr3, None):
        outs = []
        for mode in (1, 2):
            prev = L.lib().uttt_debug_set_s1_staged(mode)
            try:
                outs.append(DN._update_stage1(W02, W1, kh, vh, lr, gs))
            finally:
                L.lib().uttt_debug_set_s1_staged(prev)
        torch.cuda.synchronize()
        (dy_s, hl_s), (dy_f, hl_f) = outs
        assert torch.equal(dy_s.view(torch.int16), dy_f.view(torch.int16))
        assert torch.equal(hl_s.view(torch.int16), hl_f.view(torch.int16))
        assert torch.isfinite(dy_s.float()).all() and torch.isfinite(hl_s.float()).all()


@pytest.mark.parametrize("use_moun,with_mom,master_renorm", [
    (False, True, False), (True, False, False), (True, True, False), (True, True, True)])
def test_bank_momentum_and_muon_equal_the_functional_write(use_moun, with_mom, master_renorm):
    # the bank's write (batched UPDATE of one layer, momentum on the
    # (batch, head) buffers, Newton-Schulz per d x d slice of the packed
    # weights) against fast_weight_write.apply_shared_update on the same
    # aggregate update, whose arithmetic is checked against the oracle in
    # tests/test_gpu_write.py and tests/test_gpu_muon.py: bit-identical
    from uttt_amd import fast_weight_write as FWW

    b, H, d, r, l = 2, 4, 96, 2, 512
    fast = tuple(w.to(torch.bfloat16).to(DEV) for w in _weights(b, H, d, r, seed=11))
    g = torch.Generator().manual_seed(12)
    masters = tuple((w.float().cpu() * (1 + 0.01 * torch.rand(w.shape, generator=g))).to(DEV)
                    for w in fast)
    moms = tuple((torch.randn(w.shape, generator=g) * 0.01).to(DEV) for w in fast)
    coeffs = [torch.rand(b, 1, 1, 1, generator=g).to(DEV) for _ in range(1)]
    q, k, v, lr = (t.to(DEV) for t in _layer(b, l, H, d, seed=13))
    bank = DN.SharedFastWeights(*fast, r=r, masters=masters, lr_scale=0.7,
                                master_renorm=master_renorm, use_momentum=with_mom,
                                use_moun=use_moun)
    bank.set_weights(fast, masters, moms if with_mom else None)
    agg = DN.compute_update(k, v, lr, fast)
    bank.write([k], [v], [lr], momentum_coeffs=coeffs if with_mom else None)
    rf, rm, rmom = FWW.apply_shared_update(agg, fast, masters, moms if with_mom else None,
                                           coeffs if with_mom else None, r=r, lr_scale=0.7,
                                           master_renorm=master_renorm, use_moun=use_moun)
    (bf, bm) = bank.weights()
    for i in range(3):
        assert torch.equal(bf[i], rf[i]), f"fast {i}"
        assert torch.equal(bm[i], rm[i]), f"master {i}"
    if with_mom:
        for x, y in zip(bank.momentum(), rmom):
            assert torch.equal(x, y)


def test_bank_owns_its_weights():
    # weights() hands out copies: editing one leaves the bank's reads alone
    b, H, d, r, l = 1, 4, 96, 2, 64
    fast = tuple(w.to(torch.bfloat16).to(DEV) for w in _weights(b, H, d, r, seed=21))
    q = _layer(b, l, H, d, seed=22)[0].to(DEV)
    bank = DN.SharedFastWeights(*fast, r=r)
    before = bank.read(q).clone()
    bank.read(q)                                   # second read: the packed copy is built
    (w0, w1, w2), _ = bank.weights()
    w0.zero_()
    assert torch.equal(bank.read(q), before)
    # set_weights replaces the state and drops the packed copy
    bank.set_weights((w0, w1, w2))
    assert not torch.equal(bank.read(q), before)
    fresh = DN.SharedFastWeights(w0, w1, w2, r=r)
    assert torch.equal(bank.read(q), fresh.read(q))


@pytest.mark.parametrize("b,H,d,r,L,l,lr_kind", [
    (1, 4, 192, 2, 12, 2048, "shared_f32"),   # the configs[1] write: 12 layers, 12 K runs
    (2, 2, 64, 2, 3, 512, "per_head_bf16"),
    (1, 4, 96, 2, 1, 512, "none"),            # one layer (configs[0]'s shape)
])
def test_layered_update_equals_gathered_heads(b, H, d, r, L, l, lr_kind):
    """The aggregate write's UPDATE read from every layer's own k, v, lr
    (uttt_dense_update_stage1_layers, uttt_dense_wgrad_pair_layers) equals
    the per-head copy path (uttt_dense_gather_heads, then stage 1 and the
    weight gradients) bit for bit at shapes where the copy path's K split is
    one run per layer."""
    import torch
    from uttt_amd import dense as DN
    from uttt_amd.lact_moe_triton import _grouped as G
    dh = r * d
    g = torch.Generator(device="cuda").manual_seed(L * l + d)
    W02 = (torch.randn(b * H, 1, 2 * dh, d, generator=g, device="cuda") * d ** -0.5).to(torch.bfloat16)
    W1 = (torch.randn(b * H, 1, d, dh, generator=g, device="cuda") * d ** -0.5).to(torch.bfloat16)
    ks = [torch.nn.functional.normalize(torch.randn(b, l, H * d, generator=g, device="cuda"), dim=-1)
          .to(torch.bfloat16) for _ in range(L)]
    vs = [torch.randn(b, l, H * d, generator=g, device="cuda").to(torch.bfloat16) for _ in range(L)]
    if lr_kind == "none":
        lrs = None
    elif lr_kind == "shared_f32":
        lrs = [torch.sigmoid(torch.randn(b, l, 3, generator=g, device="cuda")) * 0.1 for _ in range(L)]
    else:
        lrs = [(torch.sigmoid(torch.randn(b, l, 3 * H, generator=g, device="cuda")) * 0.1)
               .to(torch.bfloat16) for _ in range(L)]
    lay = DN._layered(ks, vs, lrs, H, d, dh)
    assert lay is not None
    got = DN._update_layered(W02, W1, lay[0], lay[1], lay[2], b, l, H, None)
    kh, vh, lr3 = DN._gather_heads(ks, vs, lrs, H)
    gs = DN._gs(b * H, L * l, kh.device)
    dy, hl = DN._update_stage1(W02, W1, kh, vh, lr3, gs)
    ref = G.wgrad_pair(dy, kh, hl, vh, gs)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    assert torch.isfinite(got[0].float()).all() and torch.isfinite(got[1].float()).all()

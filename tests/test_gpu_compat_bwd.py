"""GPU parity of the kernel-level pieces of the UPDATE backward that the
reference exposes as their own modules (grouping_four_grouped_gemm_triton,
fused_grouped_grad_kv, the second-order SwiGLU pointwise pass) against
oracle/fastweight.py, whose pieces are pinned by autograd and by composing
them into the autograd-pinned UPDATE backward.

Bar: rtol 2e-2 for bf16 outputs (tests.helpers.assert_bf16_close) on the
token columns the expert segments cover; fp32 lr gradients within rtol 1e-4
(fp32 sums over the hidden rows in a different order).
"""
import pytest
import torch

from oracle import fastweight as FW
from tests.helpers import assert_bf16_close
from tests.test_gpu_grouped import case, dev, tok_mask
from uttt_amd.lact_moe_triton import triton_lact_bwd_grouped_four_mm as FM
from uttt_amd.lact_moe_triton import triton_lact_bwd_grouped_grad_kv as GKV
from uttt_amd.lact_moe_triton import triton_pointwise_kernels as PW

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _grads(c, seed):
    g = torch.Generator().manual_seed(seed)
    GW02 = (torch.randn(c["W02"].shape, generator=g) * 0.05).to(torch.bfloat16)
    GW1 = (torch.randn(c["W1"].shape, generator=g) * 0.05).to(torch.bfloat16)
    return GW02, GW1


@pytest.mark.parametrize("name", ["ragged", "slack", "c3_chunk"])
def test_four_grouped_gemm(name):
    c = case(name, seed=3)
    GW02, GW1 = _grads(c, 4)
    W02, W1, K, V, gs = dev(c, "W02", "W1", "K", "V", "gs")
    outs = FM.grouping_four_grouped_gemm_triton(W02, GW02.to(DEV), W1, GW1.to(DEV), K, V, gs)
    refs = FW.four_grouped(c["W02"], GW02, c["W1"], GW1, c["K"], c["V"], c["gs"])
    m = tok_mask(c)
    for o, r, n in zip(outs, refs, ("Y0_Y2", "G_Y0_Y2", "DHidden", "G_DHidden")):
        assert_bf16_close(o.cpu().transpose(1, 2)[m], r.transpose(1, 2)[m], name=n)


@pytest.mark.parametrize("name", ["ragged", "slack", "c3_chunk"])
def test_fused_grad_kv(name):
    c = case(name, seed=5)
    GW02, GW1 = _grads(c, 6)
    B, N = c["K"].shape[:2]
    I = c["W1"].shape[3]
    g = torch.Generator().manual_seed(7)
    rnd = lambda *s: (torch.randn(*s, generator=g) * 0.1).to(torch.bfloat16)
    DY, dY, dH, Hl = rnd(B, 2 * I, N), rnd(B, 2 * I, N), rnd(B, I, N), rnd(B, I, N)
    W02, W1, gs = dev(c, "W02", "W1", "gs")
    gk, gv = GKV.fused_grouped_grad_kv(GW02.to(DEV), W02, DY.to(DEV), dY.to(DEV), W1, GW1.to(DEV),
                                       dH.to(DEV), Hl.to(DEV), gs)
    rk, rv = FW.grad_kv(GW02, c["W02"], DY, dY, c["W1"], GW1, dH, Hl, c["gs"])
    m = tok_mask(c)
    assert_bf16_close(gk.cpu()[m], rk[m], name="grad_K")
    assert_bf16_close(gv.cpu()[m], rv[m], name="grad_V")


@pytest.mark.parametrize("xd,ld", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                   (torch.float32, torch.float32)])
def test_swiglu_bwd_bwd_pointwise(xd, ld):
    B, I, Lt = 2, 200, 777   # ragged column tiles and row chunks
    g = torch.Generator().manual_seed(8)
    dh = torch.randn(B, I, Lt, generator=g).to(xd)
    x02 = torch.randn(B, 2 * I, Lt, generator=g).to(xd)
    lr = [(torch.rand(B, Lt, generator=g) * 0.1).to(ld) for _ in range(3)]
    gdx = torch.randn(B, 2 * I, Lt, generator=g).to(xd)
    ghl = torch.randn(B, I, Lt, generator=g).to(xd)
    for fn in (PW.triton_swiglu_bwd_bwd_fused_cat_inp_out,
               PW.ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out):
        outs = fn(dh.to(DEV), x02.to(DEV), *(x.to(DEV) for x in lr), gdx.to(DEV), ghl.to(DEV))
        refs = FW.swiglu_bwd_bwd(dh, x02, *lr, gdx, ghl)
        names = ("grad_dh", "grad_x0_x2", "grad_lr0", "grad_lr1", "grad_lr2", "dx0_x2", "hidden_lr1")
        for o, r, n in zip(outs, refs, names):
            assert o.dtype == r.dtype, n
            if n.startswith("grad_lr") and ld == torch.float32:
                torch.testing.assert_close(o.cpu(), r, rtol=1e-4, atol=1e-4 * r.abs().max().item())
            elif xd == torch.float32 and not n.startswith("grad_lr"):
                torch.testing.assert_close(o.cpu(), r, rtol=1e-4, atol=1e-5)
            else:
                assert_bf16_close(o.cpu(), r, name=n)

"""GPU parity of the decode read (csrc/decode_read.hip through
uttt_amd.decode) against oracle/moe_read.py on the same seeded inputs, and
against this build's own grouped path (row map -> permute -> grouped SwiGLU
apply -> unpermute) on the GPU.

Bar: rtol 2e-2 in bf16 (the fp32 dot products accumulate in another order
than the oracle's fp64 sums, which can move the bf16 hidden or expert output
by one rounding); tokens that select no expert read exact zeros.
"""
import pytest
import torch

from oracle import moe_read as MR
from tests.helpers import assert_bf16_close
from uttt_amd import _lib as L
from uttt_amd import decode as DEC
from uttt_amd.lact_moe_triton import lact_swiglu_ffn as SF
from uttt_amd.lact_moe_triton import triton_permute as TP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, T, E, k, D, I, seed, ragged=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(torch.bfloat16)
    scores = torch.rand(B, E, T, generator=g)
    top = scores.topk(k, dim=1).indices
    mask = torch.zeros(B, E, T, dtype=torch.bool).scatter_(1, top, True)
    if ragged and T > 1:
        mask[:, :, 1] = False                          # token 1 selects nothing
        mask[:, top[0, 0, 0], 0] = False               # token 0 of batch 0: k-1 experts
    probs = torch.softmax(torch.randn(B, E, T, generator=g), dim=1) * mask
    return x, W02, W1, mask, probs


@pytest.mark.parametrize("B,T,E,k,D,I,mask_dtype", [
    (1, 1, 32, 2, 1536, 3072, torch.bool),     # the 760M decode step
    (3, 1, 16, 2, 768, 1536, torch.int32),     # 124M shapes, three sequences
    (2, 5, 8, 3, 64, 96, torch.bool),          # partial chunks on both axes
    (1, 13, 16, 2, 128, 256, torch.int32),     # two token groups per expert
    (2, 64, 64, 4, 96, 192, torch.bool),       # the largest T and E
    (1, 3, 8, 2, 2560, 4096, torch.bool),      # long rows: 5 and 8 chunks per lane, 2-token groups
])
def test_decode_read_matches_oracle(B, T, E, k, D, I, mask_dtype):
    x, W02, W1, mask, probs = _case(B, T, E, k, D, I, seed=T * 31 + E)
    ref = MR.apply_moe_grouped(x, W02, W1, mask, probs, k)
    ours = DEC.moe_decode_read(x.to(DEV), W02.to(DEV), W1.to(DEV), mask.to(mask_dtype).to(DEV),
                               probs.to(DEV), k)
    assert ours.dtype == torch.bfloat16 and ours.shape == (B, T, D)
    assert_bf16_close(ours, ref, name="decode read")
    if T > 1:
        assert (ours[:, 1].cpu() == 0).all()


def test_decode_read_token_major_views():
    """Mask and probs as [B, T, E] tensors viewed [B, E, T] (the router's
    token-major layout), any strides."""
    B, T, E, k, D, I = 2, 3, 16, 2, 256, 512
    x, W02, W1, mask, probs = _case(B, T, E, k, D, I, seed=5, ragged=False)
    ref = MR.apply_moe_grouped(x, W02, W1, mask, probs, k)
    m_tm = mask.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    p_tm = probs.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    ours = DEC.moe_decode_read(x.to(DEV), W02.to(DEV), W1.to(DEV), m_tm, p_tm, k)
    assert_bf16_close(ours, ref, name="decode read, token-major views")


def test_decode_read_equals_grouped_path():
    """The same read through the grouped path on the GPU (the prefill route)."""
    B, T, E, k, D, I = 2, 4, 32, 2, 1536, 3072
    x, W02, W1, mask, probs = _case(B, T, E, k, D, I, seed=11, ragged=False)
    x, W02, W1, mask, probs = (t.to(DEV) for t in (x, W02, W1, mask, probs))
    xp, _, rmap = TP.permute_with_expert_mask(x, mask, probs, k)
    y = SF.grouped_swiglu_ffn_fwd(W02, W1, xp, mask.sum(-1).to(torch.int32))
    grouped = TP.unpermute_and_merge_with_probs(y, rmap, probs)
    ours = DEC.moe_decode_read(x, W02, W1, mask, probs, k)
    assert_bf16_close(ours, grouped, name="decode read vs grouped path")


def test_route_and_read_matches_oracle():
    """The whole read of modeling_recurrent_lact.py:296-349 for one decode
    token per sequence: the fused router, then the decode read."""
    B, T, E, k, D, I = 4, 1, 32, 2, 768, 1536
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    R = torch.randn(E, D, generator=g) / D ** 0.5
    w0 = (torch.randn(B, E, I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    w2 = (torch.randn(B, E, I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    w1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(torch.bfloat16)
    out, (mask, _, probs, _) = DEC.apply_moe_fast_weights_decode(
        x.to(DEV), w0.to(DEV), w1.to(DEV), w2.to(DEV), R.to(DEV), k)
    # routing parity is tests/test_gpu_router.py's; here the read of the
    # routing the GPU chose
    assert (mask.sum(dim=1) == k).all()
    ref = MR.apply_moe_grouped(x, torch.cat([w0, w2], dim=2), w1, mask.cpu(), probs.cpu(), k)
    assert_bf16_close(out, ref, name="route + decode read")


def test_decode_read_rejects_bad_sizes():
    x = torch.zeros(1, 65, 64, dtype=torch.bfloat16, device=DEV)
    W02 = torch.zeros(1, 4, 32, 64, dtype=torch.bfloat16, device=DEV)
    W1 = torch.zeros(1, 4, 64, 16, dtype=torch.bfloat16, device=DEV)
    m = torch.zeros(1, 4, 65, dtype=torch.bool, device=DEV)
    p = torch.zeros(1, 4, 65, device=DEV)
    with pytest.raises(AssertionError):
        DEC.moe_decode_read(x, W02, W1, m, p, 2)
    out = torch.empty(1, 65, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="exceed 64"):
        L.call("uttt_moe_decode_read", L.ptr(x), 1, 65, 64, L.ptr(W02), L.ptr(W1), 4, 16,
               L.ptr(m), 1, m.stride(0), m.stride(1), m.stride(2), L.ptr(p), p.stride(0),
               p.stride(1), p.stride(2), 2, L.ptr(out), None, 0, L.stream_of(x))

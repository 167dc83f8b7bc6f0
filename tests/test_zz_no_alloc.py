"""The no-allocation decode read (uttt_moe_decode_read_noalloc, scratch in a
file-scope device array) against the workspace entry point
(uttt_moe_decode_read) through the C ABI: bit-identical outputs on two calls
in a row, the second with a smaller problem (fewer sequences, tokens and
hidden units), so stale contents of the shared array from the first call
must not leak into the second; problems beyond the array are refused."""
import ctypes

import pytest
import torch

from uttt_amd import _lib as L

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, T, E, k, D, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16)
    W1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(torch.bfloat16)
    top = torch.rand(B, E, T, generator=g).topk(k, dim=1).indices
    mask = torch.zeros(B, E, T, dtype=torch.bool).scatter_(1, top, True)
    probs = torch.softmax(torch.randn(B, E, T, generator=g), dim=1) * mask
    return [t.to(DEV) for t in (x, W02, W1, mask, probs)]


def _call(noalloc, x, W02, W1, mask, probs, k):
    B, T, D = x.shape
    E, I = W02.shape[1], W02.shape[2] // 2
    m = mask.view(torch.uint8)
    out = torch.full((B, T, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    common = [L.ptr(x), B, T, D, L.ptr(W02), L.ptr(W1), E, I, L.ptr(m), 1, m.stride(0),
              m.stride(1), m.stride(2), L.ptr(probs), probs.stride(0), probs.stride(1),
              probs.stride(2), k, L.ptr(out)]
    stream = L.stream_of(x)
    if noalloc:
        L.call("uttt_moe_decode_read_noalloc", *common, stream)
    else:
        nb = L.lib().uttt_moe_decode_read_workspace_bytes(B, T, E, I)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        L.call("uttt_moe_decode_read", *common, L.ptr(ws), nb, stream)
    return out


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: 4 sequences x 2 tokens of the 760M pool shape (1.5 MiB of hidden)
    big = _case(4, 2, 32, 2, 1536, 3072, seed=1)
    ref = _call(False, *big, 2)
    got = _call(True, *big, 2)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    # second call, smaller on every axis: stale hidden rows of the first call
    # sit in the array where the second one's layout differs
    small = _case(2, 1, 16, 2, 768, 1536, seed=2)
    ref2 = _call(False, *small, 2)
    got2 = _call(True, *small, 2)
    torch.cuda.synchronize()
    assert torch.equal(got2, ref2)
    assert torch.isfinite(got2.float()).all()


def test_noalloc_refuses_problems_beyond_the_array():
    x, W02, W1, mask, probs = _case(1, 1, 8, 2, 64, 64, seed=3)
    B, T, E, I = 64, 64, 64, 4096            # 64*64*64*4096*2 bytes = 2 GiB of hidden
    rc = L.lib().uttt_moe_decode_read_noalloc(L.ptr(x), B, T, 64, L.ptr(W02), L.ptr(W1), E, I,
                                              L.ptr(mask), 1, 0, 0, 0, L.ptr(probs), 0, 0, 0, 2,
                                              L.ptr(x), L.stream_of(x))
    assert rc == -1
    assert b"exceed" in L.lib().uttt_last_error()

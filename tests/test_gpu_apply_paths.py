"""The two kernels of the weight-streaming APPLY products give identical
results: the general 256-token tiles (tn_kernel) and the skinny 128-token
tiles with the three-stage ring (apply_kernel), chosen by size
(N < 256 * E: the skinny tiles).  Both accumulate in the same k order with
the same MFMA, so the gate/up hidden state and the down projection must
match bit for bit, on ragged groups, empty experts, K tails (D % 64 != 0),
more than 64 experts, partial row tiles and two batches; the skinny path is
also checked against the oracle's grouped APPLY."""
import pytest
import torch

from oracle import fastweight as OF
from tests.helpers import assert_bf16_close
from uttt_amd import _lib as L

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _groups(B, E, N, seed, empty=()):
    g = torch.Generator().manual_seed(seed)
    w = torch.rand(B, E, generator=g) ** 3 + 1e-3
    for e in empty:
        w[:, e] = 0
    gs = torch.floor(w / w.sum(1, keepdim=True) * N).to(torch.int32)
    gs[:, 0] += N - gs.sum(1).to(torch.int32)
    return gs


def _run(path, W02, W1, X, gs, B, E, I, D, N):
    prev = L.lib().uttt_debug_set_apply_path(path)
    try:
        s = torch.cuda.current_stream().cuda_stream
        hid = torch.empty(B, N, I, dtype=torch.bfloat16, device=DEV)
        y = torch.empty(B, N, D, dtype=torch.bfloat16, device=DEV)
        L.call("uttt_grouped_gate_up", L.ptr(W02), L.ptr(X), L.ptr(gs), B, E, I, D, N, L.ptr(hid),
               1, s)
        L.call("uttt_grouped_gemm_nt", L.ptr(W1), L.ptr(hid), L.ptr(gs), B, E, D, I, N, L.ptr(y), s)
        torch.cuda.synchronize()
        return hid, y
    finally:
        L.lib().uttt_debug_set_apply_path(prev)


@pytest.mark.parametrize("B,E,I,D,N,empty", [
    (1, 32, 3072, 1536, 4096, (5, 9)),    # the configs[4] chunk shape
    (2, 8, 384, 200, 700, (3,)),          # K tails (200, 384 % 64 = 0 / 200 % 64 = 8)
    (1, 70, 136, 96, 900, (1, 68)),       # > 64 experts, partial row tiles
    (1, 4, 256, 128, 1500, ()),           # many tokens per expert (4 token tiles each)
])
def test_apply_paths_identical(B, E, I, D, N, empty):
    g = torch.Generator().manual_seed(N)
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(DEV)
    W1 = (torch.randn(B, E, D, I, generator=g) / I ** 0.5).to(torch.bfloat16).to(DEV)
    X = torch.randn(B, N, D, generator=g).to(torch.bfloat16).to(DEV)
    gs = _groups(B, E, N, N, empty).to(DEV)
    h0, y0 = _run(0, W02, W1, X, gs, B, E, I, D, N)
    for path in (1, 2):
        h, y = _run(path, W02, W1, X, gs, B, E, I, D, N)
        assert torch.equal(h, h0), f"hidden differs on path {path}"
        assert torch.equal(y, y0), f"down projection differs on path {path}"
    if D * I <= 200 * 384:
        # the skinny path against the oracle's grouped SwiGLU apply (the
        # reference's bf16 hidden state between the two products)
        ref = OF.swiglu_ffn_fwd(W02.cpu(), W1.cpu(), X.cpu(), gs.cpu())
        assert_bf16_close(y, ref, name="apply (skinny tiles)")


@pytest.mark.parametrize("B,E,I,D,T,k,empty", [
    (1, 32, 3072, 1536, 2048, 2, (5, 9)),   # the configs[4] routed read
    (1, 16, 1536, 768, 2048, 2, ()),        # the configs[3] routed read
    (2, 8, 384, 200, 350, 2, (3,)),         # K tails, two batches
    (1, 70, 136, 96, 300, 3, (1, 68)),      # > 64 experts, partial row tiles
])
def test_gate_up_gather_equals_permuted_copy(B, E, I, D, T, k, empty):
    """uttt_grouped_gate_up_gather reading x's rows through an inverse row
    map gives the hidden state of uttt_grouped_gate_up on the permuted copy,
    bit for bit, on every APPLY path (on the general tiles it copies the rows
    first); an index outside [0, T) reads row T - 1."""
    from uttt_amd.lact_moe_triton import _grouped as G
    N = T * k
    g = torch.Generator().manual_seed(T + E)
    W02 = (torch.randn(B, E, 2 * I, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(DEV)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16).to(DEV)
    gs = _groups(B, E, N, T, empty).to(DEV)
    src = torch.stack([torch.randperm(N, generator=g) % T for _ in range(B)]).to(torch.int32)
    src = src.to(DEV)
    x_perm = torch.gather(x, 1, src.long()[:, :, None].expand(B, N, D)).contiguous()
    for path in (-1, 0, 1):
        prev = L.lib().uttt_debug_set_apply_path(path)
        try:
            ref = G.gate_up(W02, x_perm, gs, token_major=True)
            got = G.gate_up_gather(W02, x, src, gs)
            torch.cuda.synchronize()
        finally:
            L.lib().uttt_debug_set_apply_path(prev)
        assert torch.equal(got, ref), f"gathered gate/up differs on path {path}"
    bad = src.clone()
    bad[0, 0], bad[-1, -1] = T + 5, -3
    want = src.clone()
    want[0, 0], want[-1, -1] = T - 1, T - 1
    xw = torch.gather(x, 1, want.long()[:, :, None].expand(B, N, D)).contiguous()
    assert torch.equal(G.gate_up_gather(W02, x, bad, gs), G.gate_up(W02, xw, gs, token_major=True))

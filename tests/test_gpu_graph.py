"""The routed read (uttt_amd.moe.apply_moe_fast_weights_grouped: router, row
map, permute, grouped SwiGLU APPLY, gate-weighted unpermute) captured in a HIP
graph (torch.cuda.CUDAGraph) and replayed: every replay must equal the eager
call on the same inputs bit for bit (the same kernels on the same data), with
new token rows copied into the captured input and the expert weights
rewritten in place between replays, and eager reads and synchronisations of
the program in between.  None of the read's kernels records a memset, a host
synchronisation or an allocation of its own.
"""
import pytest
import torch

from uttt_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # T, E, D, I, topk
    (2048, 16, 768, 1536, 2),   # the configs[3] chunk
    (300, 8, 256, 512, 3),
]


def _unit_rows(t):
    return (t / (t.norm(dim=-1, keepdim=True) + 1e-5)).to(torch.bfloat16)


@pytest.mark.parametrize("T,E,D,I,topk", CASES)
def test_routed_read_graph_replays(T, E, D, I, topk):
    g = torch.Generator(device=DEV).manual_seed(T + E)
    W02 = (torch.randn(1, E, 2 * I, D, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16)
    W1 = (torch.randn(1, E, D, I, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16)
    R = torch.randn(E, D, generator=g, device=DEV)
    rbias = torch.randn(E, generator=g, device=DEV) * 0.5
    cfg = moe.RouterConfig(topk=topk, combine_mode="topk_renorm")
    xs = [_unit_rows(torch.randn(1, T, D, generator=g, device=DEV)) for _ in range(4)]
    w_new = [(torch.randn(1, E, 2 * I, D, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16)
             for _ in range(2)]

    def read(x):
        with torch.no_grad():
            out, _ = moe.apply_moe_fast_weights_grouped(x, None, W1, None, R, cfg, 1,
                                                        routing_bias=rbias,
                                                        precomputed_w0_w2=W02)
        return out

    x_static = xs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        read(x_static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = read(x_static)
    torch.cuda.synchronize()

    # replays on new token rows, then on rewritten weights; eager work between
    steps = [(xs[1], None), (xs[2], None), (xs[3], w_new[0]), (xs[0], w_new[1]), (xs[1], None)]
    for i, (x, w) in enumerate(steps):
        if w is not None:
            W02.copy_(w)
        ref = read(x)              # eager, on the current weights
        torch.cuda.synchronize()
        x_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_static, ref), f"replay {i}: graph output differs from eager"
        assert torch.isfinite(ref.float()).all()


def test_stream_of_is_torchs_current_stream():
    """The glue launches on torch's current stream of the tensor's device:
    the default stream, a side stream inside `torch.cuda.stream`, and the
    default again after it."""
    from uttt_amd import _lib as L

    t = torch.empty(4, device=DEV)
    assert L.stream_of(t) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert L.stream_of(t) == side.cuda_stream == torch.cuda.current_stream().cuda_stream
    assert L.stream_of(t) == torch.cuda.current_stream().cuda_stream

"""Shared input generators and comparison helpers for the tests."""
from __future__ import annotations

import json
import os

import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def topk_mask_like_reference_test(B, T, E, k, gen):
    """The mask builder of uttt_nvs/tests/test_triton_permute.py:15-29: keeps
    scores strictly above the min(k, E-1)-th largest, i.e. k-1 experts."""
    kk = min(k, E - 1)
    scores = torch.rand(B, E, T, generator=gen)
    vals, _ = torch.topk(scores, k=kk, dim=1)
    thr = vals[:, [-1]]
    return (scores > thr).to(torch.int32)


def routing_c2(T=65536, E=16, k=2, seed=0, zipf=None):
    """Routing of the permute microbench: logits ~ N(0,1) [1,E,T], per-expert
    selection bias ~ N(0, 0.5) (or a Zipf prior), top-k, topk_renorm gates."""
    from oracle import routing

    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(1, E, T, generator=g)
    if zipf is not None:
        bias = (-zipf * torch.log(torch.arange(E, dtype=torch.float32) + 1.0)).view(1, E, 1)
    else:
        bias = (torch.randn(E, generator=g) * 0.5).view(1, E, 1)
    mask, gs, comb, bal, _ = routing.create_router_mask_sizes_probs(
        logits, k, combine_mode="topk_renorm", routing_bias=bias
    )
    return logits, bias, mask, gs, comb


def assert_bf16_close(ours, ref, rtol=2e-2, name=""):
    """|ours - ref| <= rtol*|ref| + rtol*rms(ref), elementwise (the bf16 bar
    is rtol 2e-2; the rms term absorbs cancellation near zero)."""
    o = ours.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert o.shape == r.shape, (name, o.shape, r.shape)
    assert torch.isfinite(o).all(), f"{name}: non-finite output"
    atol = rtol * r.pow(2).mean().sqrt().item()
    err = (o - r).abs()
    bound = rtol * r.abs() + atol
    bad = err > bound
    assert not bad.any(), (
        f"{name}: {int(bad.sum())}/{bad.numel()} elements out of tolerance; "
        f"max err {err.max().item():.3e}, atol {atol:.3e}"
    )


def assert_bf16_mostly_close(ours, ref, base=None, rtol=2e-2, rel_fro=1e-2, frac=1e-3, name=""):
    """The bar for results that pass through a chain of bf16 products whose
    fp32 accumulation order differs from the CPU's (Newton-Schulz): the
    relative Frobenius error of (ours - base) to (ref - base) is at most
    rel_fro (base: the value before the update, so the update itself is what
    is compared), and at most a fraction frac of the elements falls outside
    the elementwise rtol bar of assert_bf16_close."""
    o = ours.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert o.shape == r.shape, (name, o.shape, r.shape)
    assert torch.isfinite(o).all(), f"{name}: non-finite output"
    b = 0 if base is None else base.detach().double().cpu()
    rel = ((o - r).norm() / (r - b).norm()).item()
    assert rel <= rel_fro, f"{name}: relative Frobenius error {rel:.3e} > {rel_fro}"
    bad = (o - r).abs() > rtol * r.abs() + rtol * r.pow(2).mean().sqrt()
    assert bad.double().mean().item() <= frac, (
        f"{name}: {int(bad.sum())}/{bad.numel()} elements outside rtol {rtol}")

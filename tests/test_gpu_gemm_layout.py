"""The two wave layouts of the grouped GEMM kernels give identical results.

Every token-grouped product (tn_kernel) and weight-gradient product
(wg_kernel) exists in two layouts of its 256x256 workgroup tile: four waves
of 128x128 (one wave per SIMD) and eight waves of 64x128 (two per SIMD).  In
both, each output element is one chain of v_mfma_f32_32x32x16_bf16 over the
same k steps in the same order, so the layouts must agree bit for bit.  The
hook uttt_debug_set_gemm_layout forces one layout process-wide; each case
below runs the APPLY (general tiles), the UPDATE forward and its backward
(from saved tensors and recomputing), the split-K weight gradients, the
kernel-level compat pieces and Newton-Schulz under both layouts, on ragged
groups, empty experts, K tails, two batches and the super-tile order, and
compares every output with torch.equal.  The eight-wave kernels are also run
through the oracle parity tests of the general path.
"""
import pytest
import torch
import torch.nn.functional as F

from tests import test_gpu_compat_bwd as TC
from tests import test_gpu_grouped as TG
from tests import test_gpu_muon as TM
from uttt_amd import _lib as L
from uttt_amd.lact_moe_triton import lact_fw_grad as FG
from uttt_amd.lact_moe_triton import lact_swiglu_ffn as SF
from uttt_amd.lact_moe_triton import triton_grouped_swiglu_bwd_with_lr_kernels as U1
from uttt_amd.lact_moe_triton import triton_lact_bwd_grouped_two_mm_grad_fw as U2

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Layout:
    """Force a GEMM wave layout (and optionally the super-tile threshold)."""

    def __init__(self, na, supertile=None):
        self.na, self.supertile = na, supertile

    def __enter__(self):
        lib = L.lib()
        self.prev = lib.uttt_debug_set_gemm_layout(self.na)
        self.prev_path = lib.uttt_debug_set_apply_path(0)   # the general tiles for the APPLY
        self.prev_st = (lib.uttt_debug_set_supertile_min_tiles(self.supertile)
                        if self.supertile is not None else None)
        return self

    def __exit__(self, *exc):
        lib = L.lib()
        lib.uttt_debug_set_gemm_layout(self.prev)
        lib.uttt_debug_set_apply_path(self.prev_path)
        if self.prev_st is not None:
            lib.uttt_debug_set_supertile_min_tiles(self.prev_st)


def test_layout_hook_round_trip():
    lib = L.lib()
    prev = lib.uttt_debug_set_gemm_layout(1)
    try:
        assert lib.uttt_debug_set_gemm_layout(2) == 1
        assert lib.uttt_debug_set_gemm_layout(0) == 2
    finally:
        lib.uttt_debug_set_gemm_layout(prev)
    with pytest.raises(RuntimeError):
        L.call("uttt_debug_set_gemm_layout", 3)


def _all_products(c):
    """Outputs of every GEMM family on case c (device tensors, cloned)."""
    W02, W1, K, V, gs = TG.dev(c, "W02", "W1", "K", "V", "gs")
    lr = [x.to(DEV) for x in c["lr"]]
    out = {}
    out["apply"] = SF.grouped_swiglu_ffn_fwd(W02, W1, K, gs)
    dy, hid = U1.swiglu_backward_three_bmm_grouped_with_lr_triton(W02, W1, K, V, *lr, gs)
    out["stage1_dy"], out["stage1_hid"] = dy, hid
    w02, w1 = U2.grouped_two_gemm_fw_bwd_triton(dy, K, hid, V, gs)
    out["stage2_w02"], out["stage2_w1"] = w02, w1
    # UPDATE forward + backward through autograd (saved-tensor backward)
    g = torch.Generator().manual_seed(5)
    GW02 = (torch.randn(c["W02"].shape, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    GW1 = (torch.randn(c["W1"].shape, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    ins = [W02.clone(), W1.clone(), K.clone(), V.clone()] + [x.clone() for x in lr]
    for t in ins:
        t.requires_grad_()
    d02, d1 = FG.grouped_lact_swiglu_ffn_fast_weight_grads(*ins, gs)
    torch.autograd.backward([d02, d1], [GW02, GW1])
    out["upd_w02"], out["upd_w1"] = d02.detach(), d1.detach()
    for i, t in enumerate(ins):
        out[f"upd_grad{i}"] = t.grad
    # the recomputing backward (no saved tensors)
    from uttt_amd.lact_moe_triton import _update_bwd
    plain = _update_bwd.fast_weight_grads_backward(*(t.detach() for t in ins), gs, GW02, GW1)
    for i, t in enumerate(plain):
        out[f"plain_grad{i}"] = t
    # APPLY backward
    x = K.clone().requires_grad_()
    wa, wb = W02.clone().requires_grad_(), W1.clone().requires_grad_()
    y = SF.grouped_swiglu_ffn_fwd(wa, wb, x, gs)
    gy = (torch.randn(y.shape, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    torch.autograd.backward([y], [gy])
    out["apply_gx"], out["apply_gw02"], out["apply_gw1"] = x.grad, wa.grad, wb.grad
    torch.cuda.synchronize()
    return {k: v.detach().clone() for k, v in out.items() if v is not None}


@pytest.mark.parametrize("name", ["ragged", "slack", "one_expert", "c3_chunk"])
@pytest.mark.parametrize("supertile", [None, 1])
def test_layouts_bit_identical(name, supertile):
    c = TG.case(name)
    with _Layout(2, supertile):
        four = _all_products(c)
    with _Layout(1, supertile):
        eight = _all_products(c)
    m = TG.tok_mask(c).to(DEV)  # token columns the products write ("slack" leaves a tail)
    assert four.keys() == eight.keys() and len(four) >= 16, sorted(four)
    for k in four:
        a, b = four[k], eight[k]
        if a.dim() < 4:             # token-indexed outputs: [B, N, ...] or [B, rows, N]
            if a.shape[1] != c["N"]:
                a, b = a.transpose(1, 2), b.transpose(1, 2)
            a, b = a[m], b[m]
        assert torch.equal(a, b), f"{name}: {k} differs between the wave layouts"


@pytest.mark.parametrize("name", ["dense124m", "ragged_small"])
def test_layouts_bit_identical_split_k(name):
    B, E, D, I, gs = TG.SPLIT_CASES[name]
    gs = torch.tensor(gs, dtype=torch.int32)
    N = int(gs.sum(1).max())
    g = torch.Generator().manual_seed(3)
    dy = (torch.randn(B, 2 * I, N, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    hid = (torch.randn(B, I, N, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    K = F.normalize(torch.randn(B, N, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    V = F.normalize(torch.randn(B, N, D, generator=g), dim=-1).to(torch.bfloat16).to(DEV)
    res = []
    for na in (2, 1):
        with _Layout(na):
            a, b = U2.grouped_two_gemm_fw_bwd_triton(dy, K, hid, V, gs.to(DEV))
            torch.cuda.synchronize()
            res.append((a.clone(), b.clone()))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])


@pytest.mark.parametrize("n,R,C", [(3, 64, 128), (2, 256, 128), (1, 40, 200)])
def test_layouts_bit_identical_newton_schulz(n, R, C):
    from uttt_amd import fast_weight_write as FWW

    g = torch.Generator().manual_seed(n)
    G = torch.randn(n, R, C, generator=g).to(DEV)
    res = []
    for na in (2, 1):
        with _Layout(na):
            res.append(FWW.newton_schulz5(G).clone())
            torch.cuda.synchronize()
    assert torch.equal(res[0], res[1])


# The eight-wave kernels against the oracle (the general path's parity tests)
@pytest.fixture
def eight_waves():
    with _Layout(1):
        yield


@pytest.mark.parametrize("name", ["ragged", "slack", "c3_chunk"])
def test_eight_wave_apply_forward(name, eight_waves):
    TG.test_apply_forward(name)


@pytest.mark.parametrize("name", ["ragged", "slack"])
def test_eight_wave_apply_backward(name, eight_waves):
    TG.test_apply_backward(name)


@pytest.mark.parametrize("name", ["ragged", "slack", "one_expert", "c3_chunk"])
def test_eight_wave_update_forward(name, eight_waves):
    TG.test_update_forward(name, torch.bfloat16)


@pytest.mark.parametrize("name", ["ragged", "slack"])
def test_eight_wave_update_backward(name, eight_waves):
    TG.test_update_backward(name, torch.float32 if name == "slack" else torch.bfloat16)


@pytest.mark.parametrize("name", ["ragged", "slack"])
def test_eight_wave_compat_pieces(name, eight_waves):
    TG.test_two_mm_swiglu_compat(name)
    TG.test_gemm_transpose_compat(name)
    TG.test_update_stage_compat(name)
    TC.test_four_grouped_gemm(name)
    TC.test_fused_grad_kv(name)


@pytest.mark.parametrize("name", list(TG.SPLIT_CASES))
def test_eight_wave_wgrad_split_k(name, eight_waves):
    TG.test_wgrad_pair_split_k(name)


@pytest.mark.parametrize("n,R,C", [(3, 64, 128), (1, 40, 200)])
def test_eight_wave_newton_schulz5(n, R, C, eight_waves):
    TM.test_newton_schulz5_matches_oracle(n, R, C, torch.float32, 1.0)

"""The drop-in boundary on the CPU: every public function the reference's
callers import from lact_moe_triton exists in uttt_amd.lact_moe_triton with
the reference's parameter names, order, kinds and defaults.  The reference
side comes from tests/golden/reference_signatures.json, written from the
reference's sources by tests/golden/make_reference_signatures.py."""
import importlib
import inspect

import pytest

from tests.helpers import load_golden

# the boundary: what modeling_recurrent_lact.py, the NVS block and the
# kernel-level callers import (module -> functions)
BOUNDARY = {
    "triton_permute": ["make_row_id_map", "permute_with_expert_mask",
                       "unpermute_and_merge_with_probs", "permute_kv_and_lrs",
                       "triton_permute_with_mask_map", "triton_unpermute_with_mask_map",
                       "triton_permute_with_mask_map_bwd_batched",
                       "triton_unpermute_with_mask_map_bwd_with_merging_probs"],
    "lact_swiglu_ffn": ["grouped_swiglu_ffn_fwd"],
    "lact_fw_grad": ["grouped_lact_swiglu_ffn_fast_weight_grads"],
    "triton_grouped_swiglu_kernels": ["fused_two_mm_swiglu_triton"],
    "triton_grouped_gemm": ["grouped_gemm_transpose_triton", "grouped_gemm_bwd_triton"],
    "triton_grouped_swiglu_bwd_kernels": ["swiglu_backward_three_bmm_grouped_triton"],
    "triton_grouped_swiglu_bwd_with_lr_kernels": ["swiglu_backward_three_bmm_grouped_with_lr_triton"],
    "triton_lact_bwd_grouped_two_mm_grad_fw": ["grouped_two_gemm_fw_bwd_triton"],
    "triton_lact_bwd_grouped_four_mm": ["grouping_four_grouped_gemm_triton"],
    "triton_lact_bwd_grouped_grad_kv": ["fused_grouped_grad_kv"],
    "triton_pointwise_kernels": ["triton_swiglu_bwd_bwd_fused_cat_inp_out",
                                 "ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out"],
}
KINDS = {"positional": inspect.Parameter.POSITIONAL_OR_KEYWORD,
         "keyword_only": inspect.Parameter.KEYWORD_ONLY,
         "var_positional": inspect.Parameter.VAR_POSITIONAL,
         "var_keyword": inspect.Parameter.VAR_KEYWORD}
# documented extensions: trailing keyword parameters with defaults
EXTENSIONS = {("triton_permute", "make_row_id_map"): ["group_sizes"]}


def _cases():
    for mod, fns in BOUNDARY.items():
        for fn in fns:
            yield mod, fn


@pytest.mark.parametrize("mod,fn", list(_cases()))
def test_signature_matches_reference(mod, fn):
    ref = load_golden("reference_signatures.json")["modules"][mod][fn]["params"]
    ours = importlib.import_module(f"uttt_amd.lact_moe_triton.{mod}")
    assert hasattr(ours, fn), f"{mod}.{fn} missing"
    params = list(inspect.signature(getattr(ours, fn)).parameters.values())
    extra = EXTENSIONS.get((mod, fn), [])
    assert [p.name for p in params] == [p["name"] for p in ref] + extra, (mod, fn)
    for p, r in zip(params, ref):
        assert p.kind == KINDS[r["kind"]], (mod, fn, p.name, p.kind)
        assert (p.default is not inspect.Parameter.empty) == r["has_default"], (mod, fn, p.name)
        if r["has_default"]:
            assert p.default == r["default"], (mod, fn, p.name, p.default, r["default"])
    for p in params[len(ref):]:
        assert p.default is not inspect.Parameter.empty, (mod, fn, p.name)


def test_fixture_covers_the_boundary():
    mods = load_golden("reference_signatures.json")["modules"]
    for mod, fn in _cases():
        assert fn in mods[mod], (mod, fn)

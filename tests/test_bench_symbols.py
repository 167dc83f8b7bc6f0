"""bench.py's kernel-symbol names: the GEMM kernels' wave-layout argument and
the weight gradients' per-layer-operand flag fold into one family name, so
that per-sweep kernel times, the launch table (FLOP and bytes per symbol) and
the traffic lines of the committed profiles meet under the same key."""
import os
import re
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_layout_and_layered_flags_fold_into_the_family_name():
    cases = {
        "void uttt::(anonymous namespace)::wg_kernel<false, 2, false>(uttt::WgArgs, int)":
            "wg_kernel<false>",
        "wg_kernel<false, 1, false>": "wg_kernel<false>",
        "wg_kernel<true, 2, true>": "wg_kernel<true, layered>",
        "tn_kernel<0, EpiBwdSaved<BF16T>, false, 1>": "tn_kernel<0, EpiBwdSaved<BF16T>, false>",
        "tn_kernel<0, EpiBwdSaved<BF16T>, false, 2>": "tn_kernel<0, EpiBwdSaved<BF16T>, false>",
        "uttt::apply_kernel<ApSwiGLU, true>(uttt::ApArgs)": "apply_kernel<ApSwiGLU, true>",
    }
    for raw, want in cases.items():
        assert bench.norm_symbol(raw) == want, raw


def test_profile_traffic_lines_name_traced_kernels():
    """Every 'traffic_bytes <symbol>' line of a committed sweep profile names a
    kernel whose trace row in the same file normalises to that symbol."""
    pdir = os.path.join(ROOT, "profiles")
    for name in ("moe760m_sweep.txt", "moe124m_sweep.txt"):
        text = open(os.path.join(pdir, name)).read()
        traced = {bench.norm_symbol(m.group(1))
                  for m in re.finditer(r"^\| `([^`]+)`", text, re.M)}
        for m in re.finditer(r"^traffic_bytes (.+) (\d+)$", text, re.M):
            assert m.group(1) in traced, (name, m.group(1))
            assert bench._profile_traffic(name, m.group(1)) == int(m.group(2))

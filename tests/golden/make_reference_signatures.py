"""Write tests/golden/reference_signatures.json: the parameter lists of the
public functions of the reference's lact_moe_triton package (the drop-in
boundary), read from its sources with `ast` -- nothing of the reference is
imported or executed.

    python tests/golden/make_reference_signatures.py [REFERENCE_ROOT]

The fixture is data (module, function, parameter names, kinds, default
literals); tests/test_signatures.py checks this package's modules against it.
"""
from __future__ import annotations

import ast
import json
import os
import sys

PKG = "uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_signatures.json")


def _default(node):
    try:
        return ast.literal_eval(node)
    except ValueError:
        return ast.unparse(node)


def signatures(path):
    tree = ast.parse(open(path).read())
    out = {}
    for node in tree.body:
        if not isinstance(node, ast.FunctionDef) or node.name.startswith("_"):
            continue
        a = node.args
        params = []
        pos = a.posonlyargs + a.args
        defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
        for arg, d in zip(pos, defaults):
            params.append(dict(name=arg.arg, kind="positional",
                               default=None if d is None else _default(d),
                               has_default=d is not None))
        if a.vararg:
            params.append(dict(name=a.vararg.arg, kind="var_positional", default=None,
                               has_default=False))
        for arg, d in zip(a.kwonlyargs, a.kw_defaults):
            params.append(dict(name=arg.arg, kind="keyword_only",
                               default=None if d is None else _default(d),
                               has_default=d is not None))
        if a.kwarg:
            params.append(dict(name=a.kwarg.arg, kind="var_keyword", default=None,
                               has_default=False))
        out[node.name] = dict(line=node.lineno, params=params)
    return out


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    pkg = os.path.join(root, PKG)
    res = {}
    for fn in sorted(os.listdir(pkg)):
        if fn.endswith(".py") and fn != "__init__.py":
            res[fn[:-3]] = signatures(os.path.join(pkg, fn))
    with open(OUT, "w") as f:
        json.dump(dict(source=PKG, modules=res), f, indent=1, sort_keys=True)
    print(f"wrote {OUT}: {sum(len(v) for v in res.values())} functions in {len(res)} modules")


if __name__ == "__main__":
    main()

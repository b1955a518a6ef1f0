"""Writes tests/golden/signatures.json: the parameter lists of the reference's
public functions, read from its sources as text with `ast` (nothing of the
reference is imported or run).

    python tests/golden/make_signatures.py [/path/to/mamba-cpu]

Functions (reference file:line):
  selective_scan_fn       src/mamba_cpu/ops/selective_scan_interface.py:138-149
  causal_conv1d_fn        src/mamba_cpu/ops/causal_conv1d.py:16-25
  causal_conv1d_update    src/mamba_cpu/ops/causal_conv1d.py:56-58
  selective_state_update  src/mamba_cpu/ops/selective_state_update.py:5-7
  selective_scan_ref      src/mamba_cpu/reference.py:10-21
  causal_conv1d_ref       src/mamba_cpu/reference.py:65
Each entry is the text inspect.signature() prints for a function with those
parameters and defaults, e.g. "(x, weight, bias=None, activation=None)".
"""

import ast
import json
import os
import sys

WANT = {
    "selective_scan_fn": "src/mamba_cpu/ops/selective_scan_interface.py",
    "causal_conv1d_fn": "src/mamba_cpu/ops/causal_conv1d.py",
    "causal_conv1d_update": "src/mamba_cpu/ops/causal_conv1d.py",
    "selective_state_update": "src/mamba_cpu/ops/selective_state_update.py",
    "selective_scan_ref": "src/mamba_cpu/reference.py",
    "causal_conv1d_ref": "src/mamba_cpu/reference.py",
}


def signature_text(fn: ast.FunctionDef) -> str:
    """The parameter list as inspect.signature() renders it (positional
    parameters with literal defaults only, which is all these functions have)."""
    args = fn.args
    if args.vararg or args.kwarg or args.kwonlyargs or args.posonlyargs:
        raise ValueError(f"{fn.name}: unexpected parameter kinds")
    names = [a.arg for a in args.args]
    defaults = [None] * (len(names) - len(args.defaults)) + list(args.defaults)
    parts = []
    for name, d in zip(names, defaults):
        parts.append(name if d is None else f"{name}={ast.unparse(d)}")
    return "(" + ", ".join(parts) + ")"


def main(root):
    out = {}
    for name, rel in WANT.items():
        with open(os.path.join(root, rel)) as f:
            tree = ast.parse(f.read())
        fns = [n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == name]
        if len(fns) != 1:
            raise SystemExit(f"{rel}: expected one def {name}")
        out[name] = {"signature": signature_text(fns[0]), "source": f"{rel}:{fns[0].lineno}"}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "signatures.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps(out, indent=1, sort_keys=True))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

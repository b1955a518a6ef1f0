"""The binding examples in INTEGRATION.md stay in step with include/mamba_hip.h.

- The plain-C glue (the ```c block) compiles against the header with
  gcc -fsyntax-only -Wall -Werror.
- The ctypes example (the ```python block marked "# ctypes example") runs
  against a recording stand-in for the library on CPU tensors (nothing is
  dereferenced): every library call it makes passes as many arguments as the
  shipped binding declares for that entry point, and the forward receives
  the workspace size the query returned.
"""

import os
import re
import subprocess

import pytest
import torch

from conftest import ROOT

DOC = os.path.join(ROOT, "INTEGRATION.md")


def blocks(lang):
    text = open(DOC).read()
    return re.findall(r"```%s\n(.*?)```" % lang, text, re.S)


def test_c_glue_compiles_against_the_header(tmp_path):
    (c_src,) = blocks("c")
    src = tmp_path / "scan_hip_glue.c"
    src.write_text(c_src)
    gcc = "gcc"
    r = subprocess.run([gcc, "-std=c11", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # every mcpu_ entry point the glue calls is one the header declares
    header = open(os.path.join(ROOT, "include", "mamba_hip.h")).read()
    for name in set(re.findall(r"\b(mcpu_\w+)\s*\(", c_src)):
        assert re.search(r"\b%s\s*\(" % name, header), name


class _Recorder:
    """Stands in for the CDLL: records (name, args) of every call."""

    def __init__(self, sizes):
        self.calls = []
        self.sizes = sizes

    def __getattr__(self, name):
        def fn(*args):
            self.calls.append((name, args))
            return self.sizes.get(name, 0)

        fn.__name__ = name
        return fn


@pytest.mark.parametrize("workspace", [0, 4096])
def test_ctypes_example_calls_match_the_binding(workspace):
    from mamba_cpu import _C

    (src,) = [b for b in blocks("python") if b.startswith("# ctypes example")]
    ns = {}
    exec(compile(src, "INTEGRATION.md", "exec"), ns)
    b, d, l, n = 1, 8, 32, 4
    u = torch.randn(b, d, l)
    B = torch.randn(b, 1, n, l).transpose(-1, -2)
    rec = _Recorder({"mcpu_selective_scan_fwd_workspace_size": workspace})

    class FakeStream:
        cuda_stream = 0

    real = torch.cuda.current_stream
    torch.cuda.current_stream = lambda device=None: FakeStream()
    try:
        ns["scan_fwd"](rec, u, u, torch.randn(d, n), B, B, torch.randn(d), torch.empty_like(u),
                       torch.empty(b, d, n))
    finally:
        torch.cuda.current_stream = real
    names = [c[0] for c in rec.calls]
    assert names == ["mcpu_selective_scan_fwd_workspace_size", "mcpu_selective_scan_fwd"]
    for name, args in rec.calls:
        assert len(args) == len(getattr(_C.lib, name).argtypes), name
    fwd_args = rec.calls[1][1]
    assert fwd_args[2].value == workspace  # the size the query returned
    assert (fwd_args[1].value is None) == (workspace == 0)

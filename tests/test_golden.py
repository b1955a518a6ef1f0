"""Known-answer vectors from the reference's own CPU kernels.

tests/golden/scan_ref_vectors.npz holds inputs and the outputs/gradients of
csrc/selective_scan.cpp (compiled from the reference sources; see
tests/golden/make_golden.py). The float64 oracle is checked against them on
the CPU, and the HIP path on the GPU, at fp32 tolerances: outputs rtol 1e-4 /
atol 1e-5, gradients rtol 1e-3 (atol 1e-4 after scaling by the gradient's
magnitude). The reference's exp is a polynomial approximation, so the vectors
differ from exact arithmetic by a few ulp; the tolerances cover that.
"""

import os

import numpy as np
import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL
from oracle import numerics as O

HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = os.path.join(HERE, "golden", "scan_ref_vectors.npz")
CASES = ["full", "groups", "c1s"]
OPTIONAL = ("D", "z", "delta_bias")


def load(name):
    data = np.load(VECTORS)
    return {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}


def inputs_of(v):
    inp = {k: v[k] for k in ("u", "delta", "A", "B", "C")}
    for k in OPTIONAL:
        inp[k] = v.get(k)
    return inp


def close(got, want, rtol, atol, name):
    np.testing.assert_allclose(np.asarray(got, np.float64), want.astype(np.float64), rtol=rtol,
                               atol=atol, err_msg=name)


def close_grad(got, want, name):
    """Unscaled: rtol 1e-3 and the per-gradient atol of conftest.GRAD_ATOL
    (name is the gradient's, e.g. "dA" -> A)."""
    close(np.asarray(got, np.float64), want, GRAD_RTOL, GRAD_ATOL[name[1:]], name)


GRADS = ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias")


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_vectors(name):
    v = load(name)
    sp = bool(v["softplus"])
    out, last = O.selective_scan_fwd(**inputs_of(v), delta_softplus=sp)
    close(out, v["out"], 1e-4, 1e-5, "out")
    close(last, v["last_state"], 1e-4, 1e-5, "last_state")
    got = O.selective_scan_bwd(**inputs_of(v), delta_softplus=sp, dout=v["dout"],
                               dlast_state=v.get("dlast_state"))
    for k, g in zip(GRADS, got):
        if k in v:
            close_grad(g, v[k], k)
        else:
            assert g is None, k


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_reference_vectors(name):
    from mamba_cpu import selective_scan_fn

    v = load(name)
    sp = bool(v["softplus"])
    inp = {k: None if x is None else torch.from_numpy(x).cuda().requires_grad_()
           for k, x in inputs_of(v).items()}
    out, last = selective_scan_fn(**inp, delta_softplus=sp, return_last_state=True)
    close(out.detach().cpu(), v["out"], 1e-4, 1e-5, "out")
    close(last.detach().cpu(), v["last_state"], 1e-4, 1e-5, "last_state")
    loss = (out * torch.from_numpy(v["dout"]).cuda()).sum()
    if "dlast_state" in v:
        loss = loss + (last * torch.from_numpy(v["dlast_state"]).cuda()).sum()
    loss.backward()
    names = dict(du="u", ddelta="delta", dA="A", dB="B", dC="C", dD="D", dz="z",
                 ddelta_bias="delta_bias")
    for k in GRADS:
        if k in v:
            close_grad(inp[names[k]].grad.cpu(), v[k], k)

"""The CPU baseline path (oracle/cpu_torch.py) computes what the pinned
float64 oracle computes — CPU only, no GPU.

bench.py times oracle/cpu_torch.py on the host cores as the reference's CPU
path; these tests check that it is that computation: the ATen conv, conv
update and state update paths, and the autograd wrapper around the
reference's own C++ scan kernels (forward and backward)."""

import numpy as np
import pytest
import torch

from oracle import cpu_torch as CT
from oracle import numerics as O
from oracle import ref as R

needs_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built (make -C oracle)")


def _t(a, grad=False):
    return None if a is None else torch.tensor(a, dtype=torch.float32, requires_grad=grad)


@pytest.mark.parametrize("with_init", [False, True])
@pytest.mark.parametrize("activation", [None, "silu"])
def test_conv_fn_matches_oracle(with_init, activation):
    rng = np.random.default_rng(3)
    b, d, l, w = 2, 5, 19, 4
    x, wt, bias = rng.standard_normal((b, d, l)), rng.standard_normal((d, w)), rng.standard_normal(d)
    init = rng.standard_normal((b, d, w - 1)) if with_init else None
    G = rng.standard_normal((b, d, l))
    tx, tw, tb = _t(x, True), _t(wt, True), _t(bias, True)
    out, final = CT.causal_conv1d_fn(tx, tw, tb, _t(init), return_final_states=True, activation=activation)
    want, want_final = O.causal_conv1d_fwd(x, wt, bias, init, activation=activation)
    np.testing.assert_allclose(out.detach().numpy(), want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(final.detach().numpy(), want_final, rtol=1e-6, atol=1e-6)
    out.backward(_t(G))
    dx, dw, db, _ = O.causal_conv1d_bwd(x, wt, bias, init, G, activation)
    np.testing.assert_allclose(tx.grad.numpy(), dx, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(tw.grad.numpy(), dw, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(tb.grad.numpy(), db, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("single", [True, False])
def test_conv_update_matches_oracle(single):
    rng = np.random.default_rng(4)
    b, d, w, sl = 3, 6, 4, 5
    x = rng.standard_normal((b, d) if single else (b, d, 3))
    wt, bias, state = rng.standard_normal((d, w)), rng.standard_normal(d), rng.standard_normal((b, d, sl))
    ts = _t(state)
    out = CT.causal_conv1d_update(_t(x), ts, _t(wt), _t(bias), "silu")
    want, want_state = O.causal_conv1d_update(x, state, wt, bias, "silu")
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(ts.numpy(), want_state, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("heads", [False, True])
def test_state_update_matches_oracle(heads):
    rng = np.random.default_rng(5)
    b, h, p, n = 2, 3, 4, 8
    lead = (b, h, p) if heads else (b, h * p)
    prm = (h, p) if heads else (h * p,)
    state = rng.standard_normal(lead + (n,))
    x, dt, z = rng.standard_normal(lead), rng.random(lead), rng.standard_normal(lead)
    A, D, dtb = -rng.random(prm + (n,)), rng.standard_normal(prm), rng.random(prm) * 0.1
    B = rng.standard_normal((b, 1, n) if heads else (b, n))
    C = rng.standard_normal((b, 1, n) if heads else (b, n))
    ts = _t(state)
    out = CT.selective_state_update(ts, _t(x), _t(dt), _t(A), _t(B), _t(C), _t(D), _t(z), _t(dtb), True)
    want, want_state = O.selective_state_update(state, x, dt, A, B, C, D, z, dtb, True)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(ts.numpy(), want_state, rtol=1e-5, atol=1e-5)


@needs_ref
@pytest.mark.parametrize("ngroups", [None, 2])
def test_scan_autograd_wrapper_matches_oracle(ngroups):
    rng = np.random.default_rng(6)
    b, d, l, n = 2, 8, 21, 4
    bc = (b, n, l) if ngroups is None else (b, ngroups, n, l)
    inp = dict(u=rng.standard_normal((b, d, l)), delta=rng.random((b, d, l)) * 0.5,
               A=-(rng.random((d, n)) + 0.5), B=rng.standard_normal(bc), C=rng.standard_normal(bc),
               D=rng.standard_normal(d), z=rng.standard_normal((b, d, l)), delta_bias=rng.random(d) * 0.1)
    G = rng.standard_normal((b, d, l))
    leaves = {k: _t(v, True) for k, v in inp.items()}
    out = CT.selective_scan_fn(**leaves, delta_softplus=True, threads=2)
    want, _ = O.selective_scan_fwd(**inp, delta_softplus=True)
    np.testing.assert_allclose(out.detach().numpy(), want, rtol=1e-4, atol=1e-5)
    out.backward(_t(G))
    grads = O.selective_scan_bwd(**inp, delta_softplus=True, dout=G)
    for name, g in zip(["u", "delta", "A", "B", "C", "D", "z", "delta_bias"], grads):
        got = leaves[name].grad.numpy()
        scale = max(1.0, float(np.abs(g).max()))
        np.testing.assert_allclose(got / scale, g / scale, rtol=1e-3, atol=1e-4, err_msg=name)

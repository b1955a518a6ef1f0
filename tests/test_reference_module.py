"""mamba_cpu.reference (the exported pure-torch selective_scan_ref and
causal_conv1d_ref) against the float64 oracle, on the CPU.

Forward on every input layout the public op accepts (groups, unequal
groups, 2-D B/C, complex A, optional D / z / delta_bias, softplus), the
gradients autograd takes through it, and the conv at widths 1-5 including
sequences shorter than the kernel. Tolerances: float32 against float64,
rtol 1e-4 / atol 1e-5 on outputs, rtol 1e-3 / atol 1e-4 on gradients.
"""

import numpy as np
import pytest
import torch

from oracle import numerics as O

from mamba_cpu.reference import causal_conv1d_ref, selective_scan_ref


def scan_case(b, d, l, n, Bshape, Cshape, full, seed=0, cplx=False):
    g = torch.Generator().manual_seed(seed)
    inp = dict(u=torch.randn(b, d, l, generator=g), delta=torch.rand(b, d, l, generator=g) * 0.5,
               A=-torch.rand(d, n, generator=g) - 0.5,
               B=torch.randn(*Bshape, generator=g), C=torch.randn(*Cshape, generator=g))
    if cplx:
        inp["A"] = torch.complex(inp["A"], torch.randn(d, n, generator=g))
    if full:
        inp.update(D=torch.randn(d, generator=g), z=torch.randn(b, d, l, generator=g),
                   delta_bias=torch.rand(d, generator=g) * 0.1)
    return inp


LAYOUTS = {
    "one group": lambda b, d, n, l: ((b, n, l), (b, n, l)),
    "two groups": lambda b, d, n, l: ((b, 2, n, l), (b, 2, n, l)),
    "unequal groups": lambda b, d, n, l: ((b, 1, n, l), (b, 3, n, l)),
    "2-D B": lambda b, d, n, l: ((d, n), (b, 2, n, l)),
    "2-D B and C": lambda b, d, n, l: ((d, n), (d, n)),
}


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("full,softplus", [(True, True), (False, False)])
def test_scan_ref_matches_oracle(layout, full, softplus):
    b, d, l, n = 2, 6, 23, 4
    Bs, Cs = LAYOUTS[layout](b, d, n, l)
    inp = scan_case(b, d, l, n, Bs, Cs, full)
    leaves = {k: v.clone().requires_grad_() for k, v in inp.items()}
    out, last = selective_scan_ref(**leaves, delta_softplus=softplus, return_last_state=True)
    want, want_last = O.selective_scan_fwd(**inp, delta_softplus=softplus)
    np.testing.assert_allclose(out.detach().numpy(), want, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(last.detach().numpy(), want_last, rtol=1e-4, atol=1e-5)
    W = torch.randn(b, d, l, generator=torch.Generator().manual_seed(3))
    V = torch.randn(b, d, n, generator=torch.Generator().manual_seed(4))
    ((out * W).sum() + (last * V).sum()).backward()
    grads = O.selective_scan_bwd(**inp, delta_softplus=softplus, dout=W, dlast_state=V)
    for k, w in zip(("u", "delta", "A", "B", "C", "D", "z", "delta_bias"), grads):
        if k in leaves:
            np.testing.assert_allclose(leaves[k].grad.numpy(), w, rtol=1e-3, atol=1e-4, err_msg=k)


def test_scan_ref_complex_a_matches_oracle():
    """Complex A (mamba_ssm's semantics): input-dependent B/C of (re, im)
    pairs, and an input-independent complex C."""
    b, d, l, n = 2, 4, 9, 3
    inp = scan_case(b, d, l, n, (b, n, 2 * l), (b, n, 2 * l), True, cplx=True)
    out, last = selective_scan_ref(**inp, delta_softplus=True, return_last_state=True)
    want, want_last = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-4, atol=1e-5)
    assert last.dtype == torch.complex64
    np.testing.assert_allclose(last.numpy(), want_last, rtol=1e-4, atol=1e-5)
    inp["C"] = torch.complex(torch.randn(d, n), torch.randn(d, n))
    out = selective_scan_ref(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-4, atol=1e-5)


def test_scan_ref_keeps_u_dtype_and_handles_empty_sequences():
    inp = scan_case(1, 4, 8, 2, (1, 2, 8), (1, 2, 8), True)
    inp = {k: v.to(torch.bfloat16) if k in ("u", "delta", "z") else v for k, v in inp.items()}
    out, last = selective_scan_ref(**inp, return_last_state=True)
    assert out.dtype == torch.bfloat16 and last.dtype == torch.float32
    empty = scan_case(1, 4, 0, 2, (1, 2, 0), (1, 2, 0), False)
    out, last = selective_scan_ref(**empty, return_last_state=True)
    assert out.shape == (1, 4, 0) and torch.equal(last, torch.zeros(1, 4, 2))


@pytest.mark.parametrize("width", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("seqlen", [1, 3, 17])
@pytest.mark.parametrize("activation", [None, "silu"])
def test_conv_ref_matches_oracle(width, seqlen, activation):
    g = torch.Generator().manual_seed(width * 100 + seqlen)
    x = torch.randn(2, 5, seqlen, generator=g).requires_grad_()
    w = torch.randn(5, width, generator=g).requires_grad_()
    bias = torch.randn(5, generator=g).requires_grad_()
    out = causal_conv1d_ref(x, w, bias, activation=activation)
    want, _ = O.causal_conv1d_fwd(x, w, bias, activation=activation)
    np.testing.assert_allclose(out.detach().numpy(), want, rtol=1e-5, atol=1e-6)
    dout = torch.randn(2, 5, seqlen, generator=g)
    out.backward(dout)
    dx, dw, db, _ = O.causal_conv1d_bwd(x, w, bias, dout=dout, activation=activation)
    for name, got, w_ in (("dx", x.grad, dx), ("dweight", w.grad, dw), ("dbias", bias.grad, db)):
        np.testing.assert_allclose(got.numpy(), w_, rtol=1e-4, atol=1e-5, err_msg=name)


def test_oracle_autograd_functions_pass_gradcheck():
    """tests/oracle_autograd.py (the checker the fused-mixer tests compose):
    its Functions' gradients, the oracle's analytic backward, agree with
    finite differences in float64, for the real and the complex-A scan and
    for the conv."""
    import oracle_autograd as OA

    g = torch.Generator().manual_seed(7)
    b, d, l, n = 1, 3, 5, 2
    f64 = dict(dtype=torch.float64)
    u = torch.randn(b, d, l, generator=g, **f64).requires_grad_()
    delta = (torch.rand(b, d, l, generator=g, **f64) * 0.5).requires_grad_()
    A = (-torch.rand(d, n, generator=g, **f64) - 0.5).requires_grad_()
    B = torch.randn(b, n, l, generator=g, **f64).requires_grad_()
    C = torch.randn(b, n, l, generator=g, **f64).requires_grad_()
    D = torch.randn(d, generator=g, **f64).requires_grad_()
    z = torch.randn(b, d, l, generator=g, **f64).requires_grad_()
    bias = (torch.rand(d, generator=g, **f64) * 0.1).requires_grad_()
    assert torch.autograd.gradcheck(lambda *a: OA.scan(*a, True), (u, delta, A, B, C, D, z, bias))
    Ac = torch.complex(-torch.rand(d, n, generator=g, **f64) - 0.5,
                       torch.randn(d, n, generator=g, **f64)).requires_grad_()
    Bp = torch.randn(b, n, 2 * l, generator=g, **f64).requires_grad_()
    Cp = torch.randn(b, n, 2 * l, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda *a: OA.scan(*a, True), (u, delta, Ac, Bp, Cp, D, z, bias))
    x = torch.randn(2, 3, 6, generator=g, **f64).requires_grad_()
    w = torch.randn(3, 4, generator=g, **f64).requires_grad_()
    cb = torch.randn(3, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda *a: OA.conv(*a, "silu"), (x, w, cb))

"""selective_scan_fn with complex A on the GPU against the float64 oracle.

Complex A follows mamba_ssm's semantics (the reference rejects it,
src/mamba_cpu/ops/selective_scan_interface.py:160-161): input-dependent B/C
are real (batch, [ngroups,] dstate, 2 * seqlen) with (re, im) pairs along the
last dim, input-independent ones (dim, dstate) complex or real, and
y = 2 Re(<h, C>) + D u. The expected values come from
oracle.numerics.selective_scan_fwd_complex / selective_scan_bwd_complex,
which tests/test_oracle.py pins against a closed-form direct sum, the real
scan and torch.autograd. Complex gradients are dLoss/dRe + i dLoss/dIm
(torch's convention).
Tolerances: float32 outputs rtol 1e-4 / atol 2e-5, gradients rtol 1e-3 / atol
1e-4 after scaling by the gradient's magnitude; bf16 inputs 1e-2 / 2e-2.
Above 32 states the kernels scan 32-state slices side by side and finish
from their shares (dstate 33 to 128, with groups, z, D, bias, both loss
terms, a long sequence and bf16 inputs).
"""

import numpy as np
import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL
from oracle import numerics as O

from mamba_cpu import selective_scan_fn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_cinputs(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias, dtype=torch.float32,
                 bc2d=(), requires_grad=False, seed=0):
    g = torch.Generator().manual_seed(seed)

    def rand(*shape, dt=torch.float32):
        return torch.randn(*shape, generator=g).to(dt)

    bc_shape = (batch, dstate, 2 * seqlen) if ngroups is None else (batch, ngroups, dstate, 2 * seqlen)

    def bc(name):
        if name in bc2d:
            return torch.complex(rand(dim, dstate), rand(dim, dstate))
        return rand(*bc_shape)

    inp = dict(
        u=rand(batch, dim, seqlen, dt=dtype),
        delta=(torch.rand(batch, dim, seqlen, generator=g) * 0.5).to(dtype),
        A=torch.complex(-torch.rand(dim, dstate, generator=g) - 0.5, rand(dim, dstate) * 3),
        B=bc("B"),
        C=bc("C"),
        D=rand(dim) if has_D else None,
        z=rand(batch, dim, seqlen, dt=dtype) if has_z else None,
        delta_bias=(torch.rand(dim, generator=g) * 0.1) if has_bias else None,
    )
    return {k: None if v is None else v.to(DEV).requires_grad_(requires_grad) for k, v in inp.items()}


def as_np(t):
    t = t.detach().cpu()
    return t.to(torch.complex128).numpy() if t.is_complex() else t.double().numpy()


def close(got, want, rtol, atol, name=""):
    got, want = as_np(got), np.asarray(want)
    if np.iscomplexobj(got) or np.iscomplexobj(want):
        got, want = got.astype(np.complex128), want.astype(np.complex128)
        got = np.stack([got.real, got.imag], -1)
        want = np.stack([want.real, want.imag], -1)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol, err_msg=name)


def run_grads(inp, softplus, W, V):
    for v in inp.values():
        if v is not None:
            v.grad = None
    out, last = selective_scan_fn(**inp, delta_softplus=softplus, return_last_state=True)
    loss = 0
    if W is not None:
        loss = loss + (out.float() * W).sum()
    if V is not None:
        loss = loss + (torch.conj(V) * last).real.sum()
    loss.backward()
    return {k: v.grad for k, v in inp.items() if v is not None}


def check_grads(inp, softplus, W, V, rtol=GRAD_RTOL, atol=None):
    """Every gradient against the oracle, unscaled; atol per gradient from
    conftest.GRAD_ATOL unless one value is given. A bf16 out's upstream
    gradient is W rounded to bf16, and the oracle gets that."""
    got = run_grads(inp, softplus, W, V)
    if W is not None:
        W = W.to(inp["u"].dtype).float()
    want = O.selective_scan_bwd_complex(**inp, delta_softplus=softplus, dout=W, dlast_state=V)
    names = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]
    for k, w in zip(names, want):
        if inp[k] is None:
            continue
        g = got[k]
        assert g is not None, k
        assert g.dtype == inp[k].dtype, k
        close(g, w, rtol, GRAD_ATOL[k] if atol is None else atol, k)


@pytest.mark.parametrize("batch,dim,seqlen,dstate", [(1, 4, 1, 1), (2, 16, 33, 16), (3, 32, 100, 8),
                                                     (2, 20, 50, 24)])
@pytest.mark.parametrize("ngroups", [None, 2])
@pytest.mark.parametrize("has_D,has_z,has_bias,softplus", [
    (False, False, False, False),
    (True, True, True, True),
])
def test_complex_forward_matches_oracle(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias, softplus):
    if ngroups is not None and dim % ngroups:
        pytest.skip("dim not divisible by ngroups")
    inp = make_cinputs(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias)
    out, last = selective_scan_fn(**inp, delta_softplus=softplus, return_last_state=True)
    want, want_last = O.selective_scan_fwd_complex(**inp, delta_softplus=softplus)
    assert out.dtype == torch.float32 and last.dtype == torch.complex64
    close(out, want, 1e-4, 2e-5, "out")
    close(last, want_last, 1e-4, 2e-5, "last_state")


@pytest.mark.parametrize("batch,dim,seqlen,dstate", [(1, 4, 1, 1), (2, 8, 17, 4), (2, 40, 70, 16),
                                                     (1, 16, 40, 32)])
@pytest.mark.parametrize("ngroups", [None, 2])
@pytest.mark.parametrize("has_D,has_z,has_bias,softplus", [
    (False, False, False, False),
    (True, True, True, True),
])
@pytest.mark.parametrize("loss_on", [("out", "last"), ("out",)])
def test_complex_backward_matches_oracle(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias,
                                         softplus, loss_on):
    if ngroups is not None and dim % ngroups:
        pytest.skip("dim not divisible by ngroups")
    inp = make_cinputs(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias, requires_grad=True)
    g = torch.Generator().manual_seed(1)
    W = torch.randn(batch, dim, seqlen, generator=g).to(DEV) if "out" in loss_on else None
    V = (torch.complex(torch.randn(batch, dim, dstate, generator=g), torch.randn(batch, dim, dstate, generator=g))
         .to(DEV) if "last" in loss_on else None)
    check_grads(inp, softplus, W, V)


@pytest.mark.parametrize("bc2d", [("B",), ("C",), ("B", "C")])
def test_complex_input_independent_bc(bc2d):
    inp = make_cinputs(2, 24, 37, 8, None, True, True, True, bc2d=bc2d, requires_grad=True, seed=3)
    out = selective_scan_fn(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    close(out, want, 1e-4, 2e-5, "out")
    W = torch.randn(2, 24, 37, generator=torch.Generator().manual_seed(4)).to(DEV)
    check_grads(inp, True, W, None)


def test_complex_real_2d_bc_is_input_independent():
    # A real (dim, dstate) B with complex A is the complex B with zero imaginary part.
    inp = make_cinputs(1, 16, 20, 4, None, True, False, False, seed=5)
    B2 = torch.randn(16, 4, generator=torch.Generator().manual_seed(6)).to(DEV)
    got = selective_scan_fn(**{**inp, "B": B2})
    want = selective_scan_fn(**{**inp, "B": B2.to(torch.complex64)})
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_complex_low_precision():
    inp = make_cinputs(2, 16, 48, 16, None, True, True, True, dtype=torch.bfloat16, requires_grad=True,
                       seed=7)
    out = selective_scan_fn(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    assert out.dtype == torch.bfloat16
    close(out, want, 1e-2, 1e-2, "out")
    W = torch.randn(2, 16, 48, generator=torch.Generator().manual_seed(8)).to(DEV)
    check_grads(inp, True, W, None, 2e-2, 2e-2)


def test_complex_long_sequence():
    # Angles and states accumulate over thousands of steps (and many blocks).
    inp = make_cinputs(1, 16, 3000, 16, None, True, True, True, requires_grad=True, seed=9)
    out = selective_scan_fn(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    close(out, want, 1e-4, 5e-5, "out")
    W = torch.randn(1, 16, 3000, generator=torch.Generator().manual_seed(10)).to(DEV)
    check_grads(inp, True, W, None)


def test_complex_rejections():
    inp = make_cinputs(1, 4, 8, 2, None, False, False, False)
    with pytest.raises(ValueError, match="input-independent"):
        selective_scan_fn(**{**inp, "B": torch.complex(inp["B"], inp["B"])})
    with pytest.raises(ValueError, match="2 \\* seqlen"):
        selective_scan_fn(**{**inp, "C": inp["C"][..., :8]})


def test_opcheck_complex_ops():
    inp = make_cinputs(2, 4, 8, 2, 2, True, True, True)
    u, delta, A = inp["u"], inp["delta"], inp["A"]
    Bk = inp["B"].unflatten(-1, (8, 2)).transpose(2, 3)
    Ck = inp["C"].unflatten(-1, (8, 2)).transpose(2, 3)
    fwd_args = (u, delta, A, Bk, Ck, inp["D"], inp["z"], inp["delta_bias"], True)
    torch.library.opcheck(torch.ops.mamba_cpu.selective_scan_cfwd.default, fwd_args)
    _, _, ckpt = torch.ops.mamba_cpu.selective_scan_cfwd(*fwd_args)
    dlast = torch.complex(torch.randn(2, 4, 2), torch.randn(2, 4, 2)).to(DEV)
    bwd_args = fwd_args + (torch.randn(2, 4, 8, device=DEV), dlast, ckpt)
    torch.library.opcheck(torch.ops.mamba_cpu.selective_scan_cbwd.default, bwd_args)


def test_complex_channel_contiguous_inputs():
    """u, delta and z as channel-contiguous views (Hugging Face's transposed
    projections): same results as the oracle, the output and du / ddelta /
    dz keep that layout."""
    inp = make_cinputs(2, 32, 45, 8, None, True, True, True, seed=11)
    cc = {k: (v.transpose(1, 2).contiguous().transpose(1, 2) if k in ("u", "delta", "z") else v.clone())
          for k, v in inp.items()}
    for v in cc.values():
        v.requires_grad_()
    out = selective_scan_fn(**cc, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    close(out, want, 1e-4, 2e-5, "out")
    assert out.stride(1) == 1
    W = torch.randn(2, 32, 45, generator=torch.Generator().manual_seed(12)).to(DEV)
    (out * W).sum().backward()
    wants = O.selective_scan_bwd_complex(**inp, delta_softplus=True, dout=W)
    for k, w in zip(["u", "delta", "A", "B", "C", "D", "z", "delta_bias"], wants):
        close(cc[k].grad, w, GRAD_RTOL, GRAD_ATOL[k], k)
    assert cc["u"].grad.stride(1) == 1 and cc["z"].grad.stride(1) == 1


@pytest.mark.parametrize("batch,dim,seqlen,dstate,ngroups", [(2, 16, 40, 33, None), (1, 20, 70, 48, 2),
                                                            (2, 8, 100, 64, None), (1, 12, 37, 128, 3)])
@pytest.mark.parametrize("has_D,has_z,has_bias,softplus", [
    (False, False, False, False),
    (True, True, True, True),
])
def test_complex_dstate_above_32_matches_oracle(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias,
                                                softplus):
    inp = make_cinputs(batch, dim, seqlen, dstate, ngroups, has_D, has_z, has_bias, requires_grad=True,
                       seed=dstate)
    with torch.no_grad():
        out, last = selective_scan_fn(**inp, delta_softplus=softplus, return_last_state=True)
    want, want_last = O.selective_scan_fwd_complex(**inp, delta_softplus=softplus)
    close(out, want, 1e-4, 2e-5, "out")
    close(last, want_last, 1e-4, 2e-5, "last_state")
    g = torch.Generator().manual_seed(dstate + 1)
    W = torch.randn(batch, dim, seqlen, generator=g).to(DEV)
    V = torch.complex(torch.randn(batch, dim, dstate, generator=g), torch.randn(batch, dim, dstate, generator=g))
    check_grads(inp, softplus, W, V.to(DEV))


def test_complex_dstate_above_32_long_sequence_and_bf16():
    inp = make_cinputs(1, 8, 2000, 80, None, True, True, True, requires_grad=True, seed=11)
    out = selective_scan_fn(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    close(out, want, 1e-4, 5e-5, "out")
    W = torch.randn(1, 8, 2000, generator=torch.Generator().manual_seed(12)).to(DEV)
    check_grads(inp, True, W, None)
    inp = make_cinputs(2, 16, 60, 40, None, True, True, True, dtype=torch.bfloat16, seed=13)
    out = selective_scan_fn(**inp, delta_softplus=True)
    want, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    close(out.float(), want, 1e-2, 2e-2, "out bf16")

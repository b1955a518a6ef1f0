"""The fused mixer (mamba_cpu.ops.mamba_inner_fn) against the same mixer
composed in float64 on the CPU around the oracle: the conv and the scan are
oracle/numerics.py's forward and analytic backward (as autograd Functions,
tests/oracle_autograd.py), the projections and mamba_ssm's optional RMS
norms (B and C over dstate, delta over dim) are torch's own float64 ops.
Forward and every gradient, unscaled: output rtol 1e-4 / atol 1e-4; the
input gradient rtol 1e-3 / atol 1e-4; weight gradients (sums over batch and
sequence) rtol 1e-3 / atol 1e-3."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle_autograd as OA
from conftest import assert_close_report

from mamba_cpu import mamba_inner_fn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rms(x, w, eps):
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def reference_inner(xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, out_proj_b, A, D, delta_bias,
                    rms_w=None, eps=1e-6):
    d = xz.shape[1] // 2
    R, N = dt_proj_w.shape[1], A.shape[1]
    x, z = xz[:, :d], xz[:, d:]
    conv = OA.conv(x, conv_w.reshape(d, -1), conv_b, "silu")
    dt, B, C = F.linear(conv.transpose(1, 2), x_proj_w).split([R, N, N], dim=-1)
    delta = F.linear(dt, dt_proj_w)
    if rms_w is not None:  # mamba_ssm's norms: B, C over dstate, delta over dim
        delta, B, C = _rms(delta, rms_w[2], eps), _rms(B, rms_w[0], eps), _rms(C, rms_w[1], eps)
    delta = delta.transpose(1, 2)
    y = OA.scan(conv, delta, A, B.transpose(1, 2), C.transpose(1, 2), D, z, delta_bias, True)
    return F.linear(y.transpose(1, 2), out_proj_w, out_proj_b)


def check_grad(name, got, want):
    atol = 1e-4 if name == "xz" else 1e-3
    assert_close_report(got, want, 1e-3, atol, name)


def make(b, d, l, N, R, Dm, width, rms, bias, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=1.0: torch.randn(*s, generator=g, dtype=torch.float64) * sc  # noqa: E731
    p = dict(
        xz=r(b, l, 2 * d).transpose(1, 2),  # transformers' transposed view of in_proj's output
        conv_w=r(d, 1, width, sc=0.5), conv_b=r(d, sc=0.3) if bias else None,
        x_proj_w=r(R + 2 * N, d, sc=d ** -0.5), dt_proj_w=r(d, R, sc=R ** -0.5),
        out_proj_w=r(Dm, d, sc=d ** -0.5), out_proj_b=r(Dm, sc=0.1) if bias else None,
        A=-torch.exp(torch.rand(d, N, generator=g, dtype=torch.float64) * 2),
        D=r(d), delta_bias=torch.rand(d, generator=g, dtype=torch.float64) - 3,
    )
    rms_w = [1 + 0.1 * r(N), 1 + 0.1 * r(N), 1 + 0.1 * r(d)] if rms else None
    return p, rms_w


@pytest.mark.parametrize("b,d,l,rms,bias", [(2, 24, 37, False, True), (2, 40, 64, True, True),
                                            (3, 16, 19, False, False), (1, 64, 3000, False, True)])
def test_fused_mixer_matches_reference(b, d, l, rms, bias):
    N, R, Dm, width = 8, 4, 16, 4
    p, rms_w = make(b, d, l, N, R, Dm, width, rms, bias)
    names = [k for k, v in p.items() if v is not None]
    cpu = {k: (v.clone().requires_grad_() if v is not None else None) for k, v in p.items()}
    cpu_rms = [w.clone().requires_grad_() for w in rms_w] if rms else None
    want = reference_inner(**cpu, rms_w=cpu_rms)
    G = torch.randn(want.shape, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    (want * G).sum().backward()

    gpu = {}
    for k, v in p.items():
        if v is None:
            gpu[k] = None
        elif k == "xz":  # keep the transposed-view layout on the GPU
            gpu[k] = v.transpose(1, 2).float().to(DEV).transpose(1, 2).detach().requires_grad_()
        else:
            gpu[k] = v.float().to(DEV).requires_grad_()
    gpu_rms = [w.float().to(DEV).requires_grad_() for w in rms_w] if rms else [None] * 3
    got = mamba_inner_fn(gpu["xz"], gpu["conv_w"], gpu["conv_b"], gpu["x_proj_w"], gpu["dt_proj_w"],
                         gpu["out_proj_w"], gpu["out_proj_b"], gpu["A"], None, None, gpu["D"],
                         gpu["delta_bias"], delta_softplus=True, b_rms_weight=gpu_rms[0],
                         c_rms_weight=gpu_rms[1], dt_rms_weight=gpu_rms[2])
    (got * G.float().to(DEV)).sum().backward()
    assert_close_report(got, want, 1e-4, 1e-4, "out")
    pairs = [(k, gpu[k], cpu[k]) for k in names]
    if rms:
        pairs += [(f"rms{i}", gpu_rms[i], cpu_rms[i]) for i in range(3)]
    for k, g_, c_ in pairs:
        check_grad(k, g_.grad, c_.grad)
    # in_proj's gradient comes back in (batch, seqlen, 2 dim) order: no copy before in_proj.
    assert gpu["xz"].grad.transpose(1, 2).is_contiguous()


def test_rejects_input_independent_bc():
    p, _ = make(1, 8, 5, 4, 2, 8, 4, False, True)
    g = {k: v.float().to(DEV) if v is not None else None for k, v in p.items()}
    with pytest.raises(NotImplementedError):
        mamba_inner_fn(g["xz"], g["conv_w"], g["conv_b"], g["x_proj_w"], g["dt_proj_w"], g["out_proj_w"],
                       g["out_proj_b"], g["A"], torch.zeros(8, 4, device=DEV), None, g["D"])


def test_opcheck_inner_ops():
    """Schemas and shape functions of the two C++ operators behind the
    norm-free mixer."""
    p, _ = make(2, 16, 20, 4, 3, 12, 4, False, True, seed=5)
    t = {k: v.float().to(DEV) for k, v in p.items()}
    args = (t["xz"], t["conv_w"], t["conv_b"], t["x_proj_w"], t["dt_proj_w"], t["out_proj_w"], t["out_proj_b"],
            t["A"], t["D"], t["delta_bias"], True)
    torch.library.opcheck(torch.ops.mamba_cpu.mamba_inner_fwd.default, args)
    res = torch.ops.mamba_cpu.mamba_inner_fwd(*args)
    bargs = ((torch.randn_like(res[0]), t["xz"], t["conv_w"], t["conv_b"], t["x_proj_w"], t["dt_proj_w"],
              t["out_proj_w"], True, t["A"], t["D"], t["delta_bias"], True) + tuple(res[1:]))
    torch.library.opcheck(torch.ops.mamba_cpu.mamba_inner_bwd.default, bargs)


def test_complex_a_mixer_matches_reference():
    """Complex A through mamba_inner_fn (mamba_ssm's layout: B and C as 2 dstate
    columns of (re, im) pairs each) against the same mixer in float64 on the
    CPU around the oracle's complex-A scan. Output and every gradient."""
    b, d, l, N, R, Dm, W = 2, 16, 12, 4, 3, 10, 4
    g = torch.Generator().manual_seed(21)
    r = lambda *s, sc=1.0: torch.randn(*s, generator=g, dtype=torch.float64) * sc  # noqa: E731
    p = dict(xz=r(b, l, 2 * d).transpose(1, 2), conv_w=r(d, 1, W, sc=0.5), conv_b=r(d, sc=0.3),
             x_proj_w=r(R + 4 * N, d, sc=d ** -0.5), dt_proj_w=r(d, R, sc=R ** -0.5),
             out_proj_w=r(Dm, d, sc=d ** -0.5),
             A=torch.complex(-torch.exp(torch.rand(d, N, generator=g, dtype=torch.float64)), r(d, N)),
             D=r(d), delta_bias=torch.rand(d, generator=g, dtype=torch.float64) - 3)
    G = r(b, l, Dm)

    def pairs(X):
        return X.unflatten(-1, (N, 2)).permute(0, 2, 1, 3).reshape(b, N, 2 * l)

    ref = {k: v.clone().requires_grad_() for k, v in p.items()}
    x, z = ref["xz"][:, :d], ref["xz"][:, d:]
    conv = OA.conv(x, ref["conv_w"].reshape(d, -1), ref["conv_b"], "silu")
    dt, Bp, Cp = F.linear(conv.transpose(1, 2), ref["x_proj_w"]).split([R, 2 * N, 2 * N], -1)
    delta = F.linear(dt, ref["dt_proj_w"]).transpose(1, 2)
    y = OA.scan(conv, delta, ref["A"], pairs(Bp), pairs(Cp), ref["D"], z, ref["delta_bias"], True)
    want = F.linear(y.transpose(1, 2), ref["out_proj_w"])
    (want * G).sum().backward()

    gpu = {k: (v.to(torch.complex64) if v.is_complex() else v.float()).to(DEV).requires_grad_()
           for k, v in p.items()}
    out = mamba_inner_fn(gpu["xz"], gpu["conv_w"], gpu["conv_b"], gpu["x_proj_w"], gpu["dt_proj_w"],
                         gpu["out_proj_w"], None, gpu["A"], None, None, gpu["D"], gpu["delta_bias"],
                         delta_softplus=True)
    assert_close_report(out, want, 1e-4, 1e-5, "out")
    (out * G.float().to(DEV)).sum().backward()
    for k in p:
        got, w = gpu[k].grad.cpu(), ref[k].grad
        if w.is_complex():
            got, w = torch.view_as_real(got.to(torch.complex128)), torch.view_as_real(w)
        check_grad(k, got, w)

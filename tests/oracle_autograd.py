"""The float64 oracle's scan and conv as torch autograd Functions (CPU,
float64), so a test can compose a whole mixer around them with torch's own
linear layers and norms, and take every gradient by autograd: the scan's and
conv's gradients come from the oracle's pinned analytic backward
(oracle/numerics.py), not from torch."""

import torch

from oracle import numerics as O


def _t(a, like):
    return None if a is None else torch.as_tensor(a, dtype=like.dtype)


class OracleScan(torch.autograd.Function):
    """selective_scan over O.selective_scan_fwd / _bwd (real A) or their
    complex-A counterparts. Arguments as selective_scan_fn's; returns out."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, softplus):
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias)
        ctx.softplus = softplus
        fwd = O.selective_scan_fwd_complex if A.is_complex() else O.selective_scan_fwd
        out, _ = fwd(u, delta, A, B, C, D, z, delta_bias, softplus)
        return torch.as_tensor(out, dtype=u.dtype)

    @staticmethod
    def backward(ctx, dout):
        u, delta, A, B, C, D, z, delta_bias = ctx.saved_tensors
        bwd = O.selective_scan_bwd_complex if A.is_complex() else O.selective_scan_bwd
        grads = bwd(u, delta, A, B, C, D, z, delta_bias, ctx.softplus, dout=dout)
        like = (u, delta, A, B, C, D, z, delta_bias)
        out = []
        for g, t in zip(grads, like):
            if g is None or t is None:
                out.append(None)
            else:
                out.append(torch.as_tensor(g).to(t.dtype) if t.is_complex() else _t(g, t))
        return (*out, None)


class OracleConv(torch.autograd.Function):
    """causal_conv1d over O.causal_conv1d_fwd / _bwd; weight (dim, width)."""

    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        ctx.save_for_backward(x, weight, bias)
        ctx.activation = activation
        out, _ = O.causal_conv1d_fwd(x, weight, bias, activation=activation)
        return torch.as_tensor(out, dtype=x.dtype)

    @staticmethod
    def backward(ctx, dout):
        x, weight, bias = ctx.saved_tensors
        dx, dw, db, _ = O.causal_conv1d_bwd(x, weight, bias, dout=dout, activation=ctx.activation)
        return _t(dx, x), _t(dw, weight), _t(db, bias) if bias is not None else None, None


def scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    return OracleScan.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus)


def conv(x, weight, bias=None, activation=None):
    return OracleConv.apply(x, weight, bias, activation)

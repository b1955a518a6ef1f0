"""Pure-PyTorch definitions of the selective scan and the causal conv1d.

Exported for API compatibility: the reference package exports
selective_scan_ref and causal_conv1d_ref with these signatures
(src/mamba_cpu/reference.py:10-21, 65). They are written for reading, not
speed: device-agnostic, differentiable by autograd, one Python step per time
step. No op of this package calls them, and the test suite pins them against
the float64 oracle (tests/test_reference_module.py).

They accept what selective_scan_fn / causal_conv1d_fn accept, so a
result of either op can be checked against them directly: B and C with their
own group counts, input-independent (dim, dstate) B/C, and complex A with
mamba_ssm's semantics (input-dependent B/C then hold (re, im) pairs along
their last dimension, and y = 2 Re(<h, C>)).
"""

import torch
import torch.nn.functional as F


def _per_channel(X, batch, dim, seqlen, pairs):
    """B or C as a (batch, dim, seqlen, dstate) view: each channel sees its
    group's values (channels split into contiguous groups); a (dim, dstate)
    tensor is constant in time. With pairs, an input-dependent X holds
    (re, im) pairs along its last dim and becomes complex."""
    if X.dim() == 2:
        X = X.to(torch.complex64) if pairs else X.float()
        return X[None, :, None, :].expand(batch, dim, seqlen, X.shape[1])
    X = X.float()
    if X.dim() == 3:
        X = X.unsqueeze(1)
    if pairs:
        X = torch.view_as_complex(X.unflatten(-1, (seqlen, 2)).contiguous())
    groups, dstate = X.shape[1], X.shape[2]
    X = X.transpose(-1, -2)  # (batch, groups, seqlen, dstate)
    return X.unsqueeze(2).expand(batch, groups, dim // groups, seqlen, dstate).reshape(
        batch, dim, seqlen, dstate)


def selective_scan_ref(
    u,
    delta,
    A,
    B,
    C,
    D=None,
    z=None,
    delta_bias=None,
    delta_softplus=False,
    return_last_state=False,
):
    """The selective scan, step by step in float32 (complex64 states for a
    complex A):
        dt_t = softplus?(delta_t + delta_bias)
        h_t  = exp(dt_t A) h_{t-1} + dt_t u_t B_t        (h_{-1} = 0)
        y_t  = <h_t, C_t> + D u_t    (2 Re<h_t, C_t> + D u_t for complex A)
        out  = y * silu(z)           when z is given
    u, delta, z: (batch, dim, seqlen); A: (dim, dstate);
    B, C: (batch, dstate, seqlen), (batch, ngroups, dstate, seqlen) or
          (dim, dstate); with complex A an input-dependent B/C is
          (batch, [ngroups,] dstate, 2 * seqlen) of (re, im) pairs;
    D, delta_bias: (dim,).
    Returns out in u's dtype [, last_state (batch, dim, dstate) float32, or
    complex64 for complex A]."""
    batch, dim, seqlen = u.shape
    cplx = A.is_complex()
    dt = delta.float()
    if delta_bias is not None:
        dt = dt + delta_bias.float().unsqueeze(-1)
    if delta_softplus:
        dt = F.softplus(dt)
    x = u.float()
    Ac = A.to(torch.complex64) if cplx else A.float()
    Bc = _per_channel(B, batch, dim, seqlen, cplx)
    Cc = _per_channel(C, batch, dim, seqlen, cplx)
    step = dt.unsqueeze(-1)                            # (batch, dim, seqlen, 1)
    decay = torch.exp(step * Ac.unsqueeze(1))          # (batch, dim, seqlen, dstate)
    drive = (step * x.unsqueeze(-1)) * Bc              # (batch, dim, seqlen, dstate)
    h = torch.zeros(batch, dim, A.shape[1], dtype=decay.dtype, device=u.device)
    ys = []
    for t in range(seqlen):
        h = torch.addcmul(drive[:, :, t], decay[:, :, t], h)
        yt = (h * Cc[:, :, t]).sum(-1)
        ys.append(2 * yt.real if cplx else yt)
    y = torch.stack(ys, dim=-1) if ys else x.new_zeros(batch, dim, 0)
    if D is not None:
        y = y + D.float().unsqueeze(-1) * x
    if z is not None:
        y = y * F.silu(z.float())
    out = y.to(u.dtype)
    return (out, h) if return_last_state else out


def causal_conv1d_ref(x, weight, bias=None, activation=None):
    """Depthwise causal conv1d, one term per tap:
        out_t = act(bias + sum_k weight[:, k] x_{t - (width - 1) + k})
    with x_s = 0 for s < 0. x: (batch, dim, seqlen); weight: (dim, width);
    bias: (dim,); activation None, "silu" or "swish". The result has the
    promoted dtype of x and weight."""
    width, seqlen = weight.shape[1], x.shape[-1]
    out = None
    for k in range(width):
        shift = width - 1 - k                          # tap k reads x delayed by `shift` steps
        delayed = F.pad(x, (shift, 0))[..., :seqlen] if shift else x
        term = weight[:, k].unsqueeze(-1) * delayed
        out = term if out is None else out + term
    if bias is not None:
        out = out + bias.unsqueeze(-1)
    if activation in ("silu", "swish"):
        out = F.silu(out)
    return out

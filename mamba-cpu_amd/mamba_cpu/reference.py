"""Readable pure-PyTorch definitions of the selective scan and the causal
conv1d, kept for API compatibility with the reference package
(src/mamba_cpu/reference.py:10-75 exports selective_scan_ref and
causal_conv1d_ref). They run on any device, loop over time in Python, and no op
of this package calls them.
"""

import torch
import torch.nn.functional as F


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
    """
    u, delta, z: (batch, dim, seqlen)
    A: (dim, dstate)
    B, C: (batch, dstate, seqlen) or (batch, ngroups, dstate, seqlen) (each
          with its own group count), or (dim, dstate) input-independent
    D, delta_bias: (dim,)
    Returns out: (batch, dim, seqlen) [, last_state: (batch, dim, dstate)]

    h_t = exp(dt_t A) h_{t-1} + dt_t u_t B_t ; y_t = <h_t, C_t> + D u_t ;
    out = y * silu(z), with dt = softplus?(delta + delta_bias), in float32.
    """
    in_dtype = u.dtype
    u = u.float()
    dt = delta.float()
    if delta_bias is not None:
        dt = dt + delta_bias.float()[:, None]
    if delta_softplus:
        dt = F.softplus(dt)
    batch, dim, seqlen = u.shape
    A = A.float()

    def per_channel(X):  # (batch, dim, dstate, seqlen); B and C group independently
        if X.dim() == 2:  # input-independent (dim, dstate)
            return X.float()[None, :, :, None].expand(batch, dim, X.shape[1], seqlen)
        Xg = X.float() if X.dim() == 4 else X.float()[:, None]
        return Xg.repeat_interleave(dim // Xg.shape[1], dim=1)

    Bd, Cd = per_channel(B), per_channel(C)
    h = u.new_zeros(batch, dim, A.shape[1])
    ys = []
    for t in range(seqlen):
        h = torch.exp(dt[:, :, t, None] * A) * h + (dt[:, :, t] * u[:, :, t])[..., None] * Bd[..., t]
        ys.append((h * Cd[..., t]).sum(-1))
    y = torch.stack(ys, dim=-1) if ys else u.new_zeros(batch, dim, 0)
    if D is not None:
        y = y + D.float()[:, None] * u
    if z is not None:
        y = y * F.silu(z.float())
    y = y.to(in_dtype)
    return (y, h) if return_last_state else y


def causal_conv1d_ref(x, weight, bias=None, activation=None):
    """x: (batch, dim, seqlen), weight: (dim, width). One term per tap."""
    width = weight.shape[1]
    seqlen = x.shape[-1]
    xp = F.pad(x, (width - 1, 0))
    out = torch.zeros_like(x)
    for k in range(width):
        out = out + weight[:, k, None] * xp[..., k:k + seqlen]
    if bias is not None:
        out = out + bias[:, None]
    if activation in ("silu", "swish"):
        out = F.silu(out)
    return out

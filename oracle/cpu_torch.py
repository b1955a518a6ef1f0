"""The reference's CPU execution path, in torch on host tensors — TEST AND
BASELINE INFRASTRUCTURE ONLY.

`bench.py` times these on the host cores as the CPU baseline of every
workload; `tests/test_oracle.py` checks them against `oracle.numerics`. The
product never imports this module.

What runs here is what mamba-cpu runs on CPU:
  selective scan       the reference's own C++ kernels (csrc/selective_scan.cpp,
                       built unchanged into oracle/_ref by oracle/Makefile),
                       wrapped in an autograd Function the way
                       ops/selective_scan_interface.py:16-124 wraps them;
  causal conv1d        the same ATen calls as ops/causal_conv1d.py:16-85
                       (F.pad / cat, depthwise F.conv1d, silu), autograd
                       through ATen;
  state update         the same ATen calls as ops/selective_state_update.py:5-57;
  transformers routing hf.py:26-112's table: the four ops above, and
                       mamba_inner_fn -> None so the mixer takes its unfused path.
"""

import contextlib
import importlib

import numpy as np
import torch
import torch.nn.functional as F

from oracle import ref as R


def _activate(x, activation):
    """ops/causal_conv1d.py:8-13."""
    if activation is None:
        return x
    if activation in ("silu", "swish"):
        return F.silu(x)
    raise ValueError(f"activation must be None, 'silu' or 'swish', got {activation!r}")


def causal_conv1d_fn(x, weight, bias=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None):
    """ops/causal_conv1d.py:16-53: left pad (or initial_states), depthwise
    F.conv1d in the weight's dtype, activation, cast back to x's dtype."""
    width = weight.shape[1]
    if initial_states is None:
        x_full = F.pad(x, (width - 1, 0))
    else:
        x_full = torch.cat([initial_states.to(x.dtype), x], dim=-1)
    out = F.conv1d(x_full.to(weight.dtype), weight.unsqueeze(1),
                   None if bias is None else bias.to(weight.dtype), groups=x.shape[1])
    out = _activate(out, activation).to(x.dtype)
    if not return_final_states:
        return out
    final = x_full[..., x_full.shape[-1] - (width - 1):]
    if final_states_out is not None:
        final = final_states_out.copy_(final)
    return out, final


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None):
    """ops/causal_conv1d.py:56-85: cat(state, x), state <- last state_len
    inputs (in place), conv over the last seqlen + width - 1 inputs."""
    single = x.dim() == 2
    xs = x.unsqueeze(-1) if single else x
    seqlen, width, state_len = xs.shape[-1], weight.shape[1], conv_state.shape[-1]
    x_full = torch.cat([conv_state.to(x.dtype), xs], dim=-1)
    conv_state.copy_(x_full[..., -state_len:])
    out = F.conv1d(x_full[..., -(seqlen + width - 1):].to(weight.dtype), weight.unsqueeze(1),
                   None if bias is None else bias.to(weight.dtype), groups=xs.shape[1])
    out = _activate(out, activation).to(x.dtype)
    return out.squeeze(-1) if single else out


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False):
    """ops/selective_state_update.py:5-57 (Mamba-1 and multi-head layouts):
    state <- state * exp(dt A) + dt x B (in place); out = <state, C> + D x,
    gated by silu(z)."""
    heads = state.dim() > 3
    if not heads:
        state, x, dt, A = state.unsqueeze(1), x.unsqueeze(1), dt.unsqueeze(1), A.unsqueeze(0)
        B, C = B.unsqueeze(1), C.unsqueeze(1)
        D = None if D is None else D.unsqueeze(0)
        z = None if z is None else z.unsqueeze(1)
        dt_bias = None if dt_bias is None else dt_bias.unsqueeze(0)
    nheads = state.shape[1]
    dt = dt.float()
    if dt_bias is not None:
        dt = dt + dt_bias.float()
    if dt_softplus:
        dt = F.softplus(dt)
    dA = torch.exp(dt.unsqueeze(-1) * A.float())
    B = B.float().repeat_interleave(nheads // B.shape[1], dim=1)
    C = C.float().repeat_interleave(nheads // C.shape[1], dim=1)
    new = state.float() * dA + (dt * x.float()).unsqueeze(-1) * B.unsqueeze(2)
    state.copy_(new)
    out = (new * C.unsqueeze(2)).sum(-1)
    if D is not None:
        out = out + x.float() * D.float()
    if z is not None:
        out = out * F.silu(z.float())
    out = out.to(x.dtype)
    return out if heads else out.squeeze(1)


def _np(t):
    return None if t is None else t.detach().float().contiguous().numpy()


class _Scan(torch.autograd.Function):
    """The reference's custom op pair with its autograd glue
    (selective_scan_interface.py:16-124): forward and backward are the C++
    kernels; dA, dD and ddelta_bias come back summed over the batch."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, softplus, threads):
        Bk, Ck = R.kernel_bc(_np(B)), R.kernel_bc(_np(C))
        out, last = R.scan_fwd(_np(u), _np(delta), _np(A), Bk, Ck, _np(D), _np(z), _np(delta_bias),
                               softplus, threads)
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias)
        ctx.softplus, ctx.threads = softplus, threads
        return torch.from_numpy(out), torch.from_numpy(last)

    @staticmethod
    def backward(ctx, gout, glast):
        u, delta, A, B, C, D, z, delta_bias = ctx.saved_tensors
        dout = torch.zeros_like(u) if gout is None else gout
        du, dd, dA, dB, dC, dD, dz, dbias = R.scan_bwd(
            _np(u), _np(delta), _np(A), R.kernel_bc(_np(B)), R.kernel_bc(_np(C)), _np(D), _np(z),
            _np(delta_bias), ctx.softplus, _np(dout), _np(glast), ctx.threads)

        def back(g, like):
            return None if like is None else torch.from_numpy(np.ascontiguousarray(g)).to(like.dtype)

        # dB/dC leave the kernels as (b, g, l, n); the inputs are (b, [g,] n, l).
        dB = torch.from_numpy(dB).transpose(-1, -2).reshape(B.shape)
        dC = torch.from_numpy(dC).transpose(-1, -2).reshape(C.shape)
        return (back(du, u), back(dd, delta), back(dA, A), dB.to(B.dtype), dC.to(C.dtype),
                back(dD, D), back(dz, z), back(dbias, delta_bias), None, None)


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False, threads=1):
    """selective_scan_interface.py:138-177 on the reference kernels: fp32
    compute, out cast to u's dtype, last_state in fp32."""
    out, last = _Scan.apply(u.float(), delta.float(), A.float(), B.float(), C.float(),
                            None if D is None else D.float(), None if z is None else z.float(),
                            None if delta_bias is None else delta_bias.float(), bool(delta_softplus),
                            int(threads))
    out = out.to(u.dtype)
    return (out, last) if return_last_state else out


@contextlib.contextmanager
def route_transformers(threads, model="mamba"):
    """Routes a transformers Mamba model's ops through the functions above, as
    hf.py:26-112 routes CPU tensors through mamba_cpu's ops, and restores the
    module globals on exit."""
    mod = importlib.import_module(f"transformers.models.{model}.modeling_{model}")

    def scan(hidden_states, dt, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
             return_last_state=False, **kwargs):
        return selective_scan_fn(hidden_states, dt, A, B, C, D, z, delta_bias, delta_softplus,
                                 return_last_state, threads)

    def state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False,
                     **kwargs):
        return selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus)

    def conv(x, weight, bias=None, activation=None, **kwargs):
        return causal_conv1d_fn(x, weight, bias, activation=activation)

    def conv_update(x, conv_state, weight, bias=None, activation=None, **kwargs):
        return causal_conv1d_update(x, conv_state, weight, bias, activation)

    table = {"mamba_selective_scan": scan, "mamba_selective_state_update": state_update,
             "causal_conv1d_fn": conv, "causal_conv1d_update": conv_update,
             "mamba_inner_fn": lambda *a, **k: None}
    saved = {k: getattr(mod, k) for k in table}
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        for k, fn in table.items():
            setattr(mod, k, fn)
        yield
    finally:
        for k, fn in saved.items():
            setattr(mod, k, fn)
        torch.set_num_threads(prev_threads)

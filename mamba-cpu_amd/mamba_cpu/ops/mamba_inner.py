"""mamba_inner_fn on MI355X: the Mamba-1 mixer after in_proj as one autograd
function.

    out = out_proj(scan(conv(x), dt_proj(x_proj(conv(x))[:dt_rank]), A, B, C, D, z, delta_bias))

with x, z = xz.chunk(2, dim=1) and B, C the next two dstate-wide column blocks
of x_proj's output. Same signature and result as mamba_ssm's
`mamba_inner_fn`, including its optional RMS norms (B and C over dstate,
delta over dim after dt_proj, each with its weight), which transformers'
Mamba mixers call in training
(transformers/models/mamba/modeling_mamba.py, the `self.training and
cache_params is None` branch). The reference answers None there
(src/mamba_cpu/hf.py:59-60), so the mixer runs its unfused path; this module
is the fused path that answer leaves out.

What the fusion buys on the GPU is layout: transformers' xz is the transposed
view of in_proj's (batch, seqlen, 2 dim) output. Here every tensor between
in_proj and out_proj stays in that channel-contiguous layout: the conv and
scan kernels read and write it directly (their operands and results take
strides), x_proj / dt_proj / out_proj are plain (batch * seqlen, .) GEMMs on
it, and the backward writes dx and dz into the two halves of one
(batch, seqlen, 2 dim) gradient, which in_proj's backward consumes as is. The
unfused path instead makes contiguous copies for every GEMM and concatenates
the input gradient through a transposing copy.

The backward keeps the forward's scan checkpoints and pre-gate y
(selective_scan_fwd_ckpt), so it does not recompute the states. Without the
RMS norms (transformers' Mamba mixers) the forward and the backward are one
C++ operator each, mamba_cpu::mamba_inner_fwd / mamba_inner_bwd, which issue
the conv, scan and GEMM calls themselves; with them, MambaInnerFn composes
the same operators from Python around the norms' autograd graph.
"""

import torch
import torch.nn.functional as F

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_ops = torch.ops.mamba_cpu


def _rms(x, weight, eps):
    """x * rsqrt(mean(x^2) + eps) * weight over the last dim."""
    return weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


class MambaInnerFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, out_proj_b, A, D,
                delta_bias, softplus, b_rms_w, c_rms_w, dt_rms_w, eps):
        b, d2, l = xz.shape
        d = d2 // 2
        R = dt_proj_w.shape[1]
        N = A.shape[1]
        x, z = xz[:, :d], xz[:, d:]
        w2 = conv_w.reshape(d, -1)
        conv_out, _ = _ops.causal_conv1d_fwd(x, w2, conv_b, None, False, True)
        conv_bl = conv_out.transpose(1, 2)  # (b, l, d)
        x_dbl = F.linear(conv_bl, x_proj_w)  # (b, l, R + 2N)
        dt_in, B, C = x_dbl.split([R, N, N], dim=-1)
        delta_bl = F.linear(dt_in, dt_proj_w)  # (b, l, d)
        if dt_rms_w is not None:
            delta_bl, B, C = _rms(delta_bl, dt_rms_w, eps), _rms(B, b_rms_w, eps), _rms(C, c_rms_w, eps)
        delta = delta_bl.transpose(1, 2)
        Bk, Ck = B.unsqueeze(1), C.unsqueeze(1)  # (b, 1, l, N) views, the kernels' layout
        y, _, ckpt, ysave = _ops.selective_scan_fwd_ckpt(conv_out, delta, A, Bk, Ck, D, z, delta_bias,
                                                         softplus)
        y_bl = y.transpose(1, 2)
        out = F.linear(y_bl, out_proj_w, out_proj_b)
        ctx.save_for_backward(xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, A, D, delta_bias,
                              conv_out, x_dbl, delta, ckpt, ysave, y, b_rms_w, c_rms_w, dt_rms_w)
        ctx.softplus, ctx.eps, ctx.has_out_b = softplus, eps, out_proj_b is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        (xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, A, D, delta_bias, conv_out, x_dbl,
         delta, ckpt, ysave, y, b_rms_w, c_rms_w, dt_rms_w) = ctx.saved_tensors
        b, d2, l = xz.shape
        d = d2 // 2
        R = dt_proj_w.shape[1]
        N = A.shape[1]
        x, z = xz[:, :d], xz[:, d:]
        dout = dout.contiguous()
        dout2 = dout.reshape(-1, dout.shape[-1])
        y2 = y.transpose(1, 2).reshape(-1, d)
        # out_proj
        d_out_proj_w = dout2.t().mm(y2)
        d_out_proj_b = dout2.sum(0) if ctx.has_out_b else None
        dy = dout.matmul(out_proj_w).transpose(1, 2)  # (b, d, l), channel-contiguous
        # x_proj output; with the RMS norms, their graph is rebuilt for their
        # own backward (delta before the norm is recomputed by one GEMM).
        dt_in, B_raw, C_raw = x_dbl.split([R, N, N], dim=-1)
        rms = dt_rms_w is not None
        if rms:
            with torch.enable_grad():
                leaves = [F.linear(dt_in, dt_proj_w).detach().requires_grad_(),
                          B_raw.detach().requires_grad_(), C_raw.detach().requires_grad_()]
                wts = [w.detach().requires_grad_() for w in (dt_rms_w, b_rms_w, c_rms_w)]
                normed = [_rms(v, w, ctx.eps) for v, w in zip(leaves, wts)]
            B, C = normed[1].detach(), normed[2].detach()
        else:
            B, C = B_raw, C_raw
        # scan
        du, ddelta, dA, dB, dC, dD, dz, ddelta_bias = _ops.selective_scan_bwd_ckpt(
            conv_out, delta, A, B.unsqueeze(1), C.unsqueeze(1), D, z, delta_bias, ctx.softplus, dy,
            None, ckpt, ysave)
        dB, dC = dB[:, 0], dC[:, 0]  # (b, l, N)
        ddelta_bl = ddelta.transpose(1, 2)  # (b, l, d)
        d_rms = (None, None, None)
        if rms:
            g = torch.autograd.grad(normed, leaves + wts, [ddelta_bl, dB, dC])
            ddelta_bl, dB, dC = g[0], g[1], g[2]
            d_rms = (g[4], g[5], g[3])  # b, c, dt weights
        # dt_proj: delta = dt_in @ dt_proj_w^T in (b, l, d)
        ddelta2 = ddelta_bl.reshape(-1, d)
        d_dt_proj_w = ddelta2.t().mm(dt_in.reshape(-1, R))
        d_dt_in = ddelta2.mm(dt_proj_w).view(b, l, R)
        dx_dbl = torch.cat([d_dt_in, dB, dC], dim=-1).reshape(-1, R + 2 * N)
        # x_proj, plus the scan's du, into the conv output's gradient (b, l, d)
        conv2 = conv_out.transpose(1, 2).reshape(-1, d)
        d_x_proj_w = dx_dbl.t().mm(conv2)
        dconv = torch.addmm(du.transpose(1, 2).reshape(-1, d), dx_dbl, x_proj_w).view(b, l, d)
        # conv, then dx and dz side by side in one (b, l, 2d) gradient
        dx, dw, dcb, _ = _ops.causal_conv1d_bwd(x, conv_w.reshape(d, -1), conv_b, None,
                                                dconv.transpose(1, 2), None, True)
        dxz = torch.empty(b, l, d2, dtype=xz.dtype, device=xz.device)
        dxz[..., :d].copy_(dx.transpose(1, 2))
        dxz[..., d:].copy_(dz.transpose(1, 2))
        return (dxz.transpose(1, 2), dw.view_as(conv_w), dcb if conv_b is not None else None, d_x_proj_w,
                d_dt_proj_w, d_out_proj_w, d_out_proj_b, dA, dD if D is not None else None,
                ddelta_bias if delta_bias is not None else None, None, d_rms[0], d_rms[1], d_rms[2],
                None)


def _like_channels(x):
    """(batch, dim, seqlen) result laid out like the operators allocate it for
    a channel-contiguous input view."""
    b, d, l = x.shape
    return torch.empty_strided((b, d, l), (d * l, 1, d), dtype=x.dtype, device=x.device)


@torch.library.register_fake("mamba_cpu::mamba_inner_fwd")
def _(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight, out_proj_bias,
      A, D, delta_bias, delta_softplus):
    b, d2, l = xz.shape
    d, N, R = d2 // 2, A.shape[1], delta_proj_weight.shape[1]
    x = xz[:, :d]
    conv_out = _like_channels(x) if x.stride(1) == 1 and x.stride(2) != 1 else x.new_empty(x.shape)
    return (xz.new_empty(b, l, out_proj_weight.shape[0]), conv_out, xz.new_empty(b, l, R + 2 * N),
            xz.new_empty(b, l, d).transpose(1, 2), xz.new_empty(b, d, (l + 15) // 16, N),
            xz.new_empty(b, d, l),
            torch.empty_strided(conv_out.shape, conv_out.stride(), dtype=xz.dtype, device=xz.device))


@torch.library.register_fake("mamba_cpu::mamba_inner_bwd")
def _(dout, xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
      has_out_proj_bias, A, D, delta_bias, delta_softplus, conv_out, x_dbl, delta, ckpt, ysave, y):
    b, d2, l = xz.shape
    d = d2 // 2
    f = A.new_empty
    return (xz.new_empty(b, l, d2).transpose(1, 2), f(conv1d_weight.shape),
            f(d) if conv1d_bias is not None else f(0), f(x_proj_weight.shape), f(delta_proj_weight.shape),
            f(out_proj_weight.shape), f(out_proj_weight.shape[0]) if has_out_proj_bias else f(0), f(A.shape),
            f(d), f(d))


class MambaInnerOpsFn(torch.autograd.Function):
    """mamba_inner_fn without the RMS norms: one C++ operator for the forward
    (conv, x_proj, dt_proj, scan, out_proj) and one for the backward, so a
    training step makes one Python call each way per layer."""

    @staticmethod
    def forward(ctx, xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, out_proj_b, A, D, delta_bias,
                softplus):
        out, conv_out, x_dbl, delta, ckpt, ysave, y = _ops.mamba_inner_fwd(
            xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, out_proj_b, A, D, delta_bias, softplus)
        ctx.save_for_backward(xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, A, D, delta_bias,
                              conv_out, x_dbl, delta, ckpt, ysave, y)
        ctx.softplus, ctx.has_out_b = softplus, out_proj_b is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        (xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, A, D, delta_bias, conv_out, x_dbl, delta,
         ckpt, ysave, y) = ctx.saved_tensors
        dxz, dcw, dcb, dxp, ddtp, dop, dopb, dA, dD, ddb = _ops.mamba_inner_bwd(
            dout, xz, conv_w, conv_b, x_proj_w, dt_proj_w, out_proj_w, ctx.has_out_b, A, D, delta_bias,
            ctx.softplus, conv_out, x_dbl, delta, ckpt, ysave, y)
        return (dxz, dcw, dcb if conv_b is not None else None, dxp, ddtp, dop,
                dopb if ctx.has_out_b else None, dA, dD if D is not None else None,
                ddb if delta_bias is not None else None, None)


def fused_path_supported(xz, conv1d_weight, x_proj_weight, delta_proj_weight, out_proj_weight, A, B, C):
    """The shapes and dtypes the fused path runs: float32 xz and weights on a
    ROCm GPU, input-dependent B/C (B = C = None), a real A."""
    tensors = (xz, conv1d_weight, x_proj_weight, delta_proj_weight, out_proj_weight, A)
    return (B is None and C is None and xz.dim() == 3 and xz.shape[1] % 2 == 0 and
            all(t.dtype == torch.float32 and t.device.type == "cuda" for t in tensors))


def _mamba_inner_complex(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                         out_proj_weight, out_proj_bias, A, D, delta_bias, delta_softplus):
    """mamba_inner_fn with complex A, composed from this package's ops (autograd
    through them): mamba_ssm's layout, where x_proj's output holds dt_rank
    columns, then B and C as 2 dstate columns each, the (re, im) pairs of each
    state side by side ("(b l) (dstate two) -> b 1 dstate (l two)")."""
    from mamba_cpu.ops.causal_conv1d import causal_conv1d_fn
    from mamba_cpu.ops.selective_scan_interface import selective_scan_fn

    b, d2, l = xz.shape
    d, R, N = d2 // 2, delta_proj_weight.shape[1], A.shape[1]
    if x_proj_weight.shape[0] != R + 4 * N:
        raise ValueError(f"with complex A, x_proj_weight has dt_rank + 4 dstate = {R + 4 * N} rows, "
                         f"got {x_proj_weight.shape[0]}")
    x, z = xz[:, :d], xz[:, d:]
    conv = causal_conv1d_fn(x, conv1d_weight.reshape(d, -1), conv1d_bias, activation="silu")
    x_dbl = F.linear(conv.transpose(1, 2), x_proj_weight)  # (b, l, R + 4N)
    dt_in, Bp, Cp = x_dbl.split([R, 2 * N, 2 * N], dim=-1)
    delta = F.linear(dt_in, delta_proj_weight).transpose(1, 2)

    def pairs(X):  # (b, l, N * 2) -> (b, N, l * 2)
        return X.unflatten(-1, (N, 2)).permute(0, 2, 1, 3).reshape(b, N, 2 * l)

    y = selective_scan_fn(conv, delta, A, pairs(Bp), pairs(Cp), D, z, delta_bias, delta_softplus)
    return F.linear(y.transpose(1, 2), out_proj_weight, out_proj_bias)


def mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                   out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                   B_proj_bias=None, C_proj_bias=None, delta_softplus=True, checkpoint_lvl=1,
                   b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None, b_c_dt_rms_eps=1e-6,
                   **kwargs):
    """The Mamba-1 mixer from xz = in_proj(hidden).transpose(1, 2) to
    out_proj's output (batch, seqlen, d_model), differentiable.

    xz: (batch, 2 dim, seqlen) float32 (any strides; transformers passes the
    transposed view of in_proj's output). conv1d_weight: (dim, 1, width) or
    (dim, width). x_proj_weight: (dt_rank + 2 dstate, dim). delta_proj_weight:
    (dim, dt_rank). out_proj_weight: (d_model, dim). A: (dim, dstate) real,
    or complex (mamba_ssm's layout: x_proj_weight then has dt_rank + 4 dstate
    rows, B and C as (re, im) pairs; composed from the ops, no RMS norms).
    D, delta_bias: (dim,). b_rms_weight / c_rms_weight (dstate,) and
    dt_rms_weight (dim,): RMS norms on B, C and delta, all or none.

    Input-independent B/C, projection biases on B/C and non-float32 inputs
    are not fused: NotImplementedError, which transformers' callers never
    reach (they pass B = C = None; the hf wrapper answers None for other
    dtypes so the mixer takes its unfused path)."""
    if B is not None or C is not None or B_proj_bias is not None or C_proj_bias is not None:
        raise NotImplementedError("mamba_inner_fn: input-independent B/C are not supported")
    if A.is_complex():
        if dt_rms_weight is not None or b_rms_weight is not None or c_rms_weight is not None:
            raise NotImplementedError("mamba_inner_fn: RMS norms with complex A are not supported")
        return _mamba_inner_complex(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                                    out_proj_weight, out_proj_bias, A, D, delta_bias, bool(delta_softplus))
    if not fused_path_supported(xz, conv1d_weight, x_proj_weight, delta_proj_weight, out_proj_weight,
                                A, B, C):
        raise NotImplementedError("mamba_inner_fn runs float32 tensors on a ROCm GPU")
    norms = (b_rms_weight, c_rms_weight, dt_rms_weight)
    if any(w is not None for w in norms) and not all(w is not None for w in norms):
        raise ValueError("mamba_inner_fn: b_rms_weight, c_rms_weight and dt_rms_weight go together")
    f32 = lambda t: None if t is None else t.float()  # noqa: E731
    if dt_rms_weight is None:
        return MambaInnerOpsFn.apply(xz, conv1d_weight, f32(conv1d_bias), x_proj_weight, delta_proj_weight,
                                     out_proj_weight, f32(out_proj_bias), A.float().contiguous(), f32(D),
                                     f32(delta_bias), bool(delta_softplus))
    return MambaInnerFn.apply(xz, conv1d_weight, f32(conv1d_bias), x_proj_weight, delta_proj_weight,
                              out_proj_weight, f32(out_proj_bias), A.float().contiguous(), f32(D),
                              f32(delta_bias), bool(delta_softplus), b_rms_weight, c_rms_weight,
                              dt_rms_weight, float(b_c_dt_rms_eps))

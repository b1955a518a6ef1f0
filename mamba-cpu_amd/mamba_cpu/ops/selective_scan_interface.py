"""selective_scan_fn on MI355X: torch operators over the gfx950 kernels.

Mirrors src/mamba_cpu/ops/selective_scan_interface.py of the reference:
the same public function, the same operator names and schemas
(`mamba_cpu::selective_scan_fwd` / `mamba_cpu::selective_scan_bwd`), the same
autograd wiring and the same exceptions. The operators are defined in C++
(csrc/torch_ops.cpp) over the library's C ABI, so a training step spends no
Python time below selective_scan_fn. What changes is the device (ROCm GPU
tensors instead of CPU tensors) and what the operators accept: besides the
reference's contiguous float32 inputs they take bfloat16/float16 u/delta/z and
strided views (B/C in the reference's kernel layout or transposed), so
Hugging Face's transposed projections reach the kernel without copies.
"""

from typing import Optional

import math

import torch

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

# The operators mamba_cpu::selective_scan_fwd / _bwd (the reference's schemas,
# selective_scan_interface.py:16-97) and the training pair
# mamba_cpu::selective_scan_fwd_ckpt / _bwd_ckpt are defined in C++
# (csrc/torch_ops.cpp, loaded by mamba_cpu._C) for ROCm GPU tensors, with their
# autograd formulas (the reference's :100-124) registered there too. The
# _ckpt forward also returns the float32 scan state at the start of every
# 16-step block and, when z is given, y before the z gate; its backward
# restarts from those instead of recomputing states and y. What follows are
# their shape functions for FakeTensor tracing (torch.compile, export, opcheck).

_BLOCK_T = 16


def _ckpt_shape(u, A):
    batch, dim, seqlen = u.shape
    return (batch, dim, (seqlen + _BLOCK_T - 1) // _BLOCK_T, A.shape[1])


def _like_x(x):
    """A (batch, dim, seqlen) result laid out like x, as the operators allocate
    it: channel-contiguous when x is, contiguous otherwise."""
    if x.dim() == 3 and x.stride(1) == 1 and x.stride(2) != 1:
        b, d, l = x.shape
        return torch.empty_strided((b, d, l), (d * l, 1, d), dtype=x.dtype, device=x.device)
    return x.new_empty(x.shape)


def _fwd_fake(u, A):
    return _like_x(u), u.new_empty(u.shape[0], u.shape[1], A.shape[1], dtype=torch.float32)


def _bwd_fake(u, delta, A, B, C, z):
    return (
        _like_x(u), _like_x(delta), A.new_empty(A.shape),
        B.new_empty(B.shape), C.new_empty(C.shape), A.new_empty(u.shape[1]),
        _like_x(z) if z is not None else u.new_empty(0), A.new_empty(u.shape[1]),
    )


@torch.library.register_fake("mamba_cpu::selective_scan_fwd")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    return _fwd_fake(u, A)


@torch.library.register_fake("mamba_cpu::selective_scan_bwd")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state):
    return _bwd_fake(u, delta, A, B, C, z)


@torch.library.register_fake("mamba_cpu::selective_scan_fwd_ckpt")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    out, last = _fwd_fake(u, A)
    return (out, last, u.new_empty(_ckpt_shape(u, A), dtype=torch.float32),
            u.new_empty(u.shape) if z is not None else u.new_empty(0))


@torch.library.register_fake("mamba_cpu::selective_scan_bwd_ckpt")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state, ckpt, ysave):
    return _bwd_fake(u, delta, A, B, C, z)


@torch.library.register_fake("mamba_cpu::selective_scan_cfwd")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    batch, dim, seqlen = u.shape
    nblk = (seqlen + _BLOCK_T - 1) // _BLOCK_T
    return (_like_x(u), u.new_empty(batch, dim, A.shape[1], dtype=torch.complex64),
            u.new_empty(batch, dim, nblk, A.shape[1], 2, dtype=torch.float32))


@torch.library.register_fake("mamba_cpu::selective_scan_cbwd")
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state, ckpt):
    return (
        _like_x(u), _like_x(delta), A.new_empty(A.shape), B.new_empty(B.shape), C.new_empty(C.shape),
        B.new_empty(u.shape[1]), _like_x(z) if z is not None else u.new_empty(0), B.new_empty(u.shape[1]),
    )


class _ComplexScan(torch.autograd.Function):
    """Autograd of the complex-A scan: the forward keeps its block
    checkpoints, the backward restarts from them."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, softplus):
        out, last, ckpt = torch.ops.mamba_cpu.selective_scan_cfwd(u, delta, A, B, C, D, z, delta_bias,
                                                                  softplus)
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, ckpt)
        ctx.softplus = softplus
        ctx.set_materialize_grads(False)
        return out, last

    @staticmethod
    def backward(ctx, dout, dlast):
        u, delta, A, B, C, D, z, delta_bias, ckpt = ctx.saved_tensors
        dout = torch.zeros_like(u) if dout is None else dout.to(u.dtype)
        dlast = None if dlast is None else dlast.to(torch.complex64)
        du, ddelta, dA, dB, dC, dD, dz, dbias = torch.ops.mamba_cpu.selective_scan_cbwd(
            u, delta, A, B, C, D, z, delta_bias, ctx.softplus, dout, dlast, ckpt)
        return (du, ddelta, dA, dB, dC, dD if D is not None else None, dz if z is not None else None,
                dbias if delta_bias is not None else None, None)


def _complex_kernel_bc(X: torch.Tensor, ngroups: int, batch: int, seqlen: int) -> torch.Tensor:
    """B or C of a complex-A scan as the kernels' float32 (b, ngroups, l, n, 2)
    operand, (re, im) in the unit-stride last dim. Input-dependent B/C are real
    (b, n, 2 l) or (b, g, n, 2 l) with the pairs interleaved along the last dim
    (mamba_ssm's layout): a view. A (dim, dstate) B/C, complex or real, is
    input-independent, one group per channel: a stride-0 view of
    view_as_real. Fewer groups than ngroups are repeated (a copy)."""
    if X.dim() == 2:
        Xr = torch.view_as_real(X.to(torch.complex64))
        return Xr[None, :, None].expand(batch, X.shape[0], seqlen, X.shape[1], 2)
    X = X if X.dim() == 4 else X.unsqueeze(1)
    Xk = X.float().unflatten(-1, (seqlen, 2)).transpose(2, 3)
    if Xk.stride(-1) != 1:
        Xk = Xk.contiguous()
    if Xk.shape[1] != ngroups:
        Xk = Xk.repeat_interleave(ngroups // Xk.shape[1], dim=1)
    return Xk


def _complex_scan(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state, xdt):
    """selective_scan_fn for complex A (mamba_ssm's semantics, which the
    reference rejects: selective_scan_interface.py:160-161)."""
    batch, dim, seqlen = u.shape
    for name, X in (("B", B), ("C", C)):
        if X.is_complex() or X.dim() == 2:
            if X.dim() != 2 or X.shape[0] != dim or X.shape[1] != A.shape[1]:
                raise ValueError(f"a complex {name} must be input-independent, (dim, dstate), "
                                 f"got {tuple(X.shape)}")
        elif X.dim() not in (3, 4) or X.shape[-1] != 2 * seqlen or X.shape[-2] != A.shape[1]:
            raise ValueError(f"with complex A, an input-dependent {name} is real (batch, [ngroups,] dstate, "
                             f"2 * seqlen) holding (re, im) pairs, got {tuple(X.shape)}")

    def groups(X):
        return dim if X.dim() == 2 else (1 if X.dim() == 3 else X.shape[1])

    for name, X in (("B", B), ("C", C)):
        if dim % groups(X) != 0:
            raise ValueError(f"dim ({dim}) must be divisible by {name}'s ngroups ({groups(X)})")
    ngroups = math.lcm(groups(B), groups(C))
    args = (
        _as_x(u, xdt), _as_x(delta, xdt), A.to(torch.complex64).contiguous(),
        _complex_kernel_bc(B, ngroups, batch, seqlen), _complex_kernel_bc(C, ngroups, batch, seqlen),
        _as_f32(D), _as_x(z, xdt), _as_f32(delta_bias), bool(delta_softplus),
    )
    out, last_state = _ComplexScan.apply(*args)
    out = out.to(u.dtype)
    return (out, last_state) if return_last_state else out


def _as_f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.float().contiguous()


def _as_kernel_bc(X: torch.Tensor) -> torch.Tensor:
    """(b, n, l) or (b, g, n, l) -> float32 (b, g, l, n) view. The kernels take
    any strides, so this never copies float32 input (the reference makes a
    contiguous copy, :131-135)."""
    if X.dim() == 3:
        X = X.unsqueeze(1)
    return X.float().transpose(-1, -2)


def _kernel_bc_groups(X: torch.Tensor, ngroups: int, batch: int, seqlen: int) -> torch.Tensor:
    """B or C as the kernels' float32 (b, ngroups, l, n) operand. A 2-D
    (dim, dstate) tensor is one group per channel, constant in time: a
    stride-0 view. Fewer groups than ngroups are repeated (a copy of the small
    B/C tensor); autograd sums the gradient back."""
    if X.dim() == 2:
        return X.float()[None, :, None, :].expand(batch, X.shape[0], seqlen, X.shape[1])
    Xk = _as_kernel_bc(X)
    if Xk.shape[1] != ngroups:
        Xk = Xk.repeat_interleave(ngroups // Xk.shape[1], dim=1)
    return Xk


def _as_x(t: Optional[torch.Tensor], dtype) -> Optional[torch.Tensor]:
    return None if t is None else t.to(dtype)


def selective_scan_fn(
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
    """Drop-in for mamba_ssm.ops.selective_scan_interface.selective_scan_fn on
    ROCm GPU tensors.

    u, delta, z: (batch, dim, seqlen), float32 / bfloat16 / float16
    A: (dim, dstate), real-valued, or complex; dstate up to 4096
    B, C: (batch, dstate, seqlen) or (batch, ngroups, dstate, seqlen), input-dependent,
          with their own group counts; or (dim, dstate), input-independent.
          With complex A (mamba_ssm's convention): input-dependent B/C are real
          (batch, [ngroups,] dstate, 2 * seqlen) with (re, im) pairs along the
          last dim, input-independent ones complex (dim, dstate); y = 2 Re(<h, C>) + D u
    D, delta_bias: (dim,)
    Returns out: (batch, dim, seqlen) in u's dtype [, last_state: (batch, dim, dstate) float32,
    complex64 with complex A]
    Arithmetic and the scan state are float32 for every input dtype.
    """
    if u.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {u.device}")
    batch, dim, seqlen = u.shape
    # u/delta/z keep their storage type when they share a supported one;
    # mixed or other types are computed from float32 copies.
    xdt = u.dtype
    if xdt not in _X_DTYPES or delta.dtype != xdt or (z is not None and z.dtype != xdt):
        xdt = torch.float32
    if A.is_complex():
        return _complex_scan(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state, xdt)

    def groups(X):
        return dim if X.dim() == 2 else (1 if X.dim() == 3 else X.shape[1])

    for name, X in (("B", B), ("C", C)):
        if X.dim() == 2 and X.shape[0] != dim:
            raise ValueError(f"an input-independent {name} must be (dim, dstate), got {tuple(X.shape)}")
        if dim % groups(X) != 0:
            raise ValueError(f"dim ({dim}) must be divisible by {name}'s ngroups ({groups(X)})")
    # The kernels take one group count for B and C. Unequal counts (and 2-D,
    # input-independent B/C, which are one group per channel) run at their
    # least common multiple; the reference rejects both (:160-170).
    ngroups = math.lcm(groups(B), groups(C))
    args = (
        _as_x(u, xdt), _as_x(delta, xdt), _as_f32(A), _kernel_bc_groups(B, ngroups, batch, seqlen),
        _kernel_bc_groups(C, ngroups, batch, seqlen), _as_f32(D), _as_x(z, xdt), _as_f32(delta_bias),
        bool(delta_softplus),
    )
    needs_grad = torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in args)
    if needs_grad:
        out, last_state, _, _ = torch.ops.mamba_cpu.selective_scan_fwd_ckpt(*args)
    else:
        out, last_state = torch.ops.mamba_cpu.selective_scan_fwd(*args)
    out = out.to(u.dtype)
    return (out, last_state) if return_last_state else out

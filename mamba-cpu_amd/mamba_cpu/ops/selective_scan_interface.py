"""selective_scan_fn on MI355X: torch.library custom ops over the gfx950 kernels.

Mirrors src/mamba_cpu/ops/selective_scan_interface.py of the reference:
the same public function, the same custom-op names and schemas
(`mamba_cpu::selective_scan_fwd` / `mamba_cpu::selective_scan_bwd`), the same
autograd wiring and the same exceptions. What changes is the device (ROCm GPU
tensors instead of CPU tensors) and what the ops accept: besides the
reference's contiguous float32 inputs they take bfloat16/float16 u/delta/z and
strided views (B/C in the reference's kernel layout or transposed), so
Hugging Face's transposed projections reach the kernel without copies.
"""

from typing import Optional

import torch

from mamba_cpu import _C

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _validate(name, u, delta, A, B, C, D, z, delta_bias, extra=()):
    """Rejects what the kernels cannot take, with the reference's exception
    type (ValueError, selective_scan_interface.py:28-30)."""
    for t in (u, delta, A, B, C, D, z, delta_bias, *extra):
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{name} runs on ROCm GPU tensors, got a tensor on {t.device}")
    if u.dtype not in _X_DTYPES or delta.dtype != u.dtype or (z is not None and z.dtype != u.dtype):
        raise ValueError(f"{name} expects u, delta and z of one dtype among float32, bfloat16 "
                         f"and float16, got {u.dtype}, {delta.dtype}, {None if z is None else z.dtype}")
    for t in (A, B, C, D, delta_bias):
        if t is not None and t.dtype != torch.float32:
            raise ValueError(f"{name} expects float32 A, B, C, D and delta_bias")
    if u.dim() != 3 or delta.shape != u.shape or (z is not None and z.shape != u.shape):
        raise ValueError(f"{name} expects u, delta and z of shape (batch, dim, seqlen)")
    batch, dim, seqlen = u.shape
    if A.dim() != 2 or A.shape[0] != dim:
        raise ValueError(f"{name} expects A of shape (dim, dstate)")
    dstate = A.shape[1]
    for X in (B, C):
        if X.dim() != 4 or X.shape[0] != batch or X.shape[2] != seqlen or X.shape[3] != dstate:
            raise ValueError(f"{name} expects B and C of shape (batch, ngroups, seqlen, dstate)")
    if B.shape[1] != C.shape[1] or dim % B.shape[1] != 0:
        raise ValueError(f"{name}: dim ({dim}) must be divisible by ngroups ({B.shape[1]})")
    for t in (D, delta_bias):
        if t is not None and (t.shape != (dim,) or not t.is_contiguous()):
            raise ValueError(f"{name} expects contiguous D and delta_bias of shape (dim,)")
    if not A.is_contiguous():
        raise ValueError(f"{name} expects a contiguous A")


def _scan_args(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    a = _C.ScanArgs()
    batch, dim, seqlen = u.shape
    a.u, a.delta, a.A = u.data_ptr(), delta.data_ptr(), A.data_ptr()
    a.B, a.C = B.data_ptr(), C.data_ptr()
    a.D, a.z, a.delta_bias = _C.ptr(D), _C.ptr(z), _C.ptr(delta_bias)
    a.batch, a.dim, a.seqlen = batch, dim, seqlen
    a.dstate, a.ngroups = A.shape[1], B.shape[1]
    a.delta_softplus = int(bool(delta_softplus))
    a.dtype = _C.DTYPES[u.dtype]
    a.u_stride = _C.strides3(u)
    a.delta_stride = _C.strides3(delta)
    a.z_stride = _C.strides3(z)
    a.B_stride = tuple(B.stride())
    a.C_stride = tuple(C.stride())
    return a


@torch.library.custom_op("mamba_cpu::selective_scan_fwd", mutates_args=(), device_types="cuda")
def _selective_scan_fwd(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    delta_softplus: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (out in u's dtype, last_state float32 (batch, dim, dstate))."""
    _validate("mamba_cpu::selective_scan_fwd", u, delta, A, B, C, D, z, delta_bias)
    batch, dim, _ = u.shape
    out = u.new_empty(u.shape)
    last_state = u.new_empty(batch, dim, A.shape[1], dtype=torch.float32)
    a = _scan_args(u, delta, A, B, C, D, z, delta_bias, delta_softplus)
    a.out, a.last_state = out.data_ptr(), last_state.data_ptr()
    with _C.device_of(u):
        _C.call(_C.lib.mcpu_selective_scan_fwd, a, "mamba_cpu::selective_scan_fwd", _C.stream_of(u))
    return out, last_state


@_selective_scan_fwd.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    return u.new_empty(u.shape), u.new_empty(u.shape[0], u.shape[1], A.shape[1], dtype=torch.float32)


def _scan_bwd_impl(name, u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state,
                   ckpt=None, ysave=None):
    _validate(name, u, delta, A, B, C, D, z, delta_bias, extra=(dout, dlast_state, ckpt, ysave))
    if dout.shape != u.shape or dout.dtype != u.dtype:
        raise ValueError(f"{name} expects dout shaped and typed like u")
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    if dlast_state is not None:
        if dlast_state.dtype != torch.float32 or dlast_state.shape != (batch, dim, dstate):
            raise ValueError(f"{name} expects float32 dlast_state (batch, dim, dstate)")
        dlast_state = dlast_state.contiguous()
    if ckpt is not None and (ckpt.dtype != torch.float32 or not ckpt.is_contiguous()
                             or ckpt.shape != _ckpt_shape(u, A)):
        raise ValueError(f"{name} expects the float32 checkpoints written by selective_scan_fwd_ckpt")
    if ysave is not None and ysave.numel() == 0:
        ysave = None
    if ysave is not None and (ysave.shape != u.shape or ysave.dtype != u.dtype
                              or not ysave.is_contiguous() or z is None):
        raise ValueError(f"{name} expects the y written by selective_scan_fwd_ckpt")
    du = u.new_empty(u.shape)
    ddelta = delta.new_empty(delta.shape)
    dA = A.new_empty(A.shape)
    dB = B.new_empty(B.shape)
    dC = C.new_empty(C.shape)
    dD = A.new_empty(dim)
    dz = z.new_empty(z.shape) if z is not None else u.new_empty(0)
    ddelta_bias = A.new_empty(dim)
    a = _scan_args(u, delta, A, B, C, D, z, delta_bias, delta_softplus)
    a.dout, a.dout_stride = dout.data_ptr(), _C.strides3(dout)
    a.dlast_state = _C.ptr(dlast_state)
    a.ckpt = _C.ptr(ckpt)
    a.ysave = _C.ptr(ysave)
    a.du, a.ddelta, a.dA, a.dB, a.dC = (du.data_ptr(), ddelta.data_ptr(), dA.data_ptr(),
                                        dB.data_ptr(), dC.data_ptr())
    a.dD, a.ddelta_bias = dD.data_ptr(), ddelta_bias.data_ptr()
    a.dz = dz.data_ptr() if z is not None else 0
    with _C.device_of(u):
        ws_bytes = _C.lib.mcpu_selective_scan_bwd_workspace_size(a)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=u.device)
        _C.call(_C.lib.mcpu_selective_scan_bwd, a, name, ws.data_ptr(), ws_bytes, _C.stream_of(u))
    return du, ddelta, dA, dB, dC, dD, dz, ddelta_bias


def _bwd_fake(u, delta, A, B, C, z):
    dim = u.shape[1]
    return (
        u.new_empty(u.shape), delta.new_empty(delta.shape), A.new_empty(A.shape),
        B.new_empty(B.shape), C.new_empty(C.shape), A.new_empty(dim),
        z.new_empty(z.shape) if z is not None else u.new_empty(0), A.new_empty(dim),
    )


@torch.library.custom_op("mamba_cpu::selective_scan_bwd", mutates_args=(), device_types="cuda")
def _selective_scan_bwd(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    delta_softplus: bool,
    dout: torch.Tensor,
    dlast_state: Optional[torch.Tensor],
) -> tuple[
    torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
    torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
]:
    """Returns (du, ddelta, dA, dB, dC, dD, dz, ddelta_bias). dz is empty when z
    is None; dD and ddelta_bias are always computed (as in the reference).
    Recomputes the forward states it needs from the inputs."""
    return _scan_bwd_impl("mamba_cpu::selective_scan_bwd", u, delta, A, B, C, D, z, delta_bias,
                          delta_softplus, dout, dlast_state)


@_selective_scan_bwd.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state):
    return _bwd_fake(u, delta, A, B, C, z)


def _setup_context(ctx, inputs, output):
    u, delta, A, B, C, D, z, delta_bias, delta_softplus = inputs
    ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias)
    ctx.delta_softplus = delta_softplus
    ctx.set_materialize_grads(False)


def _backward(ctx, grad_out, grad_last_state):
    u, delta, A, B, C, D, z, delta_bias = ctx.saved_tensors
    dout = torch.zeros_like(u) if grad_out is None else grad_out.to(u.dtype)
    dlast = None if grad_last_state is None else grad_last_state.float().contiguous()
    du, ddelta, dA, dB, dC, dD, dz, ddelta_bias = torch.ops.mamba_cpu.selective_scan_bwd(
        u, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, dout, dlast
    )
    return (
        du, ddelta, dA, dB, dC,
        dD if D is not None else None,
        dz if z is not None else None,
        ddelta_bias if delta_bias is not None else None,
        None,
    )


torch.library.register_autograd(
    "mamba_cpu::selective_scan_fwd", _backward, setup_context=_setup_context
)


# Training path: the forward also returns the scan state at the start of every
# 16-step block and, when z is given, y before the z gate; the backward
# restarts from those checkpoints and reads y instead of recomputing the
# states and y from the inputs. Same arithmetic as the pair above.

_BLOCK_T = 16


def _ckpt_shape(u, A):
    batch, dim, seqlen = u.shape
    return (batch, dim, (seqlen + _BLOCK_T - 1) // _BLOCK_T, A.shape[1])


@torch.library.custom_op("mamba_cpu::selective_scan_fwd_ckpt", mutates_args=(), device_types="cuda")
def _selective_scan_fwd_ckpt(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    delta_softplus: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """selective_scan_fwd that also returns the float32 block checkpoints
    (batch, dim, ceil(seqlen / 16), dstate) and y before the z gate (u's
    dtype and shape; empty when z is None) for selective_scan_bwd_ckpt."""
    name = "mamba_cpu::selective_scan_fwd_ckpt"
    _validate(name, u, delta, A, B, C, D, z, delta_bias)
    batch, dim, _ = u.shape
    out = u.new_empty(u.shape)
    last_state = u.new_empty(batch, dim, A.shape[1], dtype=torch.float32)
    ckpt = u.new_empty(_ckpt_shape(u, A), dtype=torch.float32)
    ysave = u.new_empty(u.shape) if z is not None else u.new_empty(0)
    a = _scan_args(u, delta, A, B, C, D, z, delta_bias, delta_softplus)
    a.out, a.last_state, a.ckpt = out.data_ptr(), last_state.data_ptr(), ckpt.data_ptr()
    a.ysave = ysave.data_ptr() if z is not None else 0
    with _C.device_of(u):
        _C.call(_C.lib.mcpu_selective_scan_fwd, a, name, _C.stream_of(u))
    return out, last_state, ckpt, ysave


@_selective_scan_fwd_ckpt.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus):
    return (u.new_empty(u.shape), u.new_empty(u.shape[0], u.shape[1], A.shape[1], dtype=torch.float32),
            u.new_empty(_ckpt_shape(u, A), dtype=torch.float32),
            u.new_empty(u.shape) if z is not None else u.new_empty(0))


@torch.library.custom_op("mamba_cpu::selective_scan_bwd_ckpt", mutates_args=(), device_types="cuda")
def _selective_scan_bwd_ckpt(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    delta_bias: Optional[torch.Tensor],
    delta_softplus: bool,
    dout: torch.Tensor,
    dlast_state: Optional[torch.Tensor],
    ckpt: torch.Tensor,
    ysave: torch.Tensor,
) -> tuple[
    torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
    torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
]:
    """selective_scan_bwd restarting from the forward's block checkpoints and
    saved y (pass an empty ysave to recompute y)."""
    return _scan_bwd_impl("mamba_cpu::selective_scan_bwd_ckpt", u, delta, A, B, C, D, z, delta_bias,
                          delta_softplus, dout, dlast_state, ckpt, ysave)


@_selective_scan_bwd_ckpt.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, delta_softplus, dout, dlast_state, ckpt, ysave):
    return _bwd_fake(u, delta, A, B, C, z)


def _setup_context_ckpt(ctx, inputs, output):
    u, delta, A, B, C, D, z, delta_bias, delta_softplus = inputs
    ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, output[2], output[3])
    ctx.delta_softplus = delta_softplus
    ctx.set_materialize_grads(False)


def _tracing(*tensors):
    """True under torch.compile / export / make_fx tracing (fake or
    functional tensors, or an active dispatch mode), where the backward must
    call the custom op rather than its body."""
    return (torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0
            or any(type(t) is not torch.Tensor for t in tensors))


def _backward_ckpt(ctx, grad_out, grad_last_state, grad_ckpt, grad_ysave):
    u, delta, A, B, C, D, z, delta_bias, ckpt, ysave = ctx.saved_tensors
    dout = torch.zeros_like(u) if grad_out is None else grad_out.to(u.dtype)
    dlast = None if grad_last_state is None else grad_last_state.float().contiguous()
    args = (u, delta, A, B, C, D, z, delta_bias, ctx.delta_softplus, dout, dlast, ckpt, ysave)
    if _tracing(u, dout):
        grads = torch.ops.mamba_cpu.selective_scan_bwd_ckpt(*args)
    else:
        # Eager: the op's body directly, without a second trip through the
        # dispatcher (the backward runs once per training step; this keeps its
        # host cost below the kernels' time).
        grads = _scan_bwd_impl("mamba_cpu::selective_scan_bwd_ckpt", *args)
    du, ddelta, dA, dB, dC, dD, dz, ddelta_bias = grads
    return (
        du, ddelta, dA, dB, dC,
        dD if D is not None else None,
        dz if z is not None else None,
        ddelta_bias if delta_bias is not None else None,
        None,
    )


torch.library.register_autograd(
    "mamba_cpu::selective_scan_fwd_ckpt", _backward_ckpt, setup_context=_setup_context_ckpt
)


def _as_f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.float().contiguous()


def _as_kernel_bc(X: torch.Tensor) -> torch.Tensor:
    """(b, n, l) or (b, g, n, l) -> float32 (b, g, l, n) view. The kernels take
    any strides, so this never copies float32 input (the reference makes a
    contiguous copy, :131-135)."""
    if X.dim() == 3:
        X = X.unsqueeze(1)
    return X.float().transpose(-1, -2)


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
    A: (dim, dstate), real-valued
    B, C: (batch, dstate, seqlen) or (batch, ngroups, dstate, seqlen)
    D, delta_bias: (dim,)
    Returns out: (batch, dim, seqlen) in u's dtype [, last_state: (batch, dim, dstate) float32]
    Arithmetic and the scan state are float32 for every input dtype.
    """
    if u.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {u.device}")
    if A.is_complex():
        raise NotImplementedError("complex A is not supported yet")
    if B.dim() < 3 or C.dim() < 3:
        raise NotImplementedError("input-independent (2D) B/C is not supported yet")
    dim = u.shape[1]
    for name, X in (("B", B), ("C", C)):
        ngroups = 1 if X.dim() == 3 else X.shape[1]
        if dim % ngroups != 0:
            raise ValueError(f"dim ({dim}) must be divisible by {name}'s ngroups ({ngroups})")
    if B.dim() != C.dim() or (B.dim() == 4 and B.shape[1] != C.shape[1]):
        raise NotImplementedError("B and C must have the same number of groups")

    # u/delta/z keep their storage type when they share a supported one;
    # mixed or other types are computed from float32 copies.
    xdt = u.dtype
    if xdt not in _X_DTYPES or delta.dtype != xdt or (z is not None and z.dtype != xdt):
        xdt = torch.float32
    args = (
        _as_x(u, xdt), _as_x(delta, xdt), _as_f32(A), _as_kernel_bc(B), _as_kernel_bc(C),
        _as_f32(D), _as_x(z, xdt), _as_f32(delta_bias), bool(delta_softplus),
    )
    needs_grad = torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in args)
    if needs_grad:
        out, last_state, _, _ = torch.ops.mamba_cpu.selective_scan_fwd_ckpt(*args)
    else:
        out, last_state = torch.ops.mamba_cpu.selective_scan_fwd(*args)
    out = out.to(u.dtype)
    return (out, last_state) if return_last_state else out

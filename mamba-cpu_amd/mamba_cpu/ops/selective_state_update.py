"""selective_state_update on MI355X: one decode step of the selective scan.

Same signature and behaviour as src/mamba_cpu/ops/selective_state_update.py
of the reference (Mamba-1 and Mamba-2 head layouts, state updated in place,
output in x's dtype), as the in-place custom op
`mamba_cpu::selective_state_update` over the gfx950 kernel.
"""

from typing import Optional

import torch

from mamba_cpu import _C

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


@torch.library.custom_op("mamba_cpu::selective_state_update", mutates_args=("state",),
                         device_types="cuda")
def _selective_state_update(
    state: torch.Tensor,
    x: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    D: Optional[torch.Tensor],
    z: Optional[torch.Tensor],
    dt_bias: Optional[torch.Tensor],
    dt_softplus: bool,
) -> torch.Tensor:
    """Head layout only: state (b, h, p, n); x/dt/z (b, h, p); A (h, p, n)
    float32 contiguous; B/C (b, g, n) float32 with unit dstate stride;
    D/dt_bias (h, p) float32 contiguous. Returns out (b, h, p) in x's dtype."""
    name = "mamba_cpu::selective_state_update"
    for t in (state, x, dt, A, B, C, D, z, dt_bias):
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{name} runs on ROCm GPU tensors, got a tensor on {t.device}")
    if x.dtype not in _X_DTYPES or dt.dtype != x.dtype or (z is not None and z.dtype != x.dtype):
        raise ValueError(f"{name} expects x, dt and z of one dtype among float32, bfloat16, float16")
    if state.dtype not in _X_DTYPES:
        raise ValueError(f"{name} expects a float32, bfloat16 or float16 state")
    if state.dim() != 4 or x.dim() != 3:
        raise ValueError(f"{name} expects state (b, h, p, n) and x (b, h, p)")
    b, h, p, n = state.shape
    if state.stride(3) != 1 and n > 1:
        raise ValueError(f"{name} expects unit stride along dstate")
    for t in (A, B, C, D, dt_bias):
        if t is not None and t.dtype != torch.float32:
            raise ValueError(f"{name} expects float32 A, B, C, D and dt_bias")
    if A.shape != (h, p, n) or not A.is_contiguous():
        raise ValueError(f"{name} expects a contiguous A of shape (nheads, headdim, dstate)")
    g = B.shape[1]
    for X in (B, C):
        if X.dim() != 3 or X.shape != (b, g, n) or (X.stride(2) != 1 and n > 1):
            raise ValueError(f"{name} expects B and C of shape (batch, ngroups, dstate), unit dstate stride")
    for t in (D, dt_bias):
        if t is not None and (t.shape != (h, p) or not t.is_contiguous()):
            raise ValueError(f"{name} expects contiguous D and dt_bias of shape (nheads, headdim)")
    out = x.new_empty(b, h, p)
    a = _C.StateUpdateArgs()
    a.state, a.x, a.dt, a.A = state.data_ptr(), x.data_ptr(), dt.data_ptr(), A.data_ptr()
    a.B, a.C, a.D, a.z, a.dt_bias = B.data_ptr(), C.data_ptr(), _C.ptr(D), _C.ptr(z), _C.ptr(dt_bias)
    a.out = out.data_ptr()
    a.batch, a.nheads, a.headdim, a.dstate, a.ngroups = b, h, p, n, g
    a.dt_softplus = int(bool(dt_softplus))
    a.dtype, a.state_dtype = _C.DTYPES[x.dtype], _C.DTYPES[state.dtype]
    a.state_stride = tuple(state.stride()[:3])
    a.x_stride, a.dt_stride, a.z_stride = _C.strides3(x), _C.strides3(dt), _C.strides3(z)
    a.B_stride = (B.stride(0), B.stride(1))
    a.C_stride = (C.stride(0), C.stride(1))
    with _C.device_of(x):
        _C.call(_C.lib.mcpu_selective_state_update, a, name, _C.stream_of(x))
    return out


@_selective_state_update.register_fake
def _(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus):
    return x.new_empty(state.shape[:3])


def selective_state_update(
    state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False, state_batch_indices=None
):
    """Single decode step of the selective scan. Updates state in place.

    Mamba-1 shapes:
        state: (batch, dim, dstate)
        x, dt, z: (batch, dim)
        A: (dim, dstate)
        B, C: (batch, dstate)
        D, dt_bias: (dim,)
    Mamba-2 (multi-head) shapes:
        state: (batch, nheads, headdim, dstate)
        x, dt, z: (batch, nheads, headdim)
        A: (nheads, headdim, dstate)
        B, C: (batch, ngroups, dstate)
        D, dt_bias: (nheads, headdim)
    Returns out shaped like x.
    """
    if state_batch_indices is not None:
        raise NotImplementedError("state_batch_indices is not supported yet")
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    has_heads = state.dim() > 3
    if not has_heads:
        # Mamba-1 is the head layout with one head of headdim = dim.
        state = state.unsqueeze(1)
        x = x.unsqueeze(1)
        dt = dt.unsqueeze(1)
        A = A.unsqueeze(0)
        B = B.unsqueeze(1)
        C = C.unsqueeze(1)
        D = None if D is None else D.unsqueeze(0)
        z = None if z is None else z.unsqueeze(1)
        dt_bias = None if dt_bias is None else dt_bias.unsqueeze(0)
    in_dtype = x.dtype
    xdt = in_dtype
    if xdt not in _X_DTYPES or dt.dtype != xdt or (z is not None and z.dtype != xdt):
        xdt = torch.float32

    def f32(t):
        return None if t is None else t.float().contiguous()

    def bc(t):
        t = t.float()
        return t if (t.stride(-1) == 1 or t.shape[-1] == 1) else t.contiguous()

    st = state
    if st.dtype not in _X_DTYPES or (st.stride(-1) != 1 and st.shape[-1] > 1):
        st = state.float().contiguous()
    out = torch.ops.mamba_cpu.selective_state_update(
        st, x.to(xdt), dt.to(xdt), f32(A), bc(B), bc(C), f32(D),
        None if z is None else z.to(xdt), f32(dt_bias), bool(dt_softplus),
    )
    if st is not state:
        state.copy_(st)
    out = out.to(in_dtype)
    return out if has_heads else out.squeeze(1)

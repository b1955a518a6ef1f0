"""selective_state_update on MI355X: one decode step of the selective scan.

Same signature and behaviour as src/mamba_cpu/ops/selective_state_update.py
of the reference (Mamba-1 and Mamba-2 head layouts, state updated in place,
output in x's dtype), as the in-place operator
`mamba_cpu::selective_state_update` (C++, csrc/torch_ops.cpp) over the gfx950
kernel.
"""

import torch

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


# mamba_cpu::selective_state_update (in place on `state`, Mamba-2 head layout:
# state (b, h, p, n); x/dt/z (b, h, p); A (h, p, n); B/C (b, g, n); D/dt_bias
# (h, p)) is defined in C++ (csrc/torch_ops.cpp, loaded by mamba_cpu._C); this
# is its shape function for FakeTensor tracing.


@torch.library.register_fake("mamba_cpu::selective_state_update")
def _(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus, state_batch_indices=None):
    return x.new_empty(x.shape)


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
    state_batch_indices: optional (batch,) int; batch row b then updates
        state[state_batch_indices[b]] (state may have more rows than the batch;
        rows whose index is out of range are skipped and get a zero output).
        Indices must be distinct. mamba_ssm's semantics; the reference raises
        NotImplementedError for it (ops/selective_state_update.py:24-25).
    Returns out shaped like x.
    """
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
    idx = None
    if state_batch_indices is not None:
        if (state_batch_indices.dtype not in (torch.int32, torch.int64)
                or state_batch_indices.shape != (x.shape[0],)):
            raise ValueError(f"state_batch_indices must be an integer tensor of shape ({x.shape[0]},)")
        idx = state_batch_indices.to(device=x.device, dtype=torch.int32).contiguous()
    out = torch.ops.mamba_cpu.selective_state_update(
        st, x.to(xdt), dt.to(xdt), f32(A), bc(B), bc(C), f32(D),
        None if z is None else z.to(xdt), f32(dt_bias), bool(dt_softplus), idx,
    )
    if st is not state:
        state.copy_(st)
    out = out.to(in_dtype)
    return out if has_heads else out.squeeze(1)

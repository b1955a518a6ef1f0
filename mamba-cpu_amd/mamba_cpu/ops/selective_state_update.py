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
    idx = None
    if state_batch_indices is not None:
        if (state_batch_indices.dtype not in (torch.int32, torch.int64)
                or state_batch_indices.shape != (x.shape[0],)):
            raise ValueError(f"state_batch_indices must be an integer tensor of shape ({x.shape[0]},)")
        idx = state_batch_indices.to(device=x.device, dtype=torch.int32).contiguous()
    xdt = x.dtype
    if (xdt in _X_DTYPES and dt.dtype == xdt and (z is None or z.dtype == xdt)
            and state.dtype in _X_DTYPES and (state.stride(-1) == 1 or state.shape[-1] == 1)):
        # The operator takes both layouts as they are and casts the float32
        # parameters itself: the common decode call is one dispatch.
        return torch.ops.mamba_cpu.selective_state_update(
            state, x, dt, A, B, C, D, z, dt_bias, bool(dt_softplus), idx)
    # Mixed or other dtypes: computed in float32, state written back.
    if xdt not in _X_DTYPES or dt.dtype != xdt or (z is not None and z.dtype != xdt):
        xdt = torch.float32
    st = state
    if state.dtype not in _X_DTYPES or (state.stride(-1) != 1 and state.shape[-1] > 1):
        st = state.float().contiguous()
    out = torch.ops.mamba_cpu.selective_state_update(
        st, x.to(xdt), dt.to(xdt), A, B, C, D, None if z is None else z.to(xdt), dt_bias,
        bool(dt_softplus), idx)
    if st is not state:
        state.copy_(st)
    return out.to(x.dtype)

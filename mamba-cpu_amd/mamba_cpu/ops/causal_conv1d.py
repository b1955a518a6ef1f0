"""causal_conv1d_fn / causal_conv1d_update on MI355X.

Same signatures and behaviour as src/mamba_cpu/ops/causal_conv1d.py of the
reference, which wraps F.conv1d; here both are torch operators over the gfx950
kernels (`mamba_cpu::causal_conv1d_fwd` with autograd through
`mamba_cpu::causal_conv1d_bwd`, and the in-place `mamba_cpu::causal_conv1d_update`),
defined in C++ (csrc/torch_ops.cpp). Arithmetic is float32; outputs are in
x's dtype.
"""

import torch

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _silu_flag(activation):
    """causal_conv1d.py:8-13: None, 'silu' or 'swish'."""
    if activation is None:
        return False
    if activation in ("silu", "swish"):
        return True
    raise ValueError(f"activation must be None, 'silu' or 'swish', got {activation!r}")


def _like_x(x):
    """Output buffer with x's layout when x is channel-contiguous (the
    transposed views Hugging Face passes), contiguous otherwise."""
    if x.dim() == 3 and x.stride(1) == 1 and x.stride(2) != 1:
        b, d, l = x.shape
        return torch.empty_strided((b, d, l), (d * l, 1, d), dtype=x.dtype, device=x.device)
    return x.new_empty(x.shape)


# mamba_cpu::causal_conv1d_fwd (autograd through mamba_cpu::causal_conv1d_bwd)
# and the in-place mamba_cpu::causal_conv1d_update are defined in C++
# (csrc/torch_ops.cpp, loaded by mamba_cpu._C); these are their shape
# functions for FakeTensor tracing.


@torch.library.register_fake("mamba_cpu::causal_conv1d_fwd")
def _(x, weight, bias, initial_states, return_final_states, silu, seq_idx=None):
    b, d, _ = x.shape
    final = x.new_empty(b, d, weight.shape[1] - 1) if return_final_states else x.new_empty(0)
    return _like_x(x), final


@torch.library.register_fake("mamba_cpu::causal_conv1d_bwd")
def _(x, weight, bias, initial_states, dout, dfinal_states, silu, seq_idx=None):
    b, d, _ = x.shape
    return (
        _like_x(x), weight.new_empty(weight.shape),
        weight.new_empty(d) if bias is not None else weight.new_empty(0),
        x.new_empty(b, d, weight.shape[1] - 1) if initial_states is not None else x.new_empty(0),
    )


@torch.library.register_fake("mamba_cpu::causal_conv1d_update")
def _(x, conv_state, weight, bias, silu, cache_seqlens=None, conv_state_indices=None):
    return x.new_empty(x.shape)


def _index(t, name, batch, device):
    """An optional (batch,) integer vector as the int32 the kernels read."""
    if t is None:
        return None
    if t.dtype not in (torch.int32, torch.int64) or t.dim() != 1 or t.shape[0] != batch:
        raise ValueError(f"{name} must be an integer tensor of shape ({batch},)")
    return t.to(device=device, dtype=torch.int32).contiguous()


def causal_conv1d_fn(
    x,
    weight,
    bias=None,
    seq_idx=None,
    initial_states=None,
    return_final_states=False,
    final_states_out=None,
    activation=None,
):
    """
    x: (batch, dim, seqlen)
    weight: (dim, width)
    bias: (dim,)
    seq_idx: optional (batch, seqlen) int: packed sequences; a tap reading an
        input of another sequence counts as zero (the upstream causal_conv1d
        package's semantics; the reference raises NotImplementedError,
        ops/causal_conv1d.py:34-35). Excludes initial_states and final states.
    initial_states: (batch, dim, width - 1)
    final_states_out: optional (batch, dim, width - 1) buffer for the final states
    Returns out: (batch, dim, seqlen) in x's dtype [, final_states: (batch, dim, width - 1)]
    """
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    silu = _silu_flag(activation)
    in_dtype = x.dtype
    if in_dtype not in _X_DTYPES:
        x = x.float()
    init = None if initial_states is None else initial_states.to(x.dtype)
    if seq_idx is not None:
        if initial_states is not None or return_final_states:
            raise ValueError("seq_idx cannot be combined with initial_states or return_final_states")
        if seq_idx.dtype not in (torch.int32, torch.int64) or seq_idx.shape != (x.shape[0], x.shape[2]):
            raise ValueError(f"seq_idx must be an integer tensor of shape ({x.shape[0]}, {x.shape[2]})")
        seq_idx = seq_idx.to(device=x.device, dtype=torch.int32).contiguous()
    out, final = torch.ops.mamba_cpu.causal_conv1d_fwd(
        x, weight.float().contiguous(), None if bias is None else bias.float().contiguous(), init,
        bool(return_final_states), silu, seq_idx,
    )
    out = out.to(in_dtype)
    if not return_final_states:
        return out
    final = final.to(in_dtype)
    if final_states_out is not None:
        final = final_states_out.copy_(final)
    return out, final


def causal_conv1d_update(
    x, conv_state, weight, bias=None, activation=None, cache_seqlens=None, conv_state_indices=None
):
    """Decode step(s). Updates conv_state in place.

    x: (batch, dim) or (batch, dim, seqlen)
    conv_state: (batch, dim, state_len), state_len >= width - 1
    weight: (dim, width)
    cache_seqlens: optional (batch,) int; conv_state is then a ring buffer
        (the upstream causal_conv1d package's semantics): the width - 1 inputs
        before x are at (cache_seqlens - (width - 1) + k) % state_len and x is
        written from cache_seqlens % state_len on.
    conv_state_indices: optional (batch,) int; batch row b then uses
        conv_state[conv_state_indices[b]] (conv_state may have more rows than
        the batch; rows whose index is out of range are skipped and get a zero
        output). Indices must be distinct.
    Returns out shaped like x.

    The reference raises NotImplementedError for the last two
    (ops/causal_conv1d.py:66-67); they serve continuous batching.
    """
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    silu = _silu_flag(activation)
    width = weight.shape[1]
    state_len = conv_state.shape[-1]
    if state_len < width - 1:
        raise ValueError(f"conv_state length ({state_len}) must be at least width - 1 ({width - 1})")
    batch = x.shape[0]
    cs = _index(cache_seqlens, "cache_seqlens", batch, x.device)
    idx = _index(conv_state_indices, "conv_state_indices", batch, x.device)
    if x.dtype in _X_DTYPES and conv_state.dtype == x.dtype:
        # The operator takes (b, dim) or (b, dim, seqlen) as they are: one dispatch.
        return torch.ops.mamba_cpu.causal_conv1d_update(x, conv_state, weight, bias, silu, cs, idx)
    # Mixed or other dtypes: the reference mixes them through conv_state.to(x.dtype)
    # and a copy back; unsupported x dtypes are computed in float32.
    xw = x if x.dtype in _X_DTYPES else x.float()
    tmp = conv_state.to(xw.dtype)
    out = torch.ops.mamba_cpu.causal_conv1d_update(xw, tmp, weight, bias, silu, cs, idx)
    conv_state.copy_(tmp)
    return out.to(x.dtype)

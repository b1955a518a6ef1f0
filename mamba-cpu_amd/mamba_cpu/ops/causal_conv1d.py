"""causal_conv1d_fn / causal_conv1d_update on MI355X.

Same signatures and behaviour as src/mamba_cpu/ops/causal_conv1d.py of the
reference, which wraps F.conv1d; here both are torch.library custom ops over
the gfx950 kernels (`mamba_cpu::causal_conv1d_fwd` with autograd through
`mamba_cpu::causal_conv1d_bwd`, and the in-place `mamba_cpu::causal_conv1d_update`).
Arithmetic is float32; outputs are in x's dtype.
"""

from typing import Optional

import torch

from mamba_cpu import _C

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


def _check(name, x, weight, bias, initial_states):
    for t in (x, weight, bias, initial_states):
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{name} runs on ROCm GPU tensors, got a tensor on {t.device}")
    if x.dtype not in _X_DTYPES:
        raise ValueError(f"{name} expects x in float32, bfloat16 or float16, got {x.dtype}")
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError(f"{name} expects x (batch, dim, seqlen) and weight (dim, width)")
    if weight.dtype != torch.float32 or not weight.is_contiguous():
        raise ValueError(f"{name} expects a contiguous float32 weight")
    if bias is not None and (bias.dtype != torch.float32 or bias.shape != (x.shape[1],)):
        raise ValueError(f"{name} expects a float32 bias of shape (dim,)")
    if initial_states is not None and (
        initial_states.dtype != x.dtype
        or initial_states.shape != (x.shape[0], x.shape[1], weight.shape[1] - 1)
    ):
        raise ValueError(f"{name} expects initial_states (batch, dim, width - 1) in x's dtype")


def _conv_args(x, weight, bias, initial_states, silu):
    a = _C.ConvArgs()
    a.x, a.weight, a.bias = x.data_ptr(), weight.data_ptr(), _C.ptr(bias)
    a.initial_states = _C.ptr(initial_states)
    a.batch, a.dim, a.seqlen = x.shape
    a.width = weight.shape[1]
    a.silu = int(bool(silu))
    a.dtype = _C.DTYPES[x.dtype]
    a.x_stride = _C.strides3(x)
    a.init_stride = _C.strides3(initial_states)
    return a


@torch.library.custom_op("mamba_cpu::causal_conv1d_fwd", mutates_args=(), device_types="cuda")
def _causal_conv1d_fwd(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    initial_states: Optional[torch.Tensor],
    return_final_states: bool,
    silu: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (out, final_states); final_states is empty unless requested."""
    _check("mamba_cpu::causal_conv1d_fwd", x, weight, bias, initial_states)
    out = _like_x(x)
    b, d, _ = x.shape
    width = weight.shape[1]
    final = x.new_empty(b, d, width - 1) if return_final_states else x.new_empty(0)
    a = _conv_args(x, weight, bias, initial_states, silu)
    a.out, a.out_stride = out.data_ptr(), _C.strides3(out)
    a.final_states = final.data_ptr() if return_final_states else 0
    with _C.device_of(x):
        _C.call(_C.lib.mcpu_causal_conv1d_fwd, a, "mamba_cpu::causal_conv1d_fwd", _C.stream_of(x))
    return out, final


@_causal_conv1d_fwd.register_fake
def _(x, weight, bias, initial_states, return_final_states, silu):
    b, d, _ = x.shape
    final = x.new_empty(b, d, weight.shape[1] - 1) if return_final_states else x.new_empty(0)
    return _like_x(x), final


@torch.library.custom_op("mamba_cpu::causal_conv1d_bwd", mutates_args=(), device_types="cuda")
def _causal_conv1d_bwd(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    initial_states: Optional[torch.Tensor],
    dout: torch.Tensor,
    dfinal_states: Optional[torch.Tensor],
    silu: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (dx, dweight, dbias, dinitial_states); dbias / dinitial_states
    are empty when bias / initial_states are None."""
    _check("mamba_cpu::causal_conv1d_bwd", x, weight, bias, initial_states)
    if dout.shape != x.shape or dout.dtype != x.dtype:
        raise ValueError("mamba_cpu::causal_conv1d_bwd expects dout shaped and typed like x")
    b, d, _ = x.shape
    width = weight.shape[1]
    if dfinal_states is not None:
        if dfinal_states.shape != (b, d, width - 1):
            raise ValueError("mamba_cpu::causal_conv1d_bwd expects dfinal_states (batch, dim, width - 1)")
        dfinal_states = dfinal_states.to(x.dtype).contiguous()
    dx = _like_x(x)
    dweight = weight.new_empty(weight.shape)
    dbias = weight.new_empty(d) if bias is not None else weight.new_empty(0)
    dinit = x.new_empty(b, d, width - 1) if initial_states is not None else x.new_empty(0)
    a = _conv_args(x, weight, bias, initial_states, silu)
    a.dout, a.dout_stride = dout.data_ptr(), _C.strides3(dout)
    a.dfinal_states = _C.ptr(dfinal_states)
    a.dx, a.dx_stride = dx.data_ptr(), _C.strides3(dx)
    a.dweight = dweight.data_ptr()
    a.dbias = dbias.data_ptr() if bias is not None else 0
    a.dinitial_states = dinit.data_ptr() if initial_states is not None else 0
    with _C.device_of(x):
        ws_bytes = _C.lib.mcpu_causal_conv1d_bwd_workspace_size(a)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        _C.call(_C.lib.mcpu_causal_conv1d_bwd, a, "mamba_cpu::causal_conv1d_bwd",
                ws.data_ptr(), ws_bytes, _C.stream_of(x))
    return dx, dweight, dbias, dinit


@_causal_conv1d_bwd.register_fake
def _(x, weight, bias, initial_states, dout, dfinal_states, silu):
    b, d, _ = x.shape
    return (
        _like_x(x), weight.new_empty(weight.shape),
        weight.new_empty(d) if bias is not None else weight.new_empty(0),
        x.new_empty(b, d, weight.shape[1] - 1) if initial_states is not None else x.new_empty(0),
    )


def _setup_context(ctx, inputs, output):
    x, weight, bias, initial_states, return_final_states, silu = inputs
    ctx.save_for_backward(x, weight, bias, initial_states)
    ctx.silu = silu
    ctx.return_final_states = return_final_states


def _backward(ctx, grad_out, grad_final):
    x, weight, bias, initial_states = ctx.saved_tensors
    dout = torch.zeros_like(x) if grad_out is None else grad_out.to(x.dtype)
    dfinal = grad_final if (ctx.return_final_states and grad_final is not None) else None
    dx, dweight, dbias, dinit = torch.ops.mamba_cpu.causal_conv1d_bwd(
        x, weight, bias, initial_states, dout, dfinal, ctx.silu
    )
    return (
        dx, dweight,
        dbias if bias is not None else None,
        dinit if initial_states is not None else None,
        None, None,
    )


torch.library.register_autograd(
    "mamba_cpu::causal_conv1d_fwd", _backward, setup_context=_setup_context
)


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
    initial_states: (batch, dim, width - 1)
    final_states_out: optional (batch, dim, width - 1) buffer for the final states
    Returns out: (batch, dim, seqlen) in x's dtype [, final_states: (batch, dim, width - 1)]
    """
    if seq_idx is not None:
        raise NotImplementedError("seq_idx is not supported yet")
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    silu = _silu_flag(activation)
    in_dtype = x.dtype
    if in_dtype not in _X_DTYPES:
        x = x.float()
    init = None if initial_states is None else initial_states.to(x.dtype)
    out, final = torch.ops.mamba_cpu.causal_conv1d_fwd(
        x, weight.float().contiguous(), None if bias is None else bias.float().contiguous(), init,
        bool(return_final_states), silu,
    )
    out = out.to(in_dtype)
    if not return_final_states:
        return out
    final = final.to(in_dtype)
    if final_states_out is not None:
        final = final_states_out.copy_(final)
    return out, final


@torch.library.custom_op("mamba_cpu::causal_conv1d_update", mutates_args=("conv_state",),
                         device_types="cuda")
def _causal_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor],
    silu: bool,
) -> torch.Tensor:
    """x: (batch, dim, seqlen); conv_state (batch, dim, state_len) in x's dtype,
    updated in place. Returns out (batch, dim, seqlen)."""
    for t in (x, conv_state, weight, bias):
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"mamba_cpu::causal_conv1d_update runs on ROCm GPU tensors, got {t.device}")
    if x.dtype not in _X_DTYPES or conv_state.dtype != x.dtype:
        raise ValueError("mamba_cpu::causal_conv1d_update expects x and conv_state of one dtype "
                         "among float32, bfloat16 and float16")
    if weight.dtype != torch.float32 or not weight.is_contiguous():
        raise ValueError("mamba_cpu::causal_conv1d_update expects a contiguous float32 weight")
    b, d, l = x.shape
    out = x.new_empty(x.shape)
    a = _C.ConvUpdateArgs()
    a.x, a.conv_state, a.weight = x.data_ptr(), conv_state.data_ptr(), weight.data_ptr()
    a.bias, a.out = _C.ptr(bias), out.data_ptr()
    a.batch, a.dim, a.seqlen = b, d, l
    a.width, a.state_len = weight.shape[1], conv_state.shape[-1]
    a.silu = int(bool(silu))
    a.dtype = _C.DTYPES[x.dtype]
    a.x_stride, a.state_stride, a.out_stride = (_C.strides3(x), _C.strides3(conv_state),
                                                _C.strides3(out))
    with _C.device_of(x):
        _C.call(_C.lib.mcpu_causal_conv1d_update, a, "mamba_cpu::causal_conv1d_update",
                _C.stream_of(x))
    return out


@_causal_conv1d_update.register_fake
def _(x, conv_state, weight, bias, silu):
    return x.new_empty(x.shape)


def causal_conv1d_update(
    x, conv_state, weight, bias=None, activation=None, cache_seqlens=None, conv_state_indices=None
):
    """Decode step(s). Updates conv_state in place.

    x: (batch, dim) or (batch, dim, seqlen)
    conv_state: (batch, dim, state_len), state_len >= width - 1
    weight: (dim, width)
    Returns out shaped like x.
    """
    if cache_seqlens is not None or conv_state_indices is not None:
        raise NotImplementedError("cache_seqlens and conv_state_indices are not supported yet")
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    silu = _silu_flag(activation)
    single_step = x.dim() == 2
    x_seq = x.unsqueeze(-1) if single_step else x
    width = weight.shape[1]
    state_len = conv_state.shape[-1]
    if state_len < width - 1:
        raise ValueError(f"conv_state length ({state_len}) must be at least width - 1 ({width - 1})")
    in_dtype = x.dtype
    if in_dtype not in _X_DTYPES:
        x_seq = x_seq.float()
    w = weight.float().contiguous()
    bb = None if bias is None else bias.float().contiguous()
    if conv_state.dtype == x_seq.dtype:
        out = torch.ops.mamba_cpu.causal_conv1d_update(x_seq, conv_state, w, bb, silu)
    else:
        # The reference mixes dtypes through conv_state.to(x.dtype) and a copy back.
        tmp = conv_state.to(x_seq.dtype)
        out = torch.ops.mamba_cpu.causal_conv1d_update(x_seq, tmp, w, bb, silu)
        conv_state.copy_(tmp)
    out = out.to(in_dtype)
    return out.squeeze(-1) if single_step else out

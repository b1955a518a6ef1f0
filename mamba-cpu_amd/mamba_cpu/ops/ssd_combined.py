"""mamba_chunk_scan_combined on MI355X: Mamba-2's SSD scan over the gfx950
kernels (csrc/ssd.hip), forward and backward.

The reference lists Mamba-2 SSD as roadmap (README.md:7, 94) and has no
implementation; this follows the public function of the mamba_ssm package
(mamba_ssm/ops/triton/ssd_combined.py, 2.x): the same signature, argument
layouts and results. Per batch row and head h (heads split into ngroups
contiguous groups that share B and C):

    dt_t = clamp(softplus?(dt_t + dt_bias_h), dt_limit)
    h_t  = exp(dt_t A_h) h_{t-1} + dt_t x_t B_t^T    (headdim x dstate state,
                                                      h_{-1} = initial_states or 0)
    y_t  = h_t C_t + D x_t ;  out = y silu(z) when z is given

With seq_idx (packed sequences: non-decreasing ids along each batch row) the
state does not cross a change of id: exp(dt_t A_h) is taken as 0 at the first
step of each new id, and the initial state belongs to id 0.

The kernels scan 64-step chunks whatever `chunk_size` says (it is accepted for
compatibility; the result does not depend on it beyond float32 rounding).
Arithmetic and states are float32 for every storage type; the chunk-local
contractions run on the matrix cores.
"""

import math

import torch

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_X_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_CHUNK = 64


def _align(n):
    return (n + 255) // 256 * 256


def _aligned(t):
    """t, copied when its data does not start on a 16-byte boundary (the
    kernels move four elements at a time)."""
    return t if t is None or t.data_ptr() % 16 == 0 else t.clone()


def _saved_bytes(b, l, h, p, n):
    """Bytes of the forward's saved buffer (the C ABI's layout): per-chunk
    running decays (a float pair) and steps, then per-chunk states, float32."""
    nch = (l + _CHUNK - 1) // _CHUNK
    chunk = 4 * b * h * nch * _CHUNK
    return 3 * _align(chunk) + _align(4 * b * nch * h * p * n)


@torch.library.register_fake("mamba_cpu::ssd_fwd")
def _(x, dt, A, B, C, D, z, dt_bias, initial_states, dt_softplus, dt_lo, dt_hi, save_for_backward,
      head_block=0, chunk_pass=0, seq_idx=None):
    b, l, h, p = x.shape
    n = B.shape[-1]
    ysave = x.new_empty(x.shape) if (save_for_backward and z is not None) else x.new_empty(0)
    return (x.new_empty(x.shape), x.new_empty(b, h, p, n, dtype=torch.float32),
            x.new_empty(_saved_bytes(b, l, h, p, n), dtype=torch.uint8), ysave)


@torch.library.register_fake("mamba_cpu::ssd_bwd")
def _(dout, dfinal_states, x, dt, A, B, C, D, z, dt_bias, initial_states, dt_softplus, dt_lo, dt_hi,
      saved, ysave, head_block=0, chunk_pass=0, seq_idx=None):
    f32 = dict(dtype=torch.float32)
    return (x.new_empty(x.shape), dt.new_empty(dt.shape, **f32), A.new_empty(A.shape, **f32),
            B.new_empty(B.shape, **f32), C.new_empty(C.shape, **f32),
            A.new_empty(D.shape, **f32) if D is not None else A.new_empty(0),
            x.new_empty(x.shape) if z is not None else x.new_empty(0),
            A.new_empty(A.shape, **f32) if dt_bias is not None else A.new_empty(0),
            A.new_empty(initial_states.shape, **f32) if initial_states is not None else A.new_empty(0))


@torch.library.register_fake("mamba_cpu::ssd_varlen_states")
def _(x, dt, A, B, C, D, z, dt_bias, initial_states, dt_softplus, dt_lo, dt_hi, saved, cu_seqlens,
      head_block=0, chunk_pass=0, seq_idx=None):
    return x.new_empty(cu_seqlens.shape[0] - 1, x.shape[2], x.shape[3], B.shape[-1], dtype=torch.float32)


def _varlen(args, saved, cu_seqlens, seq_idx):
    return torch.ops.mamba_cpu.ssd_varlen_states(*args, saved, cu_seqlens, seq_idx=seq_idx)


class _SsdScan(torch.autograd.Function):
    """Autograd of the SSD scan: the forward keeps its per-chunk decays and
    states (and y before the z gate), the backward reads them. Per-sequence
    final states, when asked for, carry no gradient (as in mamba_ssm)."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, lo, hi, seq_idx, cu_seqlens):
        args = (x, dt, A, B, C, D, z, dt_bias, initial_states, softplus, lo, hi)
        out, final, saved, ysave = torch.ops.mamba_cpu.ssd_fwd(*args, True, seq_idx=seq_idx)
        varlen = x.new_empty(0, dtype=torch.float32) if cu_seqlens is None else _varlen(args, saved, cu_seqlens,
                                                                                         seq_idx)
        ctx.mark_non_differentiable(varlen)
        ctx.save_for_backward(x, dt, A, B, C, D, z, dt_bias, initial_states, saved, ysave, seq_idx)
        ctx.cfg = (softplus, lo, hi)
        ctx.set_materialize_grads(False)
        return out, final, varlen

    @staticmethod
    def backward(ctx, dout, dfinal, _dvarlen):
        x, dt, A, B, C, D, z, dt_bias, init, saved, ysave, seq_idx = ctx.saved_tensors
        dout = torch.zeros_like(x) if dout is None else _aligned(dout.to(x.dtype).contiguous())
        dfinal = None if dfinal is None else dfinal.float().contiguous()
        dx, ddt, dA, dB, dC, dD, dz, dbias, dinit = torch.ops.mamba_cpu.ssd_bwd(
            dout, dfinal, x, dt, A, B, C, D, z, dt_bias, init, *ctx.cfg, saved, ysave, seq_idx=seq_idx)
        return (dx, ddt, dA, dB.to(B.dtype), dC.to(C.dtype), dD if D is not None else None,
                dz if z is not None else None, dbias if dt_bias is not None else None,
                dinit if init is not None else None, None, None, None, None, None)


def mamba_chunk_scan_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                              initial_states=None, seq_idx=None, cu_seqlens=None, dt_softplus=False,
                              dt_limit=(0.0, float("inf")), return_final_states=False,
                              return_varlen_states=False):
    """Drop-in for mamba_ssm.ops.triton.ssd_combined.mamba_chunk_scan_combined
    on ROCm GPU tensors.

    x: (batch, seqlen, nheads, headdim); dt: (batch, seqlen, nheads);
    A: (nheads,); B, C: (batch, seqlen, ngroups, dstate); D: (nheads, headdim)
    or (nheads,); z: like x; dt_bias: (nheads,); initial_states:
    (batch, nheads, headdim, dstate); seq_idx: (batch, seqlen) integer ids,
    non-decreasing along each row (not checked, as in mamba_ssm). headdim a
    multiple of 16 up to 64, dstate a multiple of 16 up to 128.
    Returns out (like x, in x's dtype) [, final_states (batch, nheads, headdim,
    dstate) float32] [, varlen_states (nseqs, nheads, headdim, dstate)
    float32]. varlen_states (return_varlen_states, batch 1, cu_seqlens the
    nseqs + 1 offsets of the packed sequences, seq_idx marking the same
    sequences): the state after each sequence's last step, zeros for an empty
    sequence, without gradient.
    """
    if x.device.type != "cuda":
        raise ValueError(f"mamba_cpu (MI355X build) runs on ROCm GPU tensors, got device {x.device}")
    if return_varlen_states:
        if cu_seqlens is None or seq_idx is None:
            raise ValueError("return_varlen_states needs cu_seqlens and the seq_idx of the same sequences")
        if x.shape[0] != 1:
            raise ValueError(f"return_varlen_states needs batch 1, got {x.shape[0]}")
        if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1 or cu_seqlens.dtype.is_floating_point:
            raise ValueError("cu_seqlens must be a 1-D integer tensor of nseqs + 1 offsets")
        cu_seqlens = cu_seqlens.to(device=x.device, dtype=torch.int32).contiguous()
    else:
        cu_seqlens = None   # accepted and unused, as mamba_ssm computes and drops the states
    if int(chunk_size) < 1:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    if x.dim() != 4 or dt.dim() != 3 or B.dim() != 4 or C.dim() != 4 or A.dim() != 1:
        raise ValueError("mamba_chunk_scan_combined expects x (b, l, h, p), dt (b, l, h), A (h,), "
                         "B and C (b, l, g, n)")
    b, l, h, p = x.shape
    if h % B.shape[2] != 0:
        raise ValueError(f"nheads ({h}) must be divisible by ngroups ({B.shape[2]})")
    xdt = x.dtype if x.dtype in _X_DTYPES else torch.float32
    lo, hi = float(dt_limit[0]), float(dt_limit[1])
    if D is not None:
        D = D.float()
        D = (D[:, None].expand(h, p) if D.dim() == 1 else D).contiguous()
    args = (
        _aligned(x.to(xdt).contiguous()), dt.float().contiguous(), A.float().contiguous(),
        _aligned(B.to(xdt).contiguous()), _aligned(C.to(xdt).contiguous()), D,
        None if z is None else _aligned(z.to(xdt).contiguous()),
        None if dt_bias is None else dt_bias.float().contiguous(),
        None if initial_states is None else initial_states.float().contiguous(),
        bool(dt_softplus), lo, hi,
    )
    if seq_idx is not None:
        if seq_idx.shape != (b, l) or seq_idx.dtype.is_floating_point:
            raise ValueError(f"seq_idx must hold integer ids of shape ({b}, {l}), got {tuple(seq_idx.shape)} "
                             f"{seq_idx.dtype}")
        seq_idx = seq_idx.to(device=x.device, dtype=torch.int32).contiguous()
    needs_grad = torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in args)
    if needs_grad:
        out, final, varlen = _SsdScan.apply(*args, seq_idx, cu_seqlens)
    else:
        out, final, saved, _ = torch.ops.mamba_cpu.ssd_fwd(*args, False, seq_idx=seq_idx)
        varlen = None if cu_seqlens is None else _varlen(args, saved, cu_seqlens, seq_idx)
    out = out.to(x.dtype)
    res = (out, final) if return_final_states else (out,)
    if return_varlen_states:
        res = res + (varlen,)
    return res if len(res) > 1 else out


def ssd_flops(batch, seqlen, nheads, headdim, ngroups, dstate, backward=False):
    """Matrix FLOPs of the chunked algorithm (64-step chunks), per direction,
    counting C B^T once per group and chunk (the heads of a group share it);
    used to place a timing against the float32 matrix peak. The kernels form
    C B^T once per head block, so they run somewhat more than this."""
    nch = math.ceil(seqlen / _CHUNK)
    Q, P, N = _CHUNK, headdim, dstate
    per_head = batch * nch * nheads
    per_group = batch * nch * ngroups
    cbt = per_group * 2 * Q * Q * N
    # forward: the chunk state (P x N over Q), the intra-chunk output (Q x P
    # over Q) and the state's output (Q x P over N)
    fwd = cbt + per_head * 2 * (P * N * Q + Q * P * Q + Q * P * N)
    if not backward:
        return fwd
    # backward: the seed E (P x N over Q), dY x^T (Q x Q over P), G^T dY, dCB B
    # and dCB^T C (over Q), then (dt x) dH, dY H and B~ dH^T (over the state)
    return cbt + per_head * 2 * (P * N * Q + Q * Q * P + Q * P * Q + 2 * Q * N * Q + 3 * Q * N * P)

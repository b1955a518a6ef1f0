"""Float64 numpy restatement of Mamba-2's SSD scan, mamba_ssm's
mamba_chunk_scan_combined: TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference has no SSD path: it lists it as roadmap (README.md:7, 94). Its
semantics are those of the mamba_ssm package (mamba_ssm/ops/triton/
ssd_combined.py, 2.x; not installed here), restated from the recurrence of
the Mamba-2 paper, per batch row and head h (heads split into ngroups
contiguous groups that share B and C):

    dt_t = clamp(softplus?(dt_t + dt_bias_h), dt_limit)
    h_t  = exp(dt_t A_h) h_{t-1} + dt_t x_t B_t^T     h: (headdim, dstate),
                                                       h_{-1} = initial_states or 0
    y_t  = h_t C_t + D x_t ;  out_t = y_t silu(z_t) when z is given

With seq_idx (batch, seqlen) of non-decreasing sequence ids (packed
sequences), the state does not carry across a change of id: the decay
exp(dt_t A_h) is replaced by 0 where seq_idx[t] != seq_idx[t-1], and the
initial state belongs to sequence id 0 (it is dropped when seq_idx[0] != 0),
as mamba_ssm's kernels mask it (its state passing starts from sequence id 0).

Layouts (mamba_ssm's): x, z, out (batch, seqlen, nheads, headdim); dt
(batch, seqlen, nheads); A, dt_bias (nheads,); B, C (batch, seqlen, ngroups,
dstate); D (nheads, headdim) or (nheads,); states (batch, nheads, headdim,
dstate). Chunking is the implementations' business: the result does not
depend on a chunk size.

Pinned by tests/test_oracle_ssd.py against the Mamba-1 oracle (A broadcast
over each head's channels and states), a quadratic direct sum, and
torch.autograd through that direct sum; seq_idx by running each packed
sequence on its own.
"""

import numpy as np

from oracle.numerics import _f64, sigmoid, softplus


def _dt(dt, dt_bias, dt_softplus, dt_limit):
    """The effective step and the factor d(step)/d(raw dt): softplus'
    derivative, times 0 where the clamp to dt_limit is active."""
    pre = dt if dt_bias is None else dt + dt_bias[None, None, :]
    step = softplus(pre) if dt_softplus else pre
    grad = sigmoid(pre) if dt_softplus else np.ones_like(pre)
    lo, hi = dt_limit
    # Always clamped, as mamba_ssm's _chunk_cumsum kernels and transformers'
    # mamba2_chunk_scan do: with the default (0, inf) a negative raw step is 0.
    inside = (step >= lo) & (step <= hi)
    step = np.clip(step, lo, hi)
    grad = grad * inside
    return step, grad


def _per_head(X, nheads):
    """(batch, seqlen, ngroups, dstate) -> (batch, seqlen, nheads, dstate)."""
    return np.repeat(X, nheads // X.shape[2], axis=2)


def _D_full(D, nheads, headdim):
    if D is None:
        return np.zeros((nheads, headdim))
    return np.broadcast_to(D[:, None] if D.ndim == 1 else D, (nheads, headdim))


def _keep(seq_idx, batch, seqlen):
    """(batch, seqlen) 1.0 where the state carries into step t, else 0.0."""
    if seq_idx is None:
        return np.ones((batch, seqlen))
    sq = np.asarray(seq_idx, dtype=np.int64).reshape(batch, seqlen)
    prev = np.concatenate([np.zeros((batch, 1), dtype=np.int64), sq[:, :-1]], axis=1)
    return (sq == prev).astype(np.float64)


def ssd_fwd(x, dt, A, B, C, D=None, z=None, dt_bias=None, initial_states=None, dt_softplus=False,
            dt_limit=(0.0, float("inf")), seq_idx=None):
    """Forward. Returns (out (b, l, h, p), final_states (b, h, p, n))."""
    x, dt, A, B, C = map(_f64, (x, dt, A, B, C))
    D, z, dt_bias, init = map(_f64, (D, z, dt_bias, initial_states))
    batch, seqlen, nheads, headdim = x.shape
    dstate = B.shape[-1]
    step, _ = _dt(dt, dt_bias, dt_softplus, dt_limit)
    Bh, Ch = _per_head(B, nheads), _per_head(C, nheads)
    Dh = _D_full(D, nheads, headdim)
    h = np.zeros((batch, nheads, headdim, dstate)) if init is None else init.copy()
    y = np.zeros_like(x)
    keep = _keep(seq_idx, batch, seqlen)
    with np.errstate(over="ignore", invalid="ignore"):
        for t in range(seqlen):
            a = np.exp(step[:, t] * A[None]) * keep[:, t, None]            # (b, h)
            h = a[..., None, None] * h + (step[:, t, :, None] * x[:, t])[..., None] * Bh[:, t, :, None, :]
            y[:, t] = (h * Ch[:, t, :, None, :]).sum(-1) + Dh[None] * x[:, t]
        out = y if z is None else y * z * sigmoid(z)
    return out, h


def ssd_varlen_states(x, dt, A, B, C, cu_seqlens, dt_bias=None, initial_states=None, dt_softplus=False,
                      dt_limit=(0.0, float("inf")), seq_idx=None):
    """Per-sequence final states of packed sequences in batch row 0 (the
    result of mamba_ssm's return_varlen_states): (nseqs, h, p, n), entry i
    the recurrence's state after step cu_seqlens[i + 1] - 1, zeros for an
    empty sequence. The same recurrence as ssd_fwd (seq_idx included)."""
    x, dt, A, B = map(_f64, (x, dt, A, B))
    dt_bias, init = map(_f64, (dt_bias, initial_states))
    batch, seqlen, nheads, headdim = x.shape
    step, _ = _dt(dt, dt_bias, dt_softplus, dt_limit)
    Bh = _per_head(B, nheads)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    h = np.zeros((nheads, headdim, B.shape[-1])) if init is None else init[0].copy()
    keep = _keep(seq_idx, batch, seqlen)[0]
    after = [h.copy()]                                                      # after[t + 1] = h_t
    with np.errstate(over="ignore", invalid="ignore"):
        for t in range(seqlen):
            h = np.exp(step[0, t] * A) [:, None, None] * keep[t] * h + \
                (step[0, t, :, None] * x[0, t])[..., None] * Bh[0, t, :, None, :]
            after.append(h)
    out = np.zeros((len(cu) - 1,) + h.shape)
    for i in range(len(cu) - 1):
        if cu[i + 1] > cu[i]:
            out[i] = after[cu[i + 1]]
    return out


def ssd_bwd(x, dt, A, B, C, D=None, z=None, dt_bias=None, initial_states=None, dt_softplus=False,
            dt_limit=(0.0, float("inf")), dout=None, dfinal_states=None, seq_idx=None):
    """Backward by the chain rule on the recurrence, walking t = L-1 .. 0 with
    G = dLoss/dh_t (headdim x dstate per head), started from dfinal_states:
        dy = dout silu(z) ; dz = dout y silu'(z)            (dy = dout without z)
        G += dy_t C_t^T ;  dC_t = sum over the group's heads of h_t^T dy_t
        dB_t = sum over the group's heads of (dt_t x_t)^T G ;  dx_t = dt_t G B_t + D dy_t
        dstep_t = <G, x_t B_t^T> + A <G, a_t h_{t-1}> ;  dA += dt_t <G, a_t h_{t-1}>
        G <- a_t G     (a_t = exp(dt_t A), or 0 where seq_idx starts a sequence)
    then dinitial_states = G, draw dt = dstep * softplus' * [inside dt_limit],
    ddt_bias = its sum over batch and sequence, and dD = sum of dy x.
    Returns (dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinitial_states); entries
    for absent optional inputs are None; dD has D's shape."""
    x, dt, A, B, C = map(_f64, (x, dt, A, B, C))
    D, z, dt_bias, init = map(_f64, (D, z, dt_bias, initial_states))
    dout, dfin = _f64(dout), _f64(dfinal_states)
    batch, seqlen, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    hpg = nheads // ngroups
    step, dstep_draw = _dt(dt, dt_bias, dt_softplus, dt_limit)
    Bh, Ch = _per_head(B, nheads), _per_head(C, nheads)
    Dh = _D_full(D, nheads, headdim)
    if dout is None:
        dout = np.zeros_like(x)
    with np.errstate(over="ignore", invalid="ignore"):
        hs = np.zeros((seqlen + 1, batch, nheads, headdim, dstate))       # hs[t + 1] = h_t
        hs[0] = 0.0 if init is None else init
        a_all = np.exp(step * A[None, None]) * _keep(seq_idx, batch, seqlen)[..., None]  # (b, l, h)
        for t in range(seqlen):
            hs[t + 1] = a_all[:, t, :, None, None] * hs[t] + \
                (step[:, t, :, None] * x[:, t])[..., None] * Bh[:, t, :, None, :]
        y = np.einsum("bhpn,bhn->bhp", hs[1:].transpose(1, 0, 2, 3, 4).reshape(-1, nheads, headdim, dstate),
                      Ch.reshape(-1, nheads, dstate)).reshape(batch, seqlen, nheads, headdim) + Dh[None, None] * x
        if z is not None:
            sg = sigmoid(z)
            dy = dout * z * sg
            dz = dout * y * sg * (1 + z * (1 - sg))
        else:
            dy, dz = dout, None
        G = np.zeros((batch, nheads, headdim, dstate)) if dfin is None else dfin.copy()
        dx = np.zeros_like(x)
        dstep = np.zeros_like(step)
        dA = np.zeros(nheads)
        dBh = np.zeros_like(Bh)
        dCh = np.zeros_like(Ch)
        for t in range(seqlen - 1, -1, -1):
            h_t, h_prev = hs[t + 1], hs[t]
            G = G + dy[:, t][..., None] * Ch[:, t, :, None, :]
            dCh[:, t] = (h_t * dy[:, t][..., None]).sum(2)
            xs = step[:, t, :, None] * x[:, t]                              # (b, h, p)
            dBh[:, t] = (G * xs[..., None]).sum(2)
            GB = (G * Bh[:, t, :, None, :]).sum(-1)                         # (b, h, p)
            dx[:, t] = step[:, t, :, None] * GB + Dh[None] * dy[:, t]
            a = a_all[:, t]
            decay_term = (G * h_prev).sum((-1, -2)) * a                     # <G, a h_{t-1}>
            dstep[:, t] = (GB * x[:, t]).sum(-1) + A[None] * decay_term
            dA += (step[:, t] * decay_term).sum(0)
            G = a[..., None, None] * G
        ddt = dstep * dstep_draw
        dB = dBh.reshape(batch, seqlen, ngroups, hpg, dstate).sum(3)
        dC = dCh.reshape(batch, seqlen, ngroups, hpg, dstate).sum(3)
        dD = None
        if D is not None:
            full = (dy * x).sum((0, 1))                                     # (h, p)
            dD = full.sum(-1) if D.ndim == 1 else full
        ddt_bias = None if dt_bias is None else ddt.sum((0, 1))
        dinit = None if init is None else G
    return dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinit

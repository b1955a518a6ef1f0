"""Float64 numpy restatement of the reference's Mamba-1 algorithms.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Inputs may be numpy arrays
or CPU torch tensors; everything is computed in float64 and returned as numpy
float64 arrays.

Layouts follow the reference's public API (README.md:60-67):
  u, delta, z, dout : (batch, dim, seqlen)
  A                 : (dim, dstate)
  B, C              : (batch, dstate, seqlen) or (batch, ngroups, dstate, seqlen)
  D, delta_bias     : (dim,)
Channels are split into contiguous groups sharing B/C
(csrc/selective_scan.cpp:99: slice = b * ngroups + d / (dim / ngroups)).
"""

import numpy as np


def _f64(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def softplus(x):
    """softplus with torch's default threshold 20 (csrc/selective_scan.cpp:44-45)."""
    with np.errstate(over="ignore", invalid="ignore"):
        return np.where(x <= 20.0, np.log1p(np.exp(np.minimum(x, 20.0))), x)


def sigmoid(x):
    """csrc/selective_scan.cpp:47."""
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-x))


def _groups(X, dim):
    """(b, n, l) | (b, g, n, l) -> (b, g, n, l) plus channels-per-group."""
    X = _f64(X)
    if X.ndim == 3:
        X = X[:, None]
    g = X.shape[1]
    return X, dim // g


def _input_independent(X, batch, seqlen):
    """A 2-D (dim, dstate) B or C (input-independent, mamba_ssm's
    `is_variable_B = False` case) as the equivalent (b, dim, n, l) tensor:
    one group per channel, the same values at every step; None for 3-/4-D."""
    X = _f64(X)
    if X.ndim != 2:
        return None
    return np.broadcast_to(X[None, :, :, None], (batch, X.shape[0], X.shape[1], seqlen))


def _dt(delta, delta_bias, delta_softplus):
    """row_dt (csrc/selective_scan.cpp:112-115): softplus?(delta + bias)."""
    dt = delta if delta_bias is None else delta + delta_bias[None, :, None]
    return softplus(dt) if delta_softplus else dt


def selective_scan_fwd(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    """Forward scan. Follows fwd_row_body (csrc/selective_scan.cpp:120-145) and
    selective_scan_ref (src/mamba_cpu/reference.py:10-62):
        dt_t = softplus?(delta_t + bias)
        h_t  = exp(dt_t * A) * h_{t-1} + dt_t * u_t * B_t       (h_{-1} = 0)
        y_t  = <h_t, C_t> + D * u_t ;  out_t = y_t * silu(z_t)
    B and C may have different group counts, and either may be 2-D
    (dim, dstate), input-independent (mamba_ssm's selective_scan_ref).
    Returns (out, last_state) with last_state = h_{L-1}, shape (b, d, n)."""
    u, delta, A = _f64(u), _f64(delta), _f64(A)
    D, z, delta_bias = _f64(D), _f64(z), _f64(delta_bias)
    batch, dim, seqlen = u.shape
    for name in ("B", "C"):
        X = _input_independent(B if name == "B" else C, batch, seqlen)
        if X is not None:
            B, C = (X, C) if name == "B" else (B, X)
    B, dpg = _groups(B, dim)
    C, dpgC = _groups(C, dim)
    dt = _dt(delta, delta_bias, delta_softplus)
    h = np.zeros((batch, dim, A.shape[1]))
    y = np.zeros((batch, dim, seqlen))
    with np.errstate(over="ignore", invalid="ignore"):
        for t in range(seqlen):
            Bt = np.repeat(B[:, :, :, t], dpg, axis=1)  # (b, d, n)
            Ct = np.repeat(C[:, :, :, t], dpgC, axis=1)
            a = np.exp(dt[:, :, t, None] * A[None])
            h = a * h + (dt[:, :, t] * u[:, :, t])[..., None] * Bt
            y[:, :, t] = (h * Ct).sum(-1)
        out = y if D is None else y + D[None, :, None] * u
        if z is not None:
            out = out * z * sigmoid(z)
    return out, h


def selective_scan_bwd(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                       dout=None, dlast_state=None):
    """Analytic backward, restating bwd_row_body (csrc/selective_scan.cpp:168-248)
    in float64 and vectorised over (batch, dim, dstate):
        recompute h_t for all t (:181-190), then for t = L-1 .. 0 (:200-243)
          y  = <h_t, C_t> + D u ; dz = dout * y * s(z) (1 + z (1 - s(z))) ; dy = dout * z * s(z)
          g  = gh + dy C_t ; dC_t += dy h_t ; a = exp(dt A) ; ga = g h_{t-1} a
          dA += ga dt ; ddt += ga A + g u B_t ; dB_t += g dt u ; gh = g a
          du = dy D + dt <g, B_t> ; ddt *= sigmoid(delta + bias) if softplus
    gh starts at dlast_state (:193-196). dA, dD and ddelta_bias are summed over
    the batch (the reference returns per-batch partials that its Python side
    sums, selective_scan_interface.py:87).
    Returns (du, ddelta, dA, dB, dC, dD, dz, ddelta_bias) with dB/dC in B/C's
    layout; dD / dz / ddelta_bias are None when D / z / delta_bias are None."""
    u, delta, A = _f64(u), _f64(delta), _f64(A)
    D, z, delta_bias = _f64(D), _f64(z), _f64(delta_bias)
    dout, dlast_state = _f64(dout), _f64(dlast_state)
    batch, dim, seqlen = u.shape
    N = A.shape[1]
    ndimB, ndimC = _f64(B).ndim, _f64(C).ndim
    B2, C2 = _input_independent(B, batch, seqlen), _input_independent(C, batch, seqlen)
    B = B if B2 is None else B2
    C = C if C2 is None else C2
    B, dpg = _groups(B, dim)
    C, dpgC = _groups(C, dim)
    G, GC = B.shape[1], C.shape[1]
    if dout is None:
        dout = np.zeros_like(u)
    dt = _dt(delta, delta_bias, delta_softplus)
    pre = delta if delta_bias is None else delta + delta_bias[None, :, None]
    Dv = np.zeros(dim) if D is None else D

    with np.errstate(over="ignore", invalid="ignore"):
        hs = np.zeros((seqlen + 1, batch, dim, N))  # hs[t + 1] = h_t, hs[0] = 0
        for t in range(seqlen):
            Bt = np.repeat(B[:, :, :, t], dpg, axis=1)
            hs[t + 1] = np.exp(dt[:, :, t, None] * A[None]) * hs[t] + \
                (dt[:, :, t] * u[:, :, t])[..., None] * Bt

        gh = np.zeros((batch, dim, N)) if dlast_state is None else dlast_state.copy()
        du = np.zeros_like(u)
        ddelta = np.zeros_like(u)
        dz = None if z is None else np.zeros_like(u)
        dA = np.zeros((batch, dim, N))
        dB = np.zeros((batch, G, N, seqlen))
        dC = np.zeros((batch, GC, N, seqlen))
        for t in range(seqlen - 1, -1, -1):
            Bt = np.repeat(B[:, :, :, t], dpg, axis=1)
            Ct = np.repeat(C[:, :, :, t], dpgC, axis=1)
            h, h_prev = hs[t + 1], hs[t]
            ut, dtt = u[:, :, t], dt[:, :, t]
            dy = dout[:, :, t]
            if z is not None:
                y = (h * Ct).sum(-1) + Dv[None] * ut
                zt = z[:, :, t]
                sg = sigmoid(zt)
                dz[:, :, t] = dout[:, :, t] * y * sg * (1 + zt * (1 - sg))
                dy = dout[:, :, t] * zt * sg
            g = gh + dy[..., None] * Ct
            dCc = dy[..., None] * h
            a = np.exp(dtt[..., None] * A[None])
            ga = g * h_prev * a
            dA += ga * dtt[..., None]
            ddt = (ga * A[None]).sum(-1) + ut * (g * Bt).sum(-1)
            dBc = g * (dtt * ut)[..., None]
            du[:, :, t] = dy * Dv[None] + dtt * (g * Bt).sum(-1)
            if delta_softplus:
                ddt = ddt * sigmoid(pre[:, :, t])
            ddelta[:, :, t] = ddt
            gh = g * a
            dB[:, :, :, t] = dBc.reshape(batch, G, dpg, N).sum(2)
            dC[:, :, :, t] = dCc.reshape(batch, GC, dpgC, N).sum(2)
        dD_full = None
        if D is not None:
            dy_all = dout if z is None else dout * z * sigmoid(z)
            dD_full = (dy_all * u).sum((0, 2))
        ddelta_bias = None if delta_bias is None else ddelta.sum((0, 2))
    # dB/dC in B's and C's own shapes: (b, n, l), (b, g, n, l) or (dim, n).
    dB = dB.sum((0, 3)) if ndimB == 2 else (dB[:, 0] if ndimB == 3 else dB)
    dC = dC.sum((0, 3)) if ndimC == 2 else (dC[:, 0] if ndimC == 3 else dC)
    return du, ddelta, dA.sum(0), dB, dC, dD_full, dz, ddelta_bias


def _is_complex(x):
    return x.is_complex() if hasattr(x, "is_complex") else np.iscomplexobj(x)


def _c128(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x, dtype=np.complex128)


def _complex_bc(X, dim, batch, seqlen):
    """B or C of a complex-A scan as complex (b, g, n, l) plus channels per
    group. Input-dependent B/C are real (b, n, 2l) or (b, g, n, 2l) holding
    (re, im) pairs along the last dim (mamba_ssm's selective_scan_ref:
    view_as_complex over "... (L two) -> ... L two"); a 2-D (dim, dstate)
    B/C is complex and input-independent (one group per channel)."""
    if _is_complex(X):
        X = _c128(X)
        if X.ndim != 2:
            raise ValueError("complex B/C must be 2-D (dim, dstate)")
        return np.broadcast_to(X[None, :, :, None], (batch, X.shape[0], X.shape[1], seqlen)), 1
    X = _f64(X)
    if X.ndim == 3:
        X = X[:, None]
    Xc = X[..., 0::2] + 1j * X[..., 1::2]
    return Xc, dim // Xc.shape[1]


def selective_scan_fwd_complex(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                               delta_softplus=False):
    """Forward scan with complex A (mamba_ssm's selective_scan_ref semantics;
    the reference rejects complex A, src/mamba_cpu/ops/selective_scan_interface.py:160-161):
        h_t = exp(dt_t * A) * h_{t-1} + dt_t * u_t * B_t      (complex, h_{-1} = 0)
        y_t = 2 * Re(sum_n h_t C_t) + D * u_t ;  out_t = y_t * silu(z_t)
    A: complex (dim, dstate). B/C: see _complex_bc. Returns (out, last_state)
    with last_state complex (b, d, n)."""
    u, delta, A = _f64(u), _f64(delta), _c128(A)
    D, z, delta_bias = _f64(D), _f64(z), _f64(delta_bias)
    batch, dim, seqlen = u.shape
    B, dpg = _complex_bc(B, dim, batch, seqlen)
    C, dpgC = _complex_bc(C, dim, batch, seqlen)
    dt = _dt(delta, delta_bias, delta_softplus)
    h = np.zeros((batch, dim, A.shape[1]), dtype=np.complex128)
    y = np.zeros((batch, dim, seqlen))
    with np.errstate(over="ignore", invalid="ignore"):
        for t in range(seqlen):
            Bt = np.repeat(B[:, :, :, t], dpg, axis=1)
            Ct = np.repeat(C[:, :, :, t], dpgC, axis=1)
            h = np.exp(dt[:, :, t, None] * A[None]) * h + (dt[:, :, t] * u[:, :, t])[..., None] * Bt
            y[:, :, t] = 2.0 * (h * Ct).sum(-1).real
        out = y if D is None else y + D[None, :, None] * u
        if z is not None:
            out = out * z * sigmoid(z)
    return out, h


def _complex_bc_grad(G, X, dpg):
    """dLoss/dB for B = X from the per-channel complex gradient G (b, d, n, l)
    (real part: dLoss/dRe, imaginary part: dLoss/dIm), in X's own layout."""
    b, d, n, l = G.shape
    Gg = G.reshape(b, d // dpg, dpg, n, l).sum(2)
    if _is_complex(X):
        return G.sum((0, 3))
    out = np.stack([Gg.real, Gg.imag], axis=-1).reshape(b, d // dpg, n, 2 * l)
    return out[:, 0] if _f64(X).ndim == 3 else out


def selective_scan_bwd_complex(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                               delta_softplus=False, dout=None, dlast_state=None):
    """Backward of selective_scan_fwd_complex by the chain rule on the real and
    imaginary parts. A complex gradient holds dLoss/dRe + i dLoss/dIm (torch's
    convention for complex leaves). For t = L-1 .. 0, with gh = dLoss/dh_t
    carried backwards from dlast_state:
        g  = gh + 2 dy conj(C_t) ;  dC_t = 2 dy conj(h_t) ;  dB_t = g dt u
        gh = g conj(a_t)  (a_t = exp(dt A)) ;  q = gh conj(h_{t-1}) ;  dA += dt q
        ddt = sum_n Re(q conj(A)) + u sum_n Re(g conj(B_t))
        du  = dy D + dt sum_n Re(g conj(B_t))
    (dy, dz, the softplus factor and dD / ddelta_bias as in the real scan).
    Returns (du, ddelta, dA, dB, dC, dD, dz, ddelta_bias); dA complex (d, n),
    dB/dC in B's and C's layouts."""
    u, delta, A = _f64(u), _f64(delta), _c128(A)
    D, z, delta_bias = _f64(D), _f64(z), _f64(delta_bias)
    dout = _f64(dout)
    dlast_state = _c128(dlast_state)
    batch, dim, seqlen = u.shape
    N = A.shape[1]
    Bc, dpg = _complex_bc(B, dim, batch, seqlen)
    Cc, dpgC = _complex_bc(C, dim, batch, seqlen)
    if dout is None:
        dout = np.zeros_like(u)
    dt = _dt(delta, delta_bias, delta_softplus)
    pre = delta if delta_bias is None else delta + delta_bias[None, :, None]
    Dv = np.zeros(dim) if D is None else D
    with np.errstate(over="ignore", invalid="ignore"):
        hs = np.zeros((seqlen + 1, batch, dim, N), dtype=np.complex128)
        for t in range(seqlen):
            Bt = np.repeat(Bc[:, :, :, t], dpg, axis=1)
            hs[t + 1] = np.exp(dt[:, :, t, None] * A[None]) * hs[t] + \
                (dt[:, :, t] * u[:, :, t])[..., None] * Bt
        gh = np.zeros((batch, dim, N), dtype=np.complex128) if dlast_state is None else dlast_state.copy()
        du = np.zeros_like(u)
        ddelta = np.zeros_like(u)
        dz = None if z is None else np.zeros_like(u)
        dA = np.zeros((batch, dim, N), dtype=np.complex128)
        dBf = np.zeros((batch, dim, N, seqlen), dtype=np.complex128)
        dCf = np.zeros((batch, dim, N, seqlen), dtype=np.complex128)
        for t in range(seqlen - 1, -1, -1):
            Bt = np.repeat(Bc[:, :, :, t], dpg, axis=1)
            Ct = np.repeat(Cc[:, :, :, t], dpgC, axis=1)
            h, h_prev = hs[t + 1], hs[t]
            ut, dtt = u[:, :, t], dt[:, :, t]
            dy = dout[:, :, t]
            if z is not None:
                y = 2.0 * (h * Ct).sum(-1).real + Dv[None] * ut
                zt = z[:, :, t]
                sg = sigmoid(zt)
                dz[:, :, t] = dout[:, :, t] * y * sg * (1 + zt * (1 - sg))
                dy = dout[:, :, t] * zt * sg
            g = gh + 2.0 * dy[..., None] * np.conj(Ct)
            dCf[:, :, :, t] = 2.0 * dy[..., None] * np.conj(h)
            a = np.exp(dtt[..., None] * A[None])
            gh = g * np.conj(a)
            q = gh * np.conj(h_prev)
            dA += dtt[..., None] * q
            gB = (g * np.conj(Bt)).real.sum(-1)
            ddt = (q * np.conj(A[None])).real.sum(-1) + ut * gB
            dBf[:, :, :, t] = g * (dtt * ut)[..., None]
            du[:, :, t] = dy * Dv[None] + dtt * gB
            if delta_softplus:
                ddt = ddt * sigmoid(pre[:, :, t])
            ddelta[:, :, t] = ddt
        dD_full = None
        if D is not None:
            dy_all = dout if z is None else dout * z * sigmoid(z)
            dD_full = (dy_all * u).sum((0, 2))
        ddelta_bias = None if delta_bias is None else ddelta.sum((0, 2))
    dB = _complex_bc_grad(dBf, B, dpg)
    dC = _complex_bc_grad(dCf, C, dpgC)
    return du, ddelta, dA.sum(0), dB, dC, dD_full, dz, ddelta_bias


def _tap_mask(seq_idx, width, seqlen):
    """(b, 1, width, seqlen) 0/1: tap k of output t reads x[t - (width-1) + k],
    which counts only inside t's own sequence (seq_idx equal, position >= 0),
    the upstream causal_conv1d package's seq_idx semantics. None without
    seq_idx."""
    if seq_idx is None:
        return None
    sq = np.asarray(seq_idx)
    m = np.zeros((sq.shape[0], 1, width, seqlen))
    for k in range(width):
        src = np.arange(seqlen) - (width - 1) + k
        ok = src >= 0
        m[:, 0, k, ok] = (sq[:, src[ok]] == sq[:, ok]).astype(np.float64)
    return m


def causal_conv1d_fwd(x, weight, bias=None, initial_states=None, activation=None, seq_idx=None):
    """Depthwise causal conv (src/mamba_cpu/ops/causal_conv1d.py:16-53 and the
    explicit tap loop of src/mamba_cpu/reference.py:65-75):
        x_full = [initial_states or zeros(width-1), x]
        out_t  = act(bias + sum_k w[k] * x_full[t + k])
    seq_idx (b, seqlen), which the reference rejects (:34-35): packed
    sequences; a tap reading another sequence's input counts as zero.
    Returns (out, final_states) with final_states = last width-1 columns of x_full."""
    x, w, bias, init = _f64(x), _f64(weight), _f64(bias), _f64(initial_states)
    batch, dim, seqlen = x.shape
    width = w.shape[1]
    if init is None:
        init = np.zeros((batch, dim, width - 1))
    xf = np.concatenate([init, x], axis=-1)
    mask = _tap_mask(seq_idx, width, seqlen)
    out = np.zeros((batch, dim, seqlen))
    for k in range(width):
        tap = w[None, :, k, None] * xf[:, :, k:k + seqlen]
        out += tap if mask is None else tap * mask[:, :, k]
    if bias is not None:
        out += bias[None, :, None]
    if activation in ("silu", "swish"):
        out = out * sigmoid(out)
    return out, xf[:, :, xf.shape[-1] - (width - 1):]


def causal_conv1d_bwd(x, weight, bias=None, initial_states=None, dout=None, activation=None,
                      dfinal_states=None, seq_idx=None):
    """Backward of causal_conv1d_fwd, from the chain rule:
        pre_t = bias + sum_k w[k] x_full[t+k] ; dpre = dout * act'(pre)
        dx_full[s] += w[k] dpre[s-k] ; dw[k] = sum_{b,t} dpre[t] x_full[t+k] ; dbias = sum dpre
    Returns (dx, dweight, dbias, dinitial_states); dbias / dinitial_states are
    None when bias / initial_states are None."""
    x, w, bias_, init = _f64(x), _f64(weight), _f64(bias), _f64(initial_states)
    dout = _f64(dout)
    batch, dim, seqlen = x.shape
    width = w.shape[1]
    init_ = np.zeros((batch, dim, width - 1)) if init is None else init
    xf = np.concatenate([init_, x], axis=-1)
    mask = _tap_mask(seq_idx, width, seqlen)
    one = np.ones((1, 1, seqlen))
    pre = np.zeros((batch, dim, seqlen))
    for k in range(width):
        pre += w[None, :, k, None] * xf[:, :, k:k + seqlen] * (one if mask is None else mask[:, :, k])
    if bias_ is not None:
        pre += bias_[None, :, None]
    if activation in ("silu", "swish"):
        s = sigmoid(pre)
        dpre = dout * s * (1 + pre * (1 - s))
    else:
        dpre = dout
    dxf = np.zeros_like(xf)
    dw = np.zeros_like(w)
    for k in range(width):
        dpk = dpre if mask is None else dpre * mask[:, :, k]
        dxf[:, :, k:k + seqlen] += w[None, :, k, None] * dpk
        dw[:, k] = (dpk * xf[:, :, k:k + seqlen]).sum((0, 2))
    if dfinal_states is not None:
        dxf[:, :, xf.shape[-1] - (width - 1):] += _f64(dfinal_states)
    dbias = None if bias_ is None else dpre.sum((0, 2))
    dinit = None if init is None else dxf[:, :, :width - 1]
    return dxf[:, :, width - 1:], dw, dbias, dinit


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
                         conv_state_indices=None):
    """Decode step(s) (src/mamba_cpu/ops/causal_conv1d.py:56-85):
        x_full = [conv_state, x] ; new_state = x_full[..., -state_len:]
        out = conv over the last seqlen + width - 1 columns
    x: (b, d) or (b, d, s). Returns (out shaped like x, new conv_state).

    The continuous-batching arguments the reference rejects (:66-67) follow
    the upstream causal_conv1d package's published semantics:
      conv_state_indices (b,): row b uses conv_state[conv_state_indices[b]]
        (conv_state may have more rows); an index out of range skips the row
        (zero output, state untouched);
      cache_seqlens (b,): conv_state is a ring buffer; the width - 1 inputs
        before x are at (cache_seqlens - (width - 1) + k) % state_len, and x[s]
        is written at (cache_seqlens + s) % state_len."""
    x, st, w, bias = _f64(x), _f64(conv_state), _f64(weight), _f64(bias)
    single = x.ndim == 2
    xs = x[..., None] if single else x
    batch, _, seqlen = xs.shape
    width = w.shape[1]
    state_len = st.shape[-1]
    new_state = st.copy()
    out = np.zeros(xs.shape)
    for b in range(batch):
        row = b if conv_state_indices is None else int(conv_state_indices[b])
        if not 0 <= row < st.shape[0]:
            continue
        if cache_seqlens is None:
            xf = np.concatenate([st[row], xs[b]], axis=-1)
            new_state[row] = xf[:, xf.shape[-1] - state_len:]
            hist = st[row][:, state_len - (width - 1):]
        else:
            cs = int(cache_seqlens[b])
            hist = st[row][:, [(cs - (width - 1) + k) % state_len for k in range(width - 1)]]
            for t in range(seqlen):
                new_state[row][:, (cs + t) % state_len] = xs[b][:, t]
        win = np.concatenate([hist, xs[b]], axis=-1)  # (d, width - 1 + seqlen)
        for k in range(width):
            out[b] += w[:, k, None] * win[:, k:k + seqlen]
        if bias is not None:
            out[b] += bias[:, None]
        if activation in ("silu", "swish"):
            out[b] = out[b] * sigmoid(out[b])
    return (out[..., 0] if single else out), new_state


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False,
                           state_batch_indices=None):
    """One decode step (src/mamba_cpu/ops/selective_state_update.py:5-57):
        dt = softplus?(dt + dt_bias) ; state = state * exp(dt A) + dt x B
        out = <state, C> + D x ; out *= silu(z)
    Mamba-1 layout: state (b, d, n), x/dt/z (b, d), A (d, n), B/C (b, n), D/dt_bias (d).
    Mamba-2 layout: state (b, h, p, n), x/dt/z (b, h, p), A (h, p, n),
    B/C (b, g, n), D/dt_bias (h, p); heads split into contiguous groups.
    state_batch_indices (b,), which the reference rejects (:24-25), follows
    mamba_ssm's semantics: row b updates state[state_batch_indices[b]] (state
    may have more rows); an index out of range skips the row (zero output).
    Returns (out shaped like x, new state)."""
    if state_batch_indices is not None:
        full = _f64(state).copy()
        idx = [int(i) for i in state_batch_indices]
        ok = [0 <= i < full.shape[0] for i in idx]
        rows = [i if k else 0 for i, k in zip(idx, ok)]
        out, upd = selective_state_update(full[rows], x, dt, A, B, C, D, z, dt_bias, dt_softplus)
        for b, (i, k) in enumerate(zip(idx, ok)):
            if k:
                full[i] = upd[b]
            else:
                out[b] = 0.0
        return out, full
    state, x, dt, A = _f64(state), _f64(x), _f64(dt), _f64(A)
    B, C, D, z, dt_bias = _f64(B), _f64(C), _f64(D), _f64(z), _f64(dt_bias)
    heads = state.ndim > 3
    if not heads:
        state, x, dt, A = state[:, None], x[:, None], dt[:, None], A[None]
        B, C = B[:, None], C[:, None]
        D = None if D is None else D[None]
        z = None if z is None else z[:, None]
        dt_bias = None if dt_bias is None else dt_bias[None]
    nheads = state.shape[1]
    if dt_bias is not None:
        dt = dt + dt_bias[None]
    if dt_softplus:
        dt = softplus(dt)
    with np.errstate(over="ignore", invalid="ignore"):
        dA = np.exp(dt[..., None] * A[None])
        Bh = np.repeat(B, nheads // B.shape[1], axis=1)  # (b, h, n)
        Ch = np.repeat(C, nheads // C.shape[1], axis=1)
        new_state = state * dA + (dt * x)[..., None] * Bh[:, :, None, :]
        out = (new_state * Ch[:, :, None, :]).sum(-1)
        if D is not None:
            out = out + x * D[None]
        if z is not None:
            out = out * z * sigmoid(z)
    if not heads:
        out, new_state = out[:, 0], new_state[:, 0]
    return out, new_state

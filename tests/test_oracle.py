"""Pins the float64 oracle (oracle/numerics.py) — CPU only, no GPU.

Each oracle function is checked against something it was not derived from:
  * the reference's own C++ kernels, compiled from the reference sources into
    oracle/_ref/libmcpu_ref.so (scan forward and backward);
  * closed forms and brute force (delta = 0, A = -inf, a scalar recurrence
    written out by hand, NaN confinement);
  * torch.autograd through an independent float64 torch forward, and central
    finite differences (scan backward, conv backward);
  * numpy.convolve (conv forward) and the reference tests' invariants (state
    chaining, update == full conv, step == scan, heads == flattened).
The last test plants mistakes in copies of oracle functions and checks that
these comparisons catch them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import numerics as O
from oracle import ref as R

needs_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built (make -C oracle)")


def scan_case(batch, dim, seqlen, dstate, ngroups, full, seed=0, A_scale=1.0):
    rng = np.random.default_rng(seed)
    bc = (batch, dstate, seqlen) if ngroups is None else (batch, ngroups, dstate, seqlen)
    return dict(
        u=rng.standard_normal((batch, dim, seqlen)),
        delta=rng.random((batch, dim, seqlen)) * 0.5,
        A=-(rng.random((dim, dstate)) * A_scale + 0.5),
        B=rng.standard_normal(bc),
        C=rng.standard_normal(bc),
        D=rng.standard_normal(dim) if full else None,
        z=rng.standard_normal((batch, dim, seqlen)) if full else None,
        delta_bias=rng.random(dim) * 0.1 if full else None,
    )


def f32(d):
    return {k: None if v is None else v.astype(np.float32).astype(np.float64) for k, v in d.items()}


SHAPES = [(1, 4, 1, 1), (2, 16, 33, 16), (3, 32, 70, 8), (2, 8, 17, 4)]


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("ngroups", [None, 2])
@pytest.mark.parametrize("full,softplus", [(False, False), (True, True), (True, False)])
def test_scan_fwd_matches_reference_build(shape, ngroups, full, softplus):
    b, d, l, n = shape
    if ngroups and d % ngroups:
        pytest.skip("dim not divisible")
    inp = f32(scan_case(b, d, l, n, ngroups, full))
    out, last = O.selective_scan_fwd(**inp, delta_softplus=softplus)
    ro, rl = R.scan_fwd(inp["u"], inp["delta"], inp["A"], R.kernel_bc(inp["B"]), R.kernel_bc(inp["C"]),
                        inp["D"], inp["z"], inp["delta_bias"], softplus)
    np.testing.assert_allclose(out, ro, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(last, rl, rtol=1e-4, atol=2e-5)


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("ngroups", [None, 2])
@pytest.mark.parametrize("full,softplus", [(False, False), (True, True)])
@pytest.mark.parametrize("with_dlast", [False, True])
def test_scan_bwd_matches_reference_build(shape, ngroups, full, softplus, with_dlast):
    b, d, l, n = shape
    if ngroups and d % ngroups:
        pytest.skip("dim not divisible")
    inp = f32(scan_case(b, d, l, n, ngroups, full))
    rng = np.random.default_rng(7)
    dout = rng.standard_normal((b, d, l)).astype(np.float32).astype(np.float64)
    dlast = rng.standard_normal((b, d, n)).astype(np.float32).astype(np.float64) if with_dlast else None
    got = O.selective_scan_bwd(**inp, delta_softplus=softplus, dout=dout, dlast_state=dlast)
    ref = R.scan_bwd(inp["u"], inp["delta"], inp["A"], R.kernel_bc(inp["B"]), R.kernel_bc(inp["C"]),
                     inp["D"], inp["z"], inp["delta_bias"], softplus, dout, dlast)
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias"]
    for name, g, r in zip(names, got, ref):
        if g is None:
            continue
        if name in ("dB", "dC"):
            r = np.swapaxes(r, -1, -2)
            if ngroups is None:
                r = r[:, 0]
        scale = max(np.abs(r).max(), 1.0)
        np.testing.assert_allclose(g / scale, r / scale, rtol=1e-4, atol=2e-5, err_msg=name)


def test_scan_delta_zero_is_skip_connection():
    inp = scan_case(2, 6, 9, 4, None, True)
    inp["delta"][:] = 0.0
    inp["delta_bias"] = None
    out, last = O.selective_scan_fwd(**inp, delta_softplus=False)
    u, D, z = inp["u"], inp["D"], inp["z"]
    np.testing.assert_allclose(out, D[None, :, None] * u * z / (1 + np.exp(-z)), rtol=1e-12, atol=1e-12)
    assert not last.any()


def test_scan_infinite_decay_is_memoryless():
    inp = scan_case(1, 5, 7, 3, None, False)
    inp["A"][:] = -np.inf
    out, last = O.selective_scan_fwd(**inp)
    dt, u, B, C = inp["delta"], inp["u"], inp["B"], inp["C"]
    want = dt * u * np.einsum("bnl,bnl->bl", B, C)[:, None, :]
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(last, (dt * u)[:, :, -1, None] * B[:, None, :, -1], rtol=1e-12)


def test_scan_scalar_recurrence_by_hand():
    rng = np.random.default_rng(3)
    L = 6
    u, delta, z = rng.standard_normal(L), rng.standard_normal(L), rng.standard_normal(L)
    A, D, bias = -0.7, 0.3, 0.25
    Bv, Cv = rng.standard_normal(L), rng.standard_normal(L)
    h, ys = 0.0, []
    for t in range(L):
        x = delta[t] + bias
        dt = math.log1p(math.exp(x)) if x <= 20 else x
        h = math.exp(dt * A) * h + dt * u[t] * Bv[t]
        y = h * Cv[t] + D * u[t]
        ys.append(y * z[t] / (1 + math.exp(-z[t])))
    out, last = O.selective_scan_fwd(u[None, None], delta[None, None], np.array([[A]]), Bv[None, None],
                                     Cv[None, None], np.array([D]), z[None, None], np.array([bias]), True)
    np.testing.assert_allclose(out[0, 0], ys, rtol=1e-13)
    assert abs(last[0, 0, 0] - h) < 1e-13


def test_scan_nan_confined():
    inp = scan_case(1, 4, 5, 3, None, False)
    inp["delta"][0, 2, 1] = np.nan
    out, _ = O.selective_scan_fwd(**inp)
    assert np.isnan(out[0, 2, 1:]).all() and not np.isnan(out[0, 2, :1]).any()
    assert not np.isnan(out[0, [0, 1, 3]]).any()


def torch_scan_f64(u, delta, A, B, C, D, z, bias, softplus):
    """Independent float64 forward in torch (autograd derives the backward)."""
    dt = delta + bias[:, None] if bias is not None else delta
    dt = F.softplus(dt) if softplus else dt
    Bg = B if B.dim() == 4 else B[:, None]
    Cg = C if C.dim() == 4 else C[:, None]
    rep = u.shape[1] // Bg.shape[1]
    Bd, Cd = Bg.repeat_interleave(rep, 1), Cg.repeat_interleave(rep, 1)
    h = u.new_zeros(u.shape[0], u.shape[1], A.shape[1])
    ys = []
    for t in range(u.shape[-1]):
        h = torch.exp(dt[..., t, None] * A) * h + (dt[..., t] * u[..., t])[..., None] * Bd[..., t]
        ys.append((h * Cd[..., t]).sum(-1))
    y = torch.stack(ys, -1)
    if D is not None:
        y = y + D[:, None] * u
    if z is not None:
        y = y * F.silu(z)
    return y, h


@pytest.mark.parametrize("ngroups", [None, 2])
@pytest.mark.parametrize("full,softplus", [(True, True), (False, False)])
def test_scan_bwd_matches_autograd(ngroups, full, softplus):
    inp = scan_case(2, 6, 11, 5, ngroups, full, seed=4)
    rng = np.random.default_rng(5)
    W = rng.standard_normal(inp["u"].shape)
    V = rng.standard_normal((2, 6, 5))
    t = {k: None if v is None else torch.tensor(v, requires_grad=True) for k, v in inp.items()}
    out, last = torch_scan_f64(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["z"],
                               t["delta_bias"], softplus)
    ((out * torch.tensor(W)).sum() + (last * torch.tensor(V)).sum()).backward()
    got = O.selective_scan_bwd(**inp, delta_softplus=softplus, dout=W, dlast_state=V)
    for name, g in zip(["u", "delta", "A", "B", "C", "D", "z", "delta_bias"], got):
        if t[name] is None:
            assert g is None
            continue
        np.testing.assert_allclose(g, t[name].grad.numpy(), rtol=1e-10, atol=1e-10, err_msg=name)


def test_scan_bwd_matches_finite_differences():
    inp = scan_case(1, 2, 5, 3, None, True, seed=9)
    rng = np.random.default_rng(10)
    W = rng.standard_normal(inp["u"].shape)

    def loss(d):
        out, _ = O.selective_scan_fwd(**d, delta_softplus=True)
        return float((out * W).sum())

    grads = O.selective_scan_bwd(**inp, delta_softplus=True, dout=W)
    eps = 1e-6
    for name, g in zip(["u", "delta", "A", "B", "C", "D", "z", "delta_bias"], grads):
        flat = inp[name].reshape(-1)
        fd = np.zeros_like(flat)
        for i in range(flat.size):
            old = flat[i]
            flat[i] = old + eps
            lp = loss(inp)
            flat[i] = old - eps
            lm = loss(inp)
            flat[i] = old
            fd[i] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(g.reshape(-1), fd, rtol=1e-5, atol=1e-6, err_msg=name)


@pytest.mark.parametrize("width", [1, 2, 3, 4, 7])
@pytest.mark.parametrize("with_init", [False, True])
def test_conv_fwd_matches_numpy_convolve(width, with_init):
    rng = np.random.default_rng(width)
    b, d, l = 2, 3, 13
    x, w, bias = rng.standard_normal((b, d, l)), rng.standard_normal((d, width)), rng.standard_normal(d)
    init = rng.standard_normal((b, d, width - 1)) if with_init else None
    out, final = O.causal_conv1d_fwd(x, w, bias, init, activation=None)
    for bi in range(b):
        for di in range(d):
            xf = np.concatenate([init[bi, di] if with_init else np.zeros(width - 1), x[bi, di]])
            # out[t] = sum_k w[k] xf[t + k]: a "valid" correlation = convolution with w reversed
            want = np.convolve(xf, w[di][::-1], mode="valid") + bias[di]
            np.testing.assert_allclose(out[bi, di], want, rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(final[bi, di], xf[len(xf) - (width - 1):])
    out_silu, _ = O.causal_conv1d_fwd(x, w, bias, init, activation="silu")
    np.testing.assert_allclose(out_silu, out / (1 + np.exp(-out)), rtol=1e-12)


@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("with_init", [False, True])
def test_conv_bwd_matches_autograd(activation, with_init):
    rng = np.random.default_rng(1)
    b, d, l, width = 2, 3, 9, 4
    x, w, bias = rng.standard_normal((b, d, l)), rng.standard_normal((d, width)), rng.standard_normal(d)
    init = rng.standard_normal((b, d, width - 1)) if with_init else None
    G, Gf = rng.standard_normal((b, d, l)), rng.standard_normal((b, d, width - 1))
    tx, tw, tb = (torch.tensor(v, requires_grad=True) for v in (x, w, bias))
    ti = torch.tensor(init, requires_grad=True) if with_init else None
    xf = torch.cat([ti if with_init else torch.zeros(b, d, width - 1, dtype=torch.float64), tx], -1)
    out = F.conv1d(xf, tw.unsqueeze(1), tb, groups=d)
    if activation:
        out = F.silu(out)
    final = xf[..., -(width - 1):]
    ((out * torch.tensor(G)).sum() + (final * torch.tensor(Gf)).sum()).backward()
    dx, dw, db, dinit = O.causal_conv1d_bwd(x, w, bias, init, G, activation, Gf)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-10, atol=1e-12)
    if with_init:
        np.testing.assert_allclose(dinit, ti.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_conv_states_chain_and_update_invariants():
    rng = np.random.default_rng(2)
    x, w, bias = rng.standard_normal((2, 4, 20)), rng.standard_normal((4, 4)), rng.standard_normal(4)
    full, _ = O.causal_conv1d_fwd(x, w, bias, activation="silu")
    a, st = O.causal_conv1d_fwd(x[..., :8], w, bias, activation="silu")
    b, _ = O.causal_conv1d_fwd(x[..., 8:], w, bias, initial_states=st, activation="silu")
    np.testing.assert_allclose(np.concatenate([a, b], -1), full, rtol=1e-12)
    for state_len in (3, 5):
        state = np.zeros((2, 4, state_len))
        outs = []
        for t in range(20):
            o, state = O.causal_conv1d_update(x[..., t], state, w, bias, "silu")
            outs.append(o)
        np.testing.assert_allclose(np.stack(outs, -1), full, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(state, x[..., -state_len:])
        state = np.zeros((2, 4, state_len))
        _, state = O.causal_conv1d_update(x[..., :15], state, w, bias)
        o, state = O.causal_conv1d_update(x[..., 15:], state, w, bias, "silu")
        np.testing.assert_allclose(o, full[..., 15:], rtol=1e-12, atol=1e-12)


def test_state_update_steps_equal_scan():
    inp = scan_case(2, 6, 8, 4, None, True, seed=11)
    full, last = O.selective_scan_fwd(**inp, delta_softplus=True)
    state = np.zeros((2, 6, 4))
    outs = []
    for t in range(8):
        o, state = O.selective_state_update(state, inp["u"][..., t], inp["delta"][..., t], inp["A"],
                                            inp["B"][..., t], inp["C"][..., t], inp["D"],
                                            inp["z"][..., t], inp["delta_bias"], True)
        outs.append(o)
    np.testing.assert_allclose(np.stack(outs, -1), full, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(state, last, rtol=1e-12, atol=1e-12)


def test_state_update_heads_equal_flattened():
    rng = np.random.default_rng(12)
    b, h, p, n = 2, 4, 3, 5
    state = rng.standard_normal((b, h, p, n))
    x, dt = rng.standard_normal((b, h, p)), rng.random((b, h, p))
    A, D = -rng.random((h, p, n)), rng.standard_normal((h, p))
    B, C = rng.standard_normal((b, 1, n)), rng.standard_normal((b, 1, n))
    o1, s1 = O.selective_state_update(state, x, dt, A, B, C, D)
    o2, s2 = O.selective_state_update(state.reshape(b, -1, n), x.reshape(b, -1), dt.reshape(b, -1),
                                      A.reshape(-1, n), B[:, 0], C[:, 0], D.reshape(-1))
    np.testing.assert_allclose(o1.reshape(b, -1), o2, rtol=1e-13)
    np.testing.assert_allclose(s1.reshape(b, -1, n), s2, rtol=1e-13)


@needs_ref
def test_planted_mistakes_are_caught():
    """Copies of the oracle with a plausible mistake must fail the comparisons above."""
    inp = f32(scan_case(2, 8, 12, 4, None, True))
    ro, _ = R.scan_fwd(inp["u"], inp["delta"], inp["A"], R.kernel_bc(inp["B"]), R.kernel_bc(inp["C"]),
                       inp["D"], inp["z"], inp["delta_bias"], True)
    # (1) B and C swapped, (2) D-skip dropped, (3) softplus missing
    bad = [
        O.selective_scan_fwd(**{**inp, "B": inp["C"], "C": inp["B"]}, delta_softplus=True)[0],
        O.selective_scan_fwd(**{**inp, "D": None}, delta_softplus=True)[0],
        O.selective_scan_fwd(**inp, delta_softplus=False)[0],
    ]
    for out in bad:
        assert not np.allclose(out, ro, rtol=1e-4, atol=2e-5)
    # (4) a sign error in the backward's dA term
    dout = np.random.default_rng(3).standard_normal(inp["u"].shape)
    ref = R.scan_bwd(inp["u"], inp["delta"], inp["A"], R.kernel_bc(inp["B"]), R.kernel_bc(inp["C"]),
                     inp["D"], inp["z"], inp["delta_bias"], True, dout)
    got = O.selective_scan_bwd(**inp, delta_softplus=True, dout=dout)
    assert np.allclose(got[2], ref[2], rtol=1e-4, atol=1e-5)
    assert not np.allclose(-got[2], ref[2], rtol=1e-4, atol=1e-5)
    # (5) a conv with taps in the wrong order
    rng = np.random.default_rng(4)
    x, w = rng.standard_normal((1, 2, 9)), rng.standard_normal((2, 3))
    out, _ = O.causal_conv1d_fwd(x, w[:, ::-1])
    xf = np.concatenate([np.zeros(2), x[0, 0]])
    assert not np.allclose(out[0, 0], np.convolve(xf, w[0][::-1], mode="valid"))


def test_conv_update_indices_and_ring_buffer_invariants():
    """Pins the continuous-batching arguments of the conv update oracle:
    identity indices change nothing; permuted indices update the selected rows
    only; an out-of-range index skips its row; a ring buffer stepped with
    cache_seqlens = t gives the linear update's outputs, and its contents are
    the linear state rotated by t."""
    rng = np.random.default_rng(21)
    b, d, w, S, T = 3, 4, 4, 5, 11
    x = rng.standard_normal((b, d, T))
    wt, bias = rng.standard_normal((d, w)), rng.standard_normal(d)
    st0 = rng.standard_normal((b, d, S))
    o1, s1 = O.causal_conv1d_update(x[..., 0], st0, wt, bias, "silu")
    o2, s2 = O.causal_conv1d_update(x[..., 0], st0, wt, bias, "silu", conv_state_indices=np.arange(b))
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(s1, s2)
    big = rng.standard_normal((6, d, S))
    idx = np.array([4, 0, 2])
    o3, s3 = O.causal_conv1d_update(x[..., :2], big, wt, bias, "silu", conv_state_indices=idx)
    o4, s4 = O.causal_conv1d_update(x[..., :2], big[idx], wt, bias, "silu")
    np.testing.assert_allclose(o3, o4, rtol=1e-13)
    np.testing.assert_allclose(s3[idx], s4, rtol=1e-13)
    untouched = [i for i in range(6) if i not in idx]
    np.testing.assert_array_equal(s3[untouched], big[untouched])
    o5, s5 = O.causal_conv1d_update(x[..., :2], big, wt, bias, "silu", conv_state_indices=np.array([4, -1, 9]))
    np.testing.assert_allclose(o5[0], o4[0], rtol=1e-13)
    assert (o5[1:] == 0).all()
    np.testing.assert_array_equal(s5[[0, 1, 2, 3, 5]], big[[0, 1, 2, 3, 5]])
    # Ring buffer vs linear, one token at a time, then two tokens at once.
    lin, ring = st0.copy(), np.zeros((b, d, S))
    ring[..., :] = st0  # ring slots 0..S-1 hold the state with cache_seqlens = 0 meaning "next write at 0"
    outs_l, outs_r = [], []
    for t in range(T):
        ol, lin = O.causal_conv1d_update(x[..., t], lin, wt, bias, "silu")
        orr, ring = O.causal_conv1d_update(x[..., t], ring, wt, bias, "silu",
                                           cache_seqlens=np.full(b, t))
        outs_l.append(ol)
        outs_r.append(orr)
    np.testing.assert_allclose(np.stack(outs_r, -1), np.stack(outs_l, -1), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(lin, np.roll(ring, -(T % S), axis=-1), rtol=0, atol=0)
    o6, r6 = O.causal_conv1d_update(x[..., :2], ring, wt, bias, "silu", cache_seqlens=np.full(b, T))
    o7, l7 = O.causal_conv1d_update(x[..., :2], lin, wt, bias, "silu")
    np.testing.assert_allclose(o6, o7, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(l7, np.roll(r6, -((T + 2) % S), axis=-1), rtol=0, atol=0)


def test_state_update_batch_indices_invariants():
    rng = np.random.default_rng(22)
    b, d, n = 3, 5, 4
    x, dt, z = rng.standard_normal((b, d)), rng.random((b, d)), rng.standard_normal((b, d))
    A, D, dtb = -rng.random((d, n)), rng.standard_normal(d), rng.random(d)
    B, C = rng.standard_normal((b, n)), rng.standard_normal((b, n))
    big = rng.standard_normal((7, d, n))
    idx = np.array([6, 1, 3])
    o1, s1 = O.selective_state_update(big, x, dt, A, B, C, D, z, dtb, True, state_batch_indices=idx)
    o2, s2 = O.selective_state_update(big[idx], x, dt, A, B, C, D, z, dtb, True)
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(s1[idx], s2)
    rest = [0, 2, 4, 5]
    np.testing.assert_array_equal(s1[rest], big[rest])
    o3, s3 = O.selective_state_update(big, x, dt, A, B, C, D, z, dtb, True,
                                      state_batch_indices=np.array([6, 7, -2]))
    np.testing.assert_array_equal(o3[0], o2[0])
    assert (o3[1:] == 0).all()
    np.testing.assert_array_equal(s3[:6], big[:6])


def test_scan_unequal_groups_and_2d_bc_equal_expanded():
    """Pins the oracle's extensions beyond the reference's kernels (which take
    one group count for both B and C, and no 2-D B/C): B and C with different
    group counts equal both repeated to a common count; a 2-D (dim, dstate)
    B or C equals the (batch, dim, dstate, seqlen) tensor repeating it at
    every step, and its gradient is that tensor's gradient summed over batch
    and time."""
    inp = scan_case(2, 12, 9, 4, None, True, seed=31)
    rng = np.random.default_rng(32)
    B1 = rng.standard_normal((2, 1, 4, 9))
    C3 = rng.standard_normal((2, 3, 4, 9))
    G = rng.standard_normal((2, 12, 9))
    base = {k: inp[k] for k in ("u", "delta", "A", "D", "z", "delta_bias")}
    out_u, last_u = O.selective_scan_fwd(**base, B=B1, C=C3, delta_softplus=True)
    out_e, last_e = O.selective_scan_fwd(**base, B=np.repeat(B1, 3, axis=1), C=C3, delta_softplus=True)
    np.testing.assert_allclose(out_u, out_e, rtol=1e-13)
    np.testing.assert_allclose(last_u, last_e, rtol=1e-13)
    gu = O.selective_scan_bwd(**base, B=B1, C=C3, delta_softplus=True, dout=G)
    ge = O.selective_scan_bwd(**base, B=np.repeat(B1, 3, axis=1), C=C3, delta_softplus=True, dout=G)
    for i in (0, 1, 2, 4, 5, 6, 7):
        np.testing.assert_allclose(gu[i], ge[i], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(gu[3], ge[3].reshape(2, 1, 3, 4, 9).sum(2), rtol=1e-12)
    # 2-D B and C
    B2, C2 = rng.standard_normal((12, 4)), rng.standard_normal((12, 4))
    B4 = np.broadcast_to(B2[None, :, :, None], (2, 12, 4, 9)).copy()
    C4 = np.broadcast_to(C2[None, :, :, None], (2, 12, 4, 9)).copy()
    for Bx, Cx, Be, Ce in ((B2, C3, B4, C3), (B1, C2, B1, C4), (B2, C2, B4, C4)):
        o2, _ = O.selective_scan_fwd(**base, B=Bx, C=Cx, delta_softplus=True)
        o4, _ = O.selective_scan_fwd(**base, B=Be, C=Ce, delta_softplus=True)
        np.testing.assert_allclose(o2, o4, rtol=1e-13)
        g2 = O.selective_scan_bwd(**base, B=Bx, C=Cx, delta_softplus=True, dout=G)
        g4 = O.selective_scan_bwd(**base, B=Be, C=Ce, delta_softplus=True, dout=G)
        for i in (0, 1, 2, 5, 6, 7):
            np.testing.assert_allclose(g2[i], g4[i], rtol=1e-12, atol=1e-14)
        for i, X in ((3, Bx), (4, Cx)):
            want = g4[i].sum((0, 3)) if X.ndim == 2 else g4[i]
            np.testing.assert_allclose(g2[i], want, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("activation", [None, "silu"])
def test_conv_seq_idx_equals_separate_sequences(activation):
    """Pins the seq_idx extension of the conv oracle: packed sequences give the
    outputs and input gradients of each sequence convolved on its own (zero
    history), and the weight/bias gradients are the sums over them."""
    rng = np.random.default_rng(41)
    b, d, l, w = 2, 3, 17, 4
    x, wt, bias = rng.standard_normal((b, d, l)), rng.standard_normal((d, w)), rng.standard_normal(d)
    G = rng.standard_normal((b, d, l))
    cuts = [[0, 5, 6, 17], [0, 11, 17]]
    seq = np.zeros((b, l), dtype=np.int32)
    for bi, c in enumerate(cuts):
        for si in range(len(c) - 1):
            seq[bi, c[si]:c[si + 1]] = si + 3 * bi
    out, _ = O.causal_conv1d_fwd(x, wt, bias, activation=activation, seq_idx=seq)
    dx, dw, db, _ = O.causal_conv1d_bwd(x, wt, bias, dout=G, activation=activation, seq_idx=seq)
    dw_sum, db_sum = np.zeros_like(dw), np.zeros_like(db)
    for bi, c in enumerate(cuts):
        for lo, hi in zip(c[:-1], c[1:]):
            o1, _ = O.causal_conv1d_fwd(x[bi:bi + 1, :, lo:hi], wt, bias, activation=activation)
            np.testing.assert_allclose(out[bi:bi + 1, :, lo:hi], o1, rtol=1e-13)
            g1 = O.causal_conv1d_bwd(x[bi:bi + 1, :, lo:hi], wt, bias, dout=G[bi:bi + 1, :, lo:hi],
                                     activation=activation)
            np.testing.assert_allclose(dx[bi:bi + 1, :, lo:hi], g1[0], rtol=1e-12, atol=1e-14)
            dw_sum += g1[1]
            db_sum += g1[2]
    np.testing.assert_allclose(dw, dw_sum, rtol=1e-12)
    np.testing.assert_allclose(db, db_sum, rtol=1e-12)


# ---- complex A (mamba_ssm's semantics; the reference rejects complex A) ----

def complex_case(batch, dim, seqlen, dstate, ngroups, seed=0, bc2d=False):
    """Complex-A inputs: A complex (dim, dstate) with negative real parts;
    B/C real (b[, g], n, 2 l) with (re, im) pairs along the last dim, or
    complex (dim, dstate) when bc2d."""
    rng = np.random.default_rng(seed)
    bc = (batch, dstate, 2 * seqlen) if ngroups is None else (batch, ngroups, dstate, 2 * seqlen)
    cplx = lambda *s: rng.standard_normal(s) + 1j * rng.standard_normal(s)  # noqa: E731
    return dict(
        u=rng.standard_normal((batch, dim, seqlen)),
        delta=rng.random((batch, dim, seqlen)) * 0.5,
        A=-(rng.random((dim, dstate)) + 0.5) + 1j * rng.standard_normal((dim, dstate)) * 3,
        B=cplx(dim, dstate) if bc2d else rng.standard_normal(bc),
        C=rng.standard_normal(bc),
        D=rng.standard_normal(dim),
        z=rng.standard_normal((batch, dim, seqlen)),
        delta_bias=rng.random(dim) * 0.1,
    )


def _complex_direct_sum(u, delta, A, B, C, D, z, delta_bias, softplus):
    """Torch float64/complex128 forward in closed form, no recurrence:
    h_t = sum_{s<=t} exp(A (S_t - S_s)) dt_s u_s B_s with S_t = sum_{r<=t} dt_r,
    out = (2 Re <h_t, C_t> + D u) silu(z). B/C as in complex_case (real
    interleaved pairs, or complex (dim, dstate)). Returns (out, last_state)."""
    b, d, l = u.shape
    dt = delta + delta_bias[None, :, None]
    dt = F.softplus(dt) if softplus else dt

    def per_channel(X):
        if X.is_complex():
            return X[None, :, :, None].expand(b, d, X.shape[1], l)
        X = X if X.dim() == 4 else X[:, None]
        Xc = torch.view_as_complex(X.reshape(*X.shape[:-1], l, 2).contiguous())
        return Xc.repeat_interleave(d // Xc.shape[1], dim=1)  # (b, d, n, l)

    Bf, Cf = per_channel(B), per_channel(C)
    S = torch.cumsum(dt, -1)
    diff = S[..., :, None] - S[..., None, :]  # (b, d, t, s)
    mask = torch.tril(torch.ones(l, l, dtype=torch.float64))
    K = torch.exp(diff[..., None] * A[None, :, None, None, :]) * mask[..., None]  # (b, d, t, s, n)
    x = (dt * u)[:, :, None, :, None] * Bf.permute(0, 1, 3, 2)[:, :, None]  # (b, d, 1, s, n)
    h = (K * x).sum(3)  # (b, d, t, n)
    y = 2 * (h * Cf.permute(0, 1, 3, 2)).sum(-1).real + D[None, :, None] * u
    return y * F.silu(z), h[:, :, -1]


@pytest.mark.parametrize("ngroups,bc2d", [(None, False), (2, False), (None, True)])
def test_complex_scan_fwd_equals_direct_sum(ngroups, bc2d):
    inp = complex_case(2, 4, 9, 3, ngroups, seed=51, bc2d=bc2d)
    out, last = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    t = {k: torch.from_numpy(v) for k, v in inp.items()}
    want, want_last = _complex_direct_sum(**t, softplus=True)
    np.testing.assert_allclose(out, want.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(last, want_last.numpy(), rtol=1e-11, atol=1e-12)


def test_complex_scan_real_case_and_phase_invariance():
    """A with zero imaginary part and real B, C reduce to the real scan with C
    doubled (y = 2 Re <h, C>); rotating state n's B by exp(i phi_n) and C by
    exp(-i phi_n) leaves the output unchanged."""
    rng = np.random.default_rng(52)
    r = scan_case(2, 4, 11, 3, None, True, seed=52)
    inter = lambda X: np.stack([X, np.zeros_like(X)], -1).reshape(*X.shape[:-1], -1)  # noqa: E731
    out, last = O.selective_scan_fwd_complex(r["u"], r["delta"], r["A"] + 0j, inter(r["B"]), inter(r["C"]),
                                             r["D"], r["z"], r["delta_bias"], True)
    want, want_last = O.selective_scan_fwd(r["u"], r["delta"], r["A"], r["B"], 2 * r["C"], r["D"], r["z"],
                                           r["delta_bias"], True)
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(last.real, want_last, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(last.imag, 0, atol=0)

    inp = complex_case(2, 4, 11, 3, None, seed=53)
    phi = rng.random(3) * 2 * np.pi

    def rotate(X, sign):
        Xc = X[..., 0::2] + 1j * X[..., 1::2]
        Xc = Xc * np.exp(sign * 1j * phi)[:, None]
        return np.stack([Xc.real, Xc.imag], -1).reshape(X.shape)

    out0, _ = O.selective_scan_fwd_complex(**inp, delta_softplus=True)
    out1, _ = O.selective_scan_fwd_complex(**{**inp, "B": rotate(inp["B"], 1), "C": rotate(inp["C"], -1)},
                                           delta_softplus=True)
    np.testing.assert_allclose(out1, out0, rtol=1e-11, atol=1e-12)
    # the same rotation of B and C together is not an invariance
    out2, _ = O.selective_scan_fwd_complex(**{**inp, "B": rotate(inp["B"], 1), "C": rotate(inp["C"], 1)},
                                           delta_softplus=True)
    assert not np.allclose(out2, out0, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("ngroups,bc2d", [(None, False), (2, False), (None, True)])
def test_complex_scan_bwd_matches_autograd(ngroups, bc2d):
    """The analytic complex backward against torch.autograd through the
    closed-form forward (complex gradients: dLoss/dRe + i dLoss/dIm), with a
    gradient on the last state too."""
    inp = complex_case(2, 4, 8, 3, ngroups, seed=54, bc2d=bc2d)
    rng = np.random.default_rng(55)
    W = rng.standard_normal(inp["u"].shape)
    W2 = rng.standard_normal((2, 4, 3)) + 1j * rng.standard_normal((2, 4, 3))
    got = O.selective_scan_bwd_complex(**inp, delta_softplus=True, dout=W, dlast_state=W2)
    names = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).requires_grad_() for k, v in inp.items()}
    out, last = _complex_direct_sum(**t, softplus=True)
    loss = (out * torch.from_numpy(W)).sum() + (torch.conj(torch.from_numpy(W2)) * last).real.sum()
    want = torch.autograd.grad(loss, [t[k] for k in names])
    for k, g, w in zip(names, got, want):
        np.testing.assert_allclose(g, w.numpy(), rtol=1e-9, atol=1e-10, err_msg=k)


def test_complex_scan_planted_mistakes_are_caught():
    """Copies of the complex oracle with a plausible mistake fail the checks above:
    B's (re, im) pairs swapped, the factor 2 of y dropped, dA conjugated."""
    inp = complex_case(1, 3, 7, 2, None, seed=56)
    t = {k: torch.from_numpy(v) for k, v in inp.items()}
    want, _ = _complex_direct_sum(**t, softplus=True)
    swapped = inp["B"].reshape(1, 2, 7, 2)[..., ::-1].reshape(1, 2, 14)
    out, _ = O.selective_scan_fwd_complex(**{**inp, "B": swapped}, delta_softplus=True)
    assert not np.allclose(out, want.numpy(), rtol=1e-4, atol=1e-5)
    half, _ = O.selective_scan_fwd_complex(**{**inp, "C": inp["C"] / 2}, delta_softplus=True)
    assert not np.allclose(half, want.numpy(), rtol=1e-4, atol=1e-5)
    W = np.random.default_rng(57).standard_normal(inp["u"].shape)
    dA = O.selective_scan_bwd_complex(**inp, delta_softplus=True, dout=W)[2]
    tt = {k: torch.from_numpy(v).requires_grad_() for k, v in inp.items()}
    out, _ = _complex_direct_sum(**tt, softplus=True)
    (gA,) = torch.autograd.grad((out * torch.from_numpy(W)).sum(), [tt["A"]])
    np.testing.assert_allclose(dA, gA.numpy(), rtol=1e-9, atol=1e-10)
    assert not np.allclose(np.conj(dA), gA.numpy(), rtol=1e-4, atol=1e-5)

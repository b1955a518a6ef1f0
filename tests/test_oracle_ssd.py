"""Pins oracle/ssd.py (the float64 restatement of Mamba-2's SSD scan) on the
CPU, so the GPU tests of the SSD kernels check against something known:

- with A broadcast over a head's channels and states, the SSD scan is the
  Mamba-1 selective scan over dim = nheads * headdim channels (delta the
  head's dt on each of its channels, u = x), whose oracle is pinned against
  the reference's own kernels: outputs and every gradient agree;
- a quadratic direct sum, h_t = sum_{s<=t} exp(S_t - S_s) dt_s x_s B_s^T +
  exp(S_t) h_init with S the running sum of dt A, written in torch float64
  without a recurrence: outputs and final states agree, with initial states,
  dt_bias, softplus, dt_limit clamping, D per head or per channel, z and
  groups;
- torch.autograd through that direct sum: every gradient of ssd_bwd,
  including the initial states';
- a planted mistake in a copy of ssd_bwd (the decay term's dt dropped) fails
  the autograd check;
- packed sequences (seq_idx) against each sequence run on its own.
"""

import inspect
import math
import textwrap

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import numerics as O
from oracle import ssd as S


def ssd_case(b, l, h, p, n, g, seed=0, init=False, Dshape="hp", z=True, bias=True):
    rng = np.random.default_rng(seed)
    case = dict(x=rng.standard_normal((b, l, h, p)), dt=rng.standard_normal((b, l, h)) * 0.5 - 1.0,
                A=-np.exp(rng.random(h) * math.log(8)),
                B=rng.standard_normal((b, l, g, n)), C=rng.standard_normal((b, l, g, n)))
    case["D"] = None if Dshape is None else rng.standard_normal((h, p) if Dshape == "hp" else (h,))
    case["z"] = rng.standard_normal((b, l, h, p)) if z else None
    case["dt_bias"] = rng.random(h) * 0.5 if bias else None
    case["initial_states"] = rng.standard_normal((b, h, p, n)) if init else None
    return case


def as_mamba1(c):
    """The SSD case as a Mamba-1 scan over dim = h * p channels."""
    b, l, h, p = c["x"].shape
    g, n = c["B"].shape[2], c["B"].shape[3]
    u = c["x"].transpose(0, 2, 3, 1).reshape(b, h * p, l)
    delta = np.repeat(c["dt"].transpose(0, 2, 1), p, axis=1)
    A = np.repeat(c["A"][:, None], p, axis=0) * np.ones((1, n))
    Bm, Cm = c["B"].transpose(0, 2, 3, 1), c["C"].transpose(0, 2, 3, 1)
    D = None if c["D"] is None else np.broadcast_to(
        c["D"][:, None] if c["D"].ndim == 1 else c["D"], (h, p)).reshape(-1)
    z = None if c["z"] is None else c["z"].transpose(0, 2, 3, 1).reshape(b, h * p, l)
    bias = None if c["dt_bias"] is None else np.repeat(c["dt_bias"], p)
    return dict(u=u, delta=delta, A=A, B=Bm, C=Cm, D=D, z=z, delta_bias=bias)


@pytest.mark.parametrize("g,Dshape", [(1, "hp"), (2, "h"), (4, None)])
def test_ssd_equals_mamba1_with_broadcast_A(g, Dshape):
    c = ssd_case(2, 13, 4, 3, 5, g, seed=g, Dshape=Dshape)
    b, l, h, p = c["x"].shape
    out, last = S.ssd_fwd(**c, dt_softplus=True)
    m = as_mamba1(c)
    want, want_last = O.selective_scan_fwd(**m, delta_softplus=True)
    np.testing.assert_allclose(out.transpose(0, 2, 3, 1).reshape(b, h * p, l), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(last.reshape(b, h * p, -1), want_last, rtol=1e-12, atol=1e-12)
    rng = np.random.default_rng(9)
    dout = rng.standard_normal(out.shape)
    dfin = rng.standard_normal(last.shape)
    dx, ddt, dA, dB, dC, dD, dz, dbias, _ = S.ssd_bwd(**c, dt_softplus=True, dout=dout, dfinal_states=dfin)
    mg = O.selective_scan_bwd(**m, delta_softplus=True, dout=dout.transpose(0, 2, 3, 1).reshape(b, h * p, l),
                              dlast_state=dfin.reshape(b, h * p, -1))
    du, ddelta, dAm, dBm, dCm, dDm, dzm, dbm = mg
    tol = dict(rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(dx.transpose(0, 2, 3, 1).reshape(b, h * p, l), du, **tol)
    np.testing.assert_allclose(ddt, ddelta.reshape(b, h, p, l).sum(2).transpose(0, 2, 1), **tol)
    np.testing.assert_allclose(dA, dAm.reshape(h, p, -1).sum((1, 2)), **tol)
    np.testing.assert_allclose(dB, dBm.transpose(0, 3, 1, 2), **tol)
    np.testing.assert_allclose(dC, dCm.transpose(0, 3, 1, 2), **tol)
    np.testing.assert_allclose(dz.transpose(0, 2, 3, 1).reshape(b, h * p, l), dzm, **tol)
    np.testing.assert_allclose(dbias, dbm.reshape(h, p).sum(1), **tol)
    if Dshape == "hp":
        np.testing.assert_allclose(dD, dDm.reshape(h, p), **tol)
    elif Dshape == "h":
        np.testing.assert_allclose(dD, dDm.reshape(h, p).sum(1), **tol)


def direct_sum(x, dt, A, B, C, D=None, z=None, dt_bias=None, initial_states=None, dt_softplus=False,
               dt_limit=(0.0, float("inf"))):
    """out and final states in closed form (torch float64, differentiable)."""
    b, l, h, p = x.shape
    pre = dt if dt_bias is None else dt + dt_bias
    step = F.softplus(pre) if dt_softplus else pre
    if dt_limit[0] > 0 or dt_limit[1] < math.inf:
        step = step.clamp(dt_limit[0], dt_limit[1])
    Sc = torch.cumsum(step * A, dim=1)                                  # (b, l, h)
    diff = Sc[:, :, None, :] - Sc[:, None, :, :]                          # (b, t, s, h)
    below = torch.tril(torch.ones(l, l, dtype=torch.bool))[None, :, :, None]
    K = torch.exp(diff.masked_fill(~below, -math.inf))
    rep = h // B.shape[2]
    Bh, Ch = B.repeat_interleave(rep, dim=2), C.repeat_interleave(rep, dim=2)
    CB = torch.einsum("bthn,bshn->btsh", Ch, Bh)
    xs = step[..., None] * x
    y = torch.einsum("btsh,bshp->bthp", K * CB, xs)
    Kend = torch.exp(Sc[:, -1:, :] - Sc)                                  # (b, s, h)
    final = torch.einsum("bsh,bshp,bshn->bhpn", Kend, xs, Bh)
    if initial_states is not None:
        y = y + torch.exp(Sc)[..., None] * torch.einsum("bhpn,bthn->bthp", initial_states, Ch)
        final = final + torch.exp(Sc[:, -1])[..., None, None] * initial_states
    if D is not None:
        y = y + (D[:, None] if D.dim() == 1 else D) * x
    out = y if z is None else y * F.silu(z)
    return out, final


DIRECT_CASES = [
    dict(g=1, init=True, Dshape="hp", z=True, bias=True, softplus=True, limit=(0.0, math.inf)),
    dict(g=2, init=False, Dshape="h", z=False, bias=True, softplus=True, limit=(0.05, 0.6)),
    dict(g=4, init=True, Dshape=None, z=True, bias=False, softplus=False, limit=(0.0, math.inf)),
]


@pytest.mark.parametrize("case", DIRECT_CASES, ids=lambda c: f"g{c['g']}-init{c['init']}-lim{c['limit'][1]}")
def test_ssd_matches_direct_sum_and_its_autograd(case):
    c = ssd_case(2, 11, 4, 3, 5, case["g"], seed=7, init=case["init"], Dshape=case["Dshape"],
                 z=case["z"], bias=case["bias"])
    if not case["softplus"]:
        c["dt"] = np.abs(c["dt"]) * 0.3 + 0.05                          # a positive step without softplus
    kw = dict(dt_softplus=case["softplus"], dt_limit=case["limit"])
    out, last = S.ssd_fwd(**c, **kw)
    t = {k: None if v is None else torch.tensor(v, requires_grad=True) for k, v in c.items()}
    want, want_last = direct_sum(**t, **kw)
    np.testing.assert_allclose(out, want.detach().numpy(), rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(last, want_last.detach().numpy(), rtol=1e-11, atol=1e-11)
    rng = np.random.default_rng(3)
    dout, dfin = rng.standard_normal(out.shape), rng.standard_normal(last.shape)
    ((want * torch.tensor(dout)).sum() + (want_last * torch.tensor(dfin)).sum()).backward()
    got = S.ssd_bwd(**c, **kw, dout=dout, dfinal_states=dfin)
    names = ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "initial_states")
    for name, g_ in zip(names, got):
        if t[name] is None:
            assert g_ is None, name
            continue
        np.testing.assert_allclose(g_, t[name].grad.numpy(), rtol=1e-9, atol=1e-10, err_msg=name)


def test_planted_mistake_in_backward_is_caught():
    """A copy of ssd_bwd whose dA term drops dt_t must fail the autograd check."""
    src = textwrap.dedent(inspect.getsource(S.ssd_bwd))
    bad = src.replace("dA += (step[:, t] * decay_term).sum(0)", "dA += decay_term.sum(0)")
    assert bad != src
    ns = dict(S.__dict__)
    exec(compile(bad, "planted", "exec"), ns)
    c = ssd_case(1, 7, 2, 2, 3, 1, seed=11)
    t = {k: None if v is None else torch.tensor(v, requires_grad=True) for k, v in c.items()}
    want, _ = direct_sum(**t, dt_softplus=True)
    dout = np.ones(want.shape)
    want.backward(torch.tensor(dout))
    dA = ns["ssd_bwd"](**c, dt_softplus=True, dout=dout)[2]
    assert not np.allclose(dA, t["A"].grad.numpy(), rtol=1e-6, atol=1e-8)


def _segments(ids):
    """[(start, end, id)] of the runs of equal ids in a 1-D array."""
    out, s0 = [], 0
    for t in range(1, len(ids) + 1):
        if t == len(ids) or ids[t] != ids[s0]:
            out.append((s0, t, int(ids[s0])))
            s0 = t
    return out


def test_seq_idx_equals_separate_sequences():
    """Packed sequences (seq_idx) give, on each sequence, what that sequence
    gives run alone from a zero state (the one with id 0 from the initial
    state): outputs and the gradients of x, dt, B, C, z on its steps, the final
    state and its gradient on the last one, the initial state's gradient from
    the id-0 one (zero when a row starts above id 0); dA, dD, ddt_bias are the
    sums over sequences."""
    b, l, h, p, n, g = 2, 50, 4, 8, 6, 2
    c = ssd_case(b, l, h, p, n, g, seed=3, init=True)
    seq = np.array([[0] * 13 + [1] * 20 + [2] * 17, [1] * 25 + [3] * 24 + [4]], dtype=np.int32)
    kw = dict(dt_softplus=True, dt_limit=(0.0, float("inf")))
    rng = np.random.default_rng(4)
    dout, dfin = rng.standard_normal(c["x"].shape), rng.standard_normal(c["initial_states"].shape)
    out, fin = S.ssd_fwd(**c, **kw, seq_idx=seq)
    got = S.ssd_bwd(**c, **kw, dout=dout, dfinal_states=dfin, seq_idx=seq)
    names = ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "initial_states")
    g_ = dict(zip(names, got))
    per_step = ("x", "dt", "B", "C", "z")
    sums = {k: 0.0 for k in ("A", "D", "dt_bias")}
    for r in range(b):
        segs = _segments(seq[r])
        dinit_want = np.zeros((h, p, n))
        for i, (s0, s1, sid) in enumerate(segs):
            last = i == len(segs) - 1
            sub = {k: c[k][r:r + 1, s0:s1] for k in per_step}
            sub.update(A=c["A"], D=c["D"], dt_bias=c["dt_bias"],
                       initial_states=c["initial_states"][r:r + 1] if sid == 0 else None)
            o, f = S.ssd_fwd(**sub, **kw)
            np.testing.assert_allclose(out[r, s0:s1], o[0], rtol=1e-12, atol=1e-12)
            if last:
                np.testing.assert_allclose(fin[r], f[0], rtol=1e-12, atol=1e-12)
            sg = dict(zip(names, S.ssd_bwd(**sub, **kw, dout=dout[r:r + 1, s0:s1],
                                           dfinal_states=dfin[r:r + 1] if last else None)))
            for k in per_step:
                np.testing.assert_allclose(g_[k][r, s0:s1], sg[k][0], rtol=1e-10, atol=1e-12, err_msg=k)
            for k in sums:
                sums[k] = sums[k] + sg[k]
            if sid == 0:
                dinit_want = sg["initial_states"][0]
        np.testing.assert_allclose(g_["initial_states"][r], dinit_want, rtol=1e-10, atol=1e-12)
    for k in sums:
        np.testing.assert_allclose(g_[k], sums[k], rtol=1e-10, atol=1e-10, err_msg=k)
    # all ids equal to 0 is the unpacked scan
    o0, f0 = S.ssd_fwd(**c, **kw)
    o1, f1 = S.ssd_fwd(**c, **kw, seq_idx=np.zeros((b, l), dtype=np.int32))
    assert np.array_equal(o0, o1) and np.array_equal(f0, f1)


def test_varlen_states_equal_each_sequence_alone():
    """ssd_varlen_states: entry i is the final state of sequence i run alone
    (from the initial state when it is the id-0 first sequence), zeros for an
    empty sequence; without seq_idx, the final state of the prefix up to the
    sequence's last step; the last entry is ssd_fwd's final state when the last
    sequence ends the row."""
    l, h, p, n, g = 60, 4, 8, 6, 2
    c = ssd_case(1, l, h, p, n, g, seed=5, init=True)
    kw = dict(dt_softplus=True, dt_limit=(0.0, float("inf")))
    cu = np.array([0, 9, 9, 31, 60])
    seq = np.repeat(np.arange(4), np.diff(cu))[None].astype(np.int32)
    args = {k: c[k] for k in ("x", "dt", "A", "B", "C", "dt_bias", "initial_states")}
    got = S.ssd_varlen_states(**args, cu_seqlens=cu, seq_idx=seq, **kw)
    assert got.shape == (4, h, p, n)
    for i in range(4):
        s0, s1 = cu[i], cu[i + 1]
        if s1 == s0:
            assert not got[i].any()
            continue
        sub = {k: c[k][:, s0:s1] for k in ("x", "dt", "B", "C", "z")}
        sub.update(A=c["A"], D=c["D"], dt_bias=c["dt_bias"], initial_states=c["initial_states"] if s0 == 0 else None)
        np.testing.assert_allclose(got[i], S.ssd_fwd(**sub, **kw)[1][0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got[-1], S.ssd_fwd(**c, **kw, seq_idx=seq)[1][0], rtol=1e-12, atol=1e-12)
    plain = S.ssd_varlen_states(**args, cu_seqlens=cu, **kw)
    for i in (0, 2, 3):
        pre = {k: c[k][:, :cu[i + 1]] for k in ("x", "dt", "B", "C", "z")}
        pre.update(A=c["A"], D=c["D"], dt_bias=c["dt_bias"], initial_states=c["initial_states"])
        np.testing.assert_allclose(plain[i], S.ssd_fwd(**pre, **kw)[1][0], rtol=1e-12, atol=1e-12)


def test_raw_negative_steps_clamp_like_transformers():
    """Without softplus, a negative dt + dt_bias is clamped to the default
    dt_limit (0, inf), so that step is 0 and its raw-dt gradient 0, as
    mamba_ssm's kernels and transformers' pure-torch mamba2_chunk_scan do
    (torch.clamp in its first lines). About half of the raw steps here are
    negative; the oracle's outputs, final states and every gradient match
    autograd through transformers' function (float32, so rtol 1e-4)."""
    transformers = pytest.importorskip("transformers", minversion="5.0")
    from transformers.models.mamba2 import modeling_mamba2 as M2

    fn = getattr(M2.mamba2_chunk_scan, "__wrapped__", M2.mamba2_chunk_scan)
    rng = np.random.default_rng(3)
    b, l, h, p, g, n = 2, 70, 4, 8, 2, 8
    c = dict(x=rng.standard_normal((b, l, h, p)), dt=rng.standard_normal((b, l, h)) * 0.5,
             A=-np.exp(rng.random(h) * math.log(8)), B=rng.standard_normal((b, l, g, n)),
             C=rng.standard_normal((b, l, g, n)), D=rng.standard_normal(h), dt_bias=rng.random(h) * 0.2,
             initial_states=rng.standard_normal((b, h, p, n)))
    assert 0.3 < ((c["dt"] + c["dt_bias"]) < 0).mean() < 0.7
    t = {k: torch.tensor(v, dtype=torch.float32, requires_grad=True) for k, v in c.items()}
    out, fin = fn(t["x"], t["dt"], t["A"], t["B"], t["C"], 32, D=t["D"], dt_bias=t["dt_bias"],
                  initial_states=t["initial_states"], dt_softplus=False, return_final_states=True)
    W, V = rng.standard_normal(out.shape), rng.standard_normal(fin.shape)
    ((out * torch.tensor(W, dtype=torch.float32)).sum() + (fin * torch.tensor(V, dtype=torch.float32)).sum()).backward()
    want, want_fin = S.ssd_fwd(**c, dt_softplus=False)
    np.testing.assert_allclose(want, out.detach().numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(want_fin, fin.detach().numpy(), rtol=1e-4, atol=1e-5)
    grads = S.ssd_bwd(**c, z=None, dt_softplus=False, dout=W, dfinal_states=V)
    names = ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "initial_states")
    for name, gw in zip(names, grads):
        if name == "z":
            assert gw is None
            continue
        ref = t[name].grad.numpy()
        scale = max(np.abs(ref).max(), 1.0)
        np.testing.assert_allclose(gw / scale, ref / scale, rtol=1e-4, atol=1e-5, err_msg=name)
    # the clamped steps pass no gradient to the raw dt
    assert np.all(grads[1][(c["dt"] + c["dt_bias"][None, None]) < 0] == 0)

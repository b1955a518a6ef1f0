"""causal_conv1d_fn / causal_conv1d_update on the GPU against the float64 oracle.

Mirrors the reference's tests/test_causal_conv1d.py (oracle parity over width,
activation and bias; initial/final-state chaining; update == full conv;
multi-token update; final_states_out buffer identity; mixed dtypes) and adds
the backward pass (against the oracle's analytic gradients) and strided
channel-contiguous inputs. Tolerances: float32 rtol/atol 1e-5 (forward) and
1e-4 (gradients); bf16 2e-2.
"""

import numpy as np
import pytest
import torch

from oracle import numerics as O

from mamba_cpu import causal_conv1d_fn, causal_conv1d_update

pytestmark = pytest.mark.gpu
DEV = "cuda"


def close(got, want, rtol, atol, name=""):
    np.testing.assert_allclose(got.detach().float().cpu().numpy().astype(np.float64), want,
                               rtol=rtol, atol=atol, err_msg=name)


@pytest.mark.parametrize("width", [1, 2, 3, 4, 5, 7, 16, 17, 40])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("has_bias", [False, True])
def test_matches_oracle(width, activation, has_bias):
    torch.manual_seed(0)
    x = torch.randn(2, 8, 37, device=DEV)
    w = torch.randn(8, width, device=DEV)
    b = torch.randn(8, device=DEV) if has_bias else None
    out = causal_conv1d_fn(x, w, b, activation=activation)
    want, _ = O.causal_conv1d_fwd(x, w, b, activation=activation)
    close(out, want, 1e-5, 1e-5)


def test_initial_and_final_states_chain():
    torch.manual_seed(0)
    x = torch.randn(2, 8, 40, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    full = causal_conv1d_fn(x, w, activation="silu")
    a, state = causal_conv1d_fn(x[..., :25], w, activation="silu", return_final_states=True)
    b = causal_conv1d_fn(x[..., 25:], w, initial_states=state, activation="silu")
    torch.testing.assert_close(torch.cat([a, b], -1), full)


def test_update_matches_full_conv():
    torch.manual_seed(0)
    x = torch.randn(2, 8, 12, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    bias = torch.randn(8, device=DEV)
    full = causal_conv1d_fn(x, w, bias, activation="silu")
    state = torch.zeros(2, 8, 4, device=DEV)
    steps = [causal_conv1d_update(x[..., t], state, w, bias, "silu") for t in range(12)]
    torch.testing.assert_close(torch.stack(steps, -1), full, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("state_len", [3, 4, 6])
@pytest.mark.parametrize("seqlen", [1, 5])
def test_update_multi_token_matches_full_conv(state_len, seqlen):
    torch.manual_seed(0)
    x = torch.randn(2, 8, 12 + seqlen, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    full = causal_conv1d_fn(x, w, activation="silu")
    state = torch.zeros(2, 8, state_len, device=DEV)
    causal_conv1d_update(x[..., :12], state, w)
    out = causal_conv1d_update(x[..., 12:], state, w, activation="silu")
    assert out.shape == (2, 8, seqlen)
    torch.testing.assert_close(out, full[..., 12:], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(state, x[..., -state_len:])


@pytest.mark.parametrize("state_len", [3, 4, 7])
@pytest.mark.parametrize("seqlen", [None, 1, 3])
def test_update_matches_oracle(state_len, seqlen):
    torch.manual_seed(0)
    x = torch.randn(2, 64, device=DEV) if seqlen is None else torch.randn(2, 64, seqlen, device=DEV)
    w, bias = torch.randn(64, 4, device=DEV), torch.randn(64, device=DEV)
    state = torch.randn(2, 64, state_len, device=DEV)
    want, want_state = O.causal_conv1d_update(x, state, w, bias, "silu")
    out = causal_conv1d_update(x, state, w, bias, "silu")
    close(out, want, 1e-5, 1e-5)
    close(state, want_state, 0, 0)


@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("extra", [0, 1, "max", "over"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["contiguous", "channels_last"])
def test_single_step_update_matches_oracle(width, extra, dtype, layout):
    """The single-token decode step (its own kernel for widths 2-4 and state
    lengths up to 8, the general one otherwise) over several steps, with state
    lengths width-1, width, 8 and 9, in both state layouts."""
    torch.manual_seed(3)
    b, d = 3, 300
    S = {0: width - 1, 1: width, "max": 8, "over": 9}[extra]
    w, bias = torch.randn(d, width, device=DEV), torch.randn(d, device=DEV)
    if layout == "contiguous":
        state = torch.randn(b, d, S, device=DEV).to(dtype)
    else:
        state = torch.randn(b, S, d, device=DEV).to(dtype).transpose(1, 2)
    want_state = state.cpu().double().numpy()
    for step in range(3):
        x = torch.randn(b, d, device=DEV).to(dtype)
        out = causal_conv1d_update(x, state, w, bias, "silu")
        want, want_state = O.causal_conv1d_update(x, want_state, w, bias, "silu")
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        close(out, want, tol, tol, f"out step {step}")
        close(state, want_state, 0, 0, f"state step {step}")


def test_final_states_out_buffer():
    x = torch.randn(2, 8, 10, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    buf = torch.empty(2, 8, 3, device=DEV)
    _, final = causal_conv1d_fn(x, w, return_final_states=True, final_states_out=buf)
    assert final is buf
    torch.testing.assert_close(buf, x[..., -3:])


def test_mixed_dtypes_return_input_dtype():
    x = torch.randn(2, 8, 10, device=DEV).bfloat16()
    w = torch.randn(8, 4, device=DEV)
    out = causal_conv1d_fn(x, w, torch.randn(8, device=DEV), activation="silu")
    assert out.dtype == torch.bfloat16
    state = torch.zeros(2, 8, 4, dtype=torch.bfloat16, device=DEV)
    assert causal_conv1d_update(x[..., 0], state, w).dtype == torch.bfloat16


def test_rejects_unsupported_args():
    x = torch.randn(2, 8, 10, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    with pytest.raises(ValueError):  # seq_idx excludes initial states
        causal_conv1d_fn(x, w, seq_idx=torch.zeros(2, 10, dtype=torch.int32, device=DEV),
                         initial_states=torch.zeros(2, 8, 3, device=DEV))
    with pytest.raises(ValueError):
        causal_conv1d_fn(x, w, activation="relu")
    with pytest.raises(ValueError):
        causal_conv1d_update(x, torch.zeros(2, 8, 2, device=DEV), w)
    with pytest.raises(ValueError):  # one index per batch row
        causal_conv1d_update(x[..., 0], torch.zeros(2, 8, 3, device=DEV), w,
                             cache_seqlens=torch.zeros(3, dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("seqlen", [None, 1, 3])
@pytest.mark.parametrize("state_len", [3, 6, 11])
@pytest.mark.parametrize("mode", ["indices", "ring", "both"])
@pytest.mark.parametrize("width", [2, 4])
def test_update_continuous_batching_matches_oracle(seqlen, state_len, mode, width):
    """conv_state_indices (rows of a larger state, one out of range) and
    cache_seqlens (ring buffer), which the reference rejects, against the
    oracle's restatement of the upstream semantics; several steps in a row so
    the ring wraps. Single steps take the 2-D single-step kernel (ring
    positions wrapped per batch row, any state length), longer ones the
    general kernel."""
    torch.manual_seed(7 + width)
    b, d, rows = 3, 20, 6
    w = torch.randn(d, width, device=DEV)
    bias = torch.randn(d, device=DEV)
    state = torch.randn(rows, d, state_len, device=DEV)
    idx = torch.tensor([4, 0, 9], dtype=torch.int32, device=DEV) if mode != "ring" else None
    want_state = state.cpu().double().numpy()
    if mode == "ring":
        state = state[:b].clone()
        want_state = want_state[:b]
    cs = torch.tensor([0, 5, 100003], dtype=torch.int64, device=DEV) if mode != "indices" else None
    for step in range(4):
        x = torch.randn(b, d, device=DEV) if seqlen is None else torch.randn(b, d, seqlen, device=DEV)
        out = causal_conv1d_update(x, state, w, bias, "silu", cache_seqlens=cs, conv_state_indices=idx)
        want, want_state = O.causal_conv1d_update(
            x, want_state, w, bias, "silu",
            cache_seqlens=None if cs is None else cs.cpu().numpy(),
            conv_state_indices=None if idx is None else idx.cpu().numpy())
        close(out, want, 1e-5, 1e-5, f"out step {step}")
        close(state, want_state, 0, 0, f"state step {step}")
        if cs is not None:
            cs = cs + (1 if seqlen is None else seqlen)


@pytest.mark.parametrize("width", [1, 2, 4, 7, 17, 33, 60])
@pytest.mark.parametrize("activation", [None, "silu"])
@pytest.mark.parametrize("with_init", [False, True])
@pytest.mark.parametrize("layout", ["contiguous", "channels_last"])
def test_backward_matches_oracle(width, activation, with_init, layout):
    torch.manual_seed(0)
    b, d, l = 2, 24, 45
    if layout == "contiguous":
        x = torch.randn(b, d, l, device=DEV)
    else:
        x = torch.randn(b, l, d, device=DEV).transpose(1, 2)
    x.requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    init = torch.randn(b, d, width - 1, device=DEV, requires_grad=True) if with_init else None
    out, final = causal_conv1d_fn(x, w, bias, initial_states=init, return_final_states=True,
                                  activation=activation)
    want_out, want_final = O.causal_conv1d_fwd(x, w, bias, init, activation)
    close(out, want_out, 1e-5, 1e-5, "out")
    close(final, want_final, 0, 0, "final")
    G = torch.randn(b, d, l, device=DEV)
    Gf = torch.randn(b, d, width - 1, device=DEV)
    ((out * G).sum() + (final * Gf).sum()).backward()
    dx, dw, db, dinit = O.causal_conv1d_bwd(x, w, bias, init, G, activation, Gf)
    close(x.grad, dx, 1e-4, 1e-4, "dx")
    close(w.grad, dw, 1e-4, 1e-4, "dweight")
    close(bias.grad, db, 1e-4, 1e-4, "dbias")
    if with_init:
        close(init.grad, dinit, 1e-4, 1e-4, "dinit")


def test_channels_last_output_layout():
    """A channel-contiguous x (Hugging Face's transposed view) gets a
    channel-contiguous output, so transposing it back is free."""
    x = torch.randn(2, 30, 16, device=DEV).transpose(1, 2)
    w = torch.randn(16, 4, device=DEV)
    out = causal_conv1d_fn(x, w, activation="silu")
    assert out.transpose(1, 2).is_contiguous()
    want, _ = O.causal_conv1d_fwd(x, w, activation="silu")
    close(out, want, 1e-5, 1e-5)


def test_bf16_forward_backward():
    torch.manual_seed(0)
    x = torch.randn(2, 16, 50, device=DEV).bfloat16().requires_grad_()
    w = torch.randn(16, 4, device=DEV, requires_grad=True)
    bias = torch.randn(16, device=DEV, requires_grad=True)
    out = causal_conv1d_fn(x, w, bias, activation="silu")
    assert out.dtype == torch.bfloat16
    want, _ = O.causal_conv1d_fwd(x, w, bias, activation="silu")
    close(out, want, 2e-2, 2e-2)
    G = torch.randn(2, 16, 50, device=DEV).bfloat16()
    (out.float() * G.float()).sum().backward()
    dx, dw, db, _ = O.causal_conv1d_bwd(x, w, bias, None, G, "silu")
    assert x.grad.dtype == torch.bfloat16
    close(x.grad, dx, 2e-2, 2e-2, "dx")
    close(w.grad / max(np.abs(dw).max(), 1), dw / max(np.abs(dw).max(), 1), 2e-2, 2e-2, "dw")
    close(bias.grad / max(np.abs(db).max(), 1), db / max(np.abs(db).max(), 1), 2e-2, 2e-2, "db")


def test_opcheck():
    x = torch.randn(2, 8, 12, device=DEV, requires_grad=True)
    w = torch.randn(8, 4, device=DEV, requires_grad=True)
    b = torch.randn(8, device=DEV, requires_grad=True)
    init = torch.randn(2, 8, 3, device=DEV, requires_grad=True)
    torch.library.opcheck(torch.ops.mamba_cpu.causal_conv1d_fwd.default, (x, w, b, init, True, True))
    torch.library.opcheck(torch.ops.mamba_cpu.causal_conv1d_bwd.default,
                          (x.detach(), w.detach(), b.detach(), init.detach(),
                           torch.randn(2, 8, 12, device=DEV), torch.randn(2, 8, 3, device=DEV), True))


@pytest.mark.parametrize("seqlen", [8, 16, 64, 520, 1024, 2048, 2056, 4112])
@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_vector_path_forward_backward(seqlen, width, dtype):
    """Time-contiguous x with seqlen a multiple of 8 takes the vectorised
    kernels (8 steps per thread in fp32; 16 in bf16 when seqlen is a multiple
    of 16, else 8): rows of one to four waves and rows split into 256-thread
    segments (2056 and 4112 in fp32, 2056 (8 steps) and 4112 in bf16).
    Initial/final states and their gradients ride along; the chunk at t = 0
    reads the initial states, the last one dfinal."""
    torch.manual_seed(seqlen + width)
    b, d = 2, 6
    x = torch.randn(b, d, seqlen, device=DEV).to(dtype).requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    init = torch.randn(b, d, width - 1, device=DEV).to(dtype).requires_grad_()
    out, final = causal_conv1d_fn(x, w, bias, initial_states=init, return_final_states=True,
                                  activation="silu")
    want_out, want_final = O.causal_conv1d_fwd(x, w, bias, init, "silu")
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    close(out, want_out, tol, tol, "out")
    close(final, want_final, 0, 0, "final")
    G = torch.randn(b, d, seqlen, device=DEV).to(dtype)
    Gf = torch.randn(b, d, width - 1, device=DEV).to(dtype)
    ((out.float() * G.float()).sum() + (final.float() * Gf.float()).sum()).backward()
    dx, dw, db, dinit = O.causal_conv1d_bwd(x, w, bias, init, G, "silu", Gf)
    gtol = 1e-4 if dtype == torch.float32 else 2e-2
    close(x.grad, dx, gtol, gtol, "dx")
    close(init.grad, dinit, gtol, gtol, "dinit")
    for got, want, name in ((w.grad, dw, "dweight"), (bias.grad, db, "dbias")):
        s = max(np.abs(want).max(), 1.0)
        close(got / s, want / s, gtol, gtol, name)


def test_vector_path_no_activation_no_bias():
    torch.manual_seed(3)
    x = torch.randn(3, 5, 128, device=DEV, requires_grad=True)
    w = torch.randn(5, 4, device=DEV, requires_grad=True)
    out = causal_conv1d_fn(x, w)
    want, _ = O.causal_conv1d_fwd(x, w)
    close(out, want, 1e-5, 1e-5)
    G = torch.randn(3, 5, 128, device=DEV)
    (out * G).sum().backward()
    dx, dw, _, _ = O.causal_conv1d_bwd(x, w, None, None, G, None)
    close(x.grad, dx, 1e-4, 1e-4, "dx")
    close(w.grad, dw, 1e-4, 1e-4, "dweight")


@pytest.mark.parametrize("batch,parts_per_row", [(1, 1), (3, 9), (5, 16)])
def test_dweight_reduction_over_many_partials(batch, parts_per_row):
    """dweight/dbias sum one partial per (batch, time chunk): every count of
    partials, including ones not a multiple of the reduction's unroll."""
    torch.manual_seed(1)
    d, width = 70, 4
    l = 8 * parts_per_row + 3  # ragged last chunk, off the vector path
    x = torch.randn(batch, l, d, device=DEV).transpose(1, 2).requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    out = causal_conv1d_fn(x, w, bias, activation="silu")
    G = torch.randn(batch, d, l, device=DEV)
    (out * G).sum().backward()
    _, dw, db, _ = O.causal_conv1d_bwd(x, w, bias, None, G, "silu")
    close(w.grad, dw, 1e-4, 1e-4, "dweight")
    close(bias.grad, db, 1e-4, 1e-4, "dbias")


@pytest.mark.parametrize("layout", ["contiguous", "channels_last"])
@pytest.mark.parametrize("width", [2, 4, 7])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_seq_idx_matches_oracle(layout, width, dtype):
    """Packed sequences (seq_idx, which the reference rejects): forward and
    every gradient against the oracle, with boundaries inside and across the
    8-step chunks and a one-step sequence."""
    torch.manual_seed(width)
    b, d, l = 2, 24, 45
    xs = torch.randn(b, d, l, device=DEV) if layout == "contiguous" else \
        torch.randn(b, l, d, device=DEV).transpose(1, 2)
    x = xs.to(dtype).requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    seq = torch.zeros(b, l, dtype=torch.int32)
    for bi, cuts in enumerate([[0, 3, 4, 16, 30, 45], [0, 45]]):
        for si, (lo, hi) in enumerate(zip(cuts[:-1], cuts[1:])):
            seq[bi, lo:hi] = si + 7 * bi
    seq = seq.to(DEV)
    out = causal_conv1d_fn(x, w, bias, seq_idx=seq, activation="silu")
    want, _ = O.causal_conv1d_fwd(x, w, bias, None, "silu", seq_idx=seq.cpu().numpy())
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    close(out, want, tol, tol, "out")
    G = torch.randn(b, d, l, device=DEV).to(dtype)
    (out.float() * G.float()).sum().backward()
    dx, dw, db, _ = O.causal_conv1d_bwd(x, w, bias, None, G, "silu", seq_idx=seq.cpu().numpy())
    gtol = 1e-4 if dtype == torch.float32 else 2e-2
    close(x.grad, dx, gtol, gtol, "dx")
    for got, want_, name in ((w.grad, dw, "dweight"), (bias.grad, db, "dbias")):
        sc = max(np.abs(want_).max(), 1.0)
        close(got / sc, want_ / sc, gtol, gtol, name)


def _packed_ids(b, l, cuts_per_row, device):
    """(b, l) int32 sequence ids, row r cut at cuts_per_row[r]."""
    seq = torch.zeros(b, l, dtype=torch.int32)
    for bi, cuts in enumerate(cuts_per_row):
        edges = [0] + sorted(c for c in cuts if 0 < c < l) + [l]
        for si, (lo, hi) in enumerate(zip(edges[:-1], edges[1:])):
            seq[bi, lo:hi] = si + 11 * bi
    return seq.to(device)


@pytest.mark.parametrize("width", [2, 3, 4, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seqlen", [1, 7, 45, 130])
@pytest.mark.parametrize("packed", [False, True])
def test_channel_contiguous_path_matches_oracle(width, dtype, seqlen, packed):
    """x, out, dout and dx all channel-contiguous (the fused mixer's and
    Hugging Face's layout) take the four-channels-per-lane kernels: 264
    channels (a second, partly filled 256-channel tile), 8-step segments with
    a ragged last one, and packed sequences with boundaries inside segments,
    on segment starts and a one-step sequence."""
    torch.manual_seed(width * 100 + seqlen)
    b, d = 3, 264
    x = torch.randn(b, seqlen, d, device=DEV).to(dtype).transpose(1, 2).requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    seq = _packed_ids(b, seqlen, [[3, 4, 16, 40, 41], [8, 24, 100], [1]], DEV) if packed else None
    out = causal_conv1d_fn(x, w, bias, seq_idx=seq, activation="silu")
    assert out.transpose(1, 2).is_contiguous()
    sq = None if seq is None else seq.cpu().numpy()
    want, _ = O.causal_conv1d_fwd(x, w, bias, None, "silu", seq_idx=sq)
    tol = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 3e-3}[dtype]
    close(out, want, tol, tol, "out")
    G = torch.randn(b, seqlen, d, device=DEV).to(dtype).transpose(1, 2)
    dx_, dw_, db_ = torch.autograd.grad(out, [x, w, bias], G)
    dx, dw, db, _ = O.causal_conv1d_bwd(x, w, bias, None, G, "silu", seq_idx=sq)
    gtol = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 3e-3}[dtype]
    close(dx_, dx, gtol, gtol, "dx")
    for got, want_, name in ((dw_, dw, "dweight"), (db_, db, "dbias")):
        sc = max(np.abs(want_).max(), 1.0)
        close(got / sc, want_ / sc, gtol, gtol, name)


@pytest.mark.parametrize("packed", [False, True])
def test_channel_contiguous_long_segments_match_time_contiguous(packed):
    """A long sequence gives the channel-contiguous kernels 16-step segments
    walked in two unrolled groups (one group when a segment holds a sequence
    boundary) and a ragged last segment. The outputs and input gradients are
    the same sums in the same order as the time-contiguous kernels': the
    outputs match bitwise, the input gradients to rounding (the activation's
    derivative is associated differently); the weight gradients sum the
    partials in another order."""
    torch.manual_seed(5)
    b, d, l, width = 8, 256, 16384 + 5, 4
    xt = torch.randn(b, l, d, device=DEV)
    w = torch.randn(d, width, device=DEV) * 0.5
    bias = torch.randn(d, device=DEV) * 0.3
    Gt = torch.randn(b, l, d, device=DEV)
    cuts = [[16, 17, 4000, 9999], [5], [], [8192, 8193, 8194], [16], [1, 2, 3], [16384], [777]]
    seq = _packed_ids(b, l, cuts, DEV) if packed else None
    res = []
    for x, G in ((xt.transpose(1, 2), Gt.transpose(1, 2)),
                 (xt.transpose(1, 2).contiguous(), Gt.transpose(1, 2).contiguous())):
        xx, ww, bb = x.clone().requires_grad_(), w.clone().requires_grad_(), bias.clone().requires_grad_()
        out = causal_conv1d_fn(xx, ww, bb, seq_idx=seq, activation="silu")
        res.append((out, *torch.autograd.grad(out, [xx, ww, bb], G)))
    (o1, dx1, dw1, db1), (o2, dx2, dw2, db2) = res
    assert torch.equal(o1, o2)
    torch.testing.assert_close(dx1, dx2, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(dw1, dw2, rtol=1e-5, atol=1e-2)
    torch.testing.assert_close(db1, db2, rtol=1e-5, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["contiguous", "channels_last"])
def test_wide_width_packed_sequences_and_long_rows(dtype, layout):
    """Widths above 16 run per-element kernels (the reference's F.conv1d takes
    any width): forward, final states and every gradient against the oracle
    with packed sequences (seq_idx, cuts inside and across the taps' reach),
    and over 700 steps (three dweight segments of 256 steps), in float32 and
    bfloat16."""
    torch.manual_seed(3)
    b, d, l, width = 2, 12, 700, 24
    if layout == "contiguous":
        x = torch.randn(b, d, l, device=DEV).to(dtype)
    else:
        x = torch.randn(b, l, d, device=DEV).to(dtype).transpose(1, 2)
    x.requires_grad_()
    w = torch.randn(d, width, device=DEV, requires_grad=True)
    bias = torch.randn(d, device=DEV, requires_grad=True)
    seq = torch.zeros(b, l, dtype=torch.int32)
    for r, cuts in enumerate([[5, 30, 31, 400], [300]]):
        for c in cuts:
            seq[r, c:] += 1
    seq = seq.to(DEV)
    out = causal_conv1d_fn(x, w, bias, seq_idx=seq, activation="silu")
    want, _ = O.causal_conv1d_fwd(x.float(), w, bias, None, "silu", seq_idx=seq.cpu().numpy())
    tol = (1e-5, 1e-5) if dtype == torch.float32 else (2e-2, 2e-2)
    close(out, want, *tol, "out")
    G = torch.randn(b, d, l, device=DEV).to(dtype)
    (out.float() * G.float()).sum().backward()
    dx, dw, db, _ = O.causal_conv1d_bwd(x.float(), w, bias, None, G.float(), "silu", None,
                                        seq_idx=seq.cpu().numpy())
    gtol = (1e-4, 1e-4) if dtype == torch.float32 else (2e-2, 2e-2)
    close(x.grad, dx, *gtol, "dx")
    scale = max(np.abs(dw).max(), 1.0)
    close(w.grad / scale, dw / scale, *gtol, "dweight")
    close(bias.grad / max(np.abs(db).max(), 1.0), db / max(np.abs(db).max(), 1.0), *gtol, "dbias")


@pytest.mark.parametrize("seqlen", [None, 3])
def test_wide_width_update_matches_oracle(seqlen):
    """The decode update at width 20 (taps read from memory), several steps,
    against the oracle, output and state."""
    torch.manual_seed(5)
    b, d, width, state_len = 3, 10, 20, 22
    w = torch.randn(d, width, device=DEV)
    bias = torch.randn(d, device=DEV)
    state = torch.randn(b, d, state_len, device=DEV)
    want_state = state.cpu().double().numpy()
    for step in range(3):
        x = torch.randn(b, d, device=DEV) if seqlen is None else torch.randn(b, d, seqlen, device=DEV)
        out = causal_conv1d_update(x, state, w, bias, "silu")
        want, want_state = O.causal_conv1d_update(x, want_state, w, bias, "silu")
        close(out, want, 1e-5, 1e-5, f"out step {step}")
        close(state, want_state, 0, 0, f"state step {step}")

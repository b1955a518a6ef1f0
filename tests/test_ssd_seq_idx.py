"""Packed sequences (seq_idx) in mamba_chunk_scan_combined on the GPU.

Against the float64 oracle (oracle/ssd.py with seq_idx, pinned by
tests/test_oracle_ssd.py against each packed sequence run on its own):
sequence starts inside chunks, on chunk edges (steps 64, 128) and one step
after them, a new sequence at step 0 with an id above 0 (the initial state
is dropped), one sequence per step, one id for the whole row, ragged tails;
the two ways chunk states are carried; 16-bit storage; the autograd path
through mamba_chunk_scan_combined with int64 ids. At 2048 steps (beyond
what the oracle finishes quickly) a packed run is checked against the same
sequences run one at a time on the GPU. Ids that are all 0 give the result
without seq_idx bit for bit (every mask is open). Per-sequence final states
(cu_seqlens, return_varlen_states) against oracle.ssd_varlen_states: empty
and one-step sequences, ends on chunk edges, a first sequence that ends
inside the first chunk with an initial state, both ways of carrying chunk
states, 16-bit storage, and through mamba_chunk_scan_combined with autograd;
head blocks of 1, 2 and 4 heads; opcheck of the operators with seq_idx and
of ssd_varlen_states.
Tolerances as in tests/test_ssd.py: float32 outputs and states rtol 1e-4 /
atol 1e-5, gradients rtol 1e-3 with atol 1e-4 (dx, ddt, dz) or 1e-3 (sums);
16-bit storage 2e-2.
"""

import numpy as np
import pytest
import torch

from conftest import assert_close_report
from oracle import ssd as S
from test_ssd import DEV, NAMES, case, check_ops, run_ops

import mamba_cpu

pytestmark = pytest.mark.gpu


def ids(l, starts, first=0):
    """One row of ids: `first` from step 0, one more at each step in starts."""
    row = np.full(l, first, dtype=np.int32)
    for s in sorted(starts):
        row[s:] += 1
    return row


LAYOUTS = {
    # name: (b, l, rows of (starts, first id))
    "inside-chunks": (2, 200, [([30, 100, 150], 0), ([5, 6, 199], 0)]),
    "chunk-edges": (2, 260, [([64, 128, 192], 0), ([63, 65, 129, 256], 0)]),
    "first-id-above-0": (2, 130, [([], 1), ([70], 2)]),
    "one-id": (1, 150, [([], 0)]),
    "every-step": (1, 70, [(list(range(1, 70)), 0)]),
}


def _seq(b, l, rows):
    return np.stack([ids(l, st, first) for st, first in rows[:b]])


@pytest.mark.parametrize("layout", list(LAYOUTS), ids=list(LAYOUTS))
@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_seq_idx_matches_oracle(layout, chunk_pass):
    b, l, rows = LAYOUTS[layout]
    seq = _seq(b, l, rows)
    c = case(b, l, 4, 32, 2, 64, seed=11 + l, init=True)
    print(f" {layout} chunk_pass {chunk_pass} ids {seq.tolist() if l < 80 else seq[:, ::16].tolist()}",
          flush=True)
    check_ops(c, run_ops(c, chunk_pass=chunk_pass, seq=seq), seq=seq)


@pytest.mark.parametrize("shape,opts", [
    ((1, 300, 8, 64, 1, 128), dict(init=True, z=False)),
    ((3, 129, 4, 16, 4, 16), dict(init=True, D="h")),
    ((2, 100, 2, 48, 1, 32), dict(D=None, bias=False)),
], ids=["n128", "p16-g4", "p48-noD"])
@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_seq_idx_shapes_match_oracle(shape, opts, chunk_pass):
    b, l = shape[:2]
    rng = np.random.default_rng(sum(shape))
    seq = np.stack([ids(l, rng.choice(np.arange(1, l), size=int(rng.integers(1, 6)), replace=False),
                        int(rng.integers(0, 2))) for _ in range(b)])
    c = case(*shape, seed=sum(shape) + 3, **opts)
    check_ops(c, run_ops(c, chunk_pass=chunk_pass, seq=seq), seq=seq)


@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_seq_idx_head_blocks(chunk_pass):
    """Packed sequences with the chunk kernels' head block pinned to 1, 2 and
    4 heads (8 heads, 2 groups): each against the oracle."""
    b, l = 2, 170
    seq = _seq(b, l, [([20, 64, 120], 0), ([100], 1)])
    c = case(b, l, 8, 32, 2, 64, seed=17, init=True)
    for hb in (1, 2, 4):
        print(f" head_block {hb}", flush=True)
        check_ops(c, run_ops(c, head_block=hb, chunk_pass=chunk_pass, seq=seq), seq=seq)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_seq_idx_low_precision(dtype):
    b, l = 2, 200
    seq = _seq(b, l, [([64, 90], 0), ([1, 128], 1)])
    c = case(b, l, 8, 64, 2, 64, seed=4, init=True, dtype=dtype)
    for cp in (1, 2):
        check_ops(c, run_ops(c, chunk_pass=cp, seq=seq), low=True, seq=seq)


def test_seq_idx_through_autograd():
    """mamba_chunk_scan_combined with int64 ids and autograd: every gradient
    against the oracle."""
    b, l = 2, 140
    seq = _seq(b, l, [([40, 64], 0), ([100], 0)])
    c = case(b, l, 4, 32, 1, 32, seed=8, init=True)
    dev = {k: None if v is None else v.to(DEV).requires_grad_(True) for k, v in c.items()}
    out, fin = mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=256, dt_softplus=True,
                                                   seq_idx=torch.as_tensor(seq, dtype=torch.int64, device=DEV),
                                                   return_final_states=True)
    gen = torch.Generator().manual_seed(2)
    W, V = torch.randn(out.shape, generator=gen), torch.randn(fin.shape, generator=gen)
    ((out * W.to(DEV)).sum() + (fin * V.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    got = (out.detach(), fin.detach(), [dev[k].grad for k in NAMES], W, V)
    check_ops(c, got, seq=seq)


@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_zero_ids_equal_no_ids(chunk_pass):
    c = case(2, 200, 4, 32, 2, 64, seed=21, init=True)
    a = run_ops(c, chunk_pass=chunk_pass)
    z = run_ops(c, chunk_pass=chunk_pass, seq=np.zeros((2, 200), dtype=np.int32))
    assert torch.equal(a[0], z[0]) and torch.equal(a[1], z[1])
    for name, x, y in zip(NAMES, a[2], z[2]):
        assert torch.equal(x, y), name


@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_packed_equals_separate_at_2048_steps(chunk_pass):
    """A row of four packed sequences (2048 steps, starts at 500, 1024 and
    1500) against each sequence run alone on the GPU: outputs and per-step
    gradients of each segment, dB / dC, the final state (the last
    sequence's) and summed gradients (dA, dD, ddt_bias)."""
    l, starts = 2048, [0, 500, 1024, 1500, 2048]
    seq = ids(l, starts[1:-1])[None]
    c = case(1, l, 8, 64, 1, 128, seed=31, init=False)
    packed = run_ops(c, chunk_pass=chunk_pass, seq=seq)
    out, fin, g, W, V = packed
    sums = {k: torch.zeros_like(g[NAMES.index(k)]) for k in ("A", "D", "dt_bias")}
    for i, (s0, s1) in enumerate(zip(starts[:-1], starts[1:])):
        sub = {k: (v[:, s0:s1].contiguous() if k in ("x", "dt", "B", "C", "z") else v) for k, v in c.items()}
        last = s1 == l
        # the segment's upstream gradients: its slice of W, and V only on the last sequence
        d = {k: None if v is None else v.to(DEV) for k, v in sub.items()}
        args = (d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["z"], d["dt_bias"], None, True, 0.0,
                float("inf"))
        o, f, saved, ysave = torch.ops.mamba_cpu.ssd_fwd(*args, True, 0, chunk_pass)
        Vs = V if last else torch.zeros_like(V)
        gs = torch.ops.mamba_cpu.ssd_bwd(W[:, s0:s1].contiguous().to(DEV), Vs.to(DEV), *args, saved, ysave, 0,
                                         chunk_pass)
        torch.cuda.synchronize()
        print(f" segment {i} [{s0}, {s1})", flush=True)
        assert_close_report(out[:, s0:s1], o, 1e-4, 1e-5, f"out[{i}]")
        if last:
            assert_close_report(fin, f, 1e-4, 1e-5, "final_states")
        for name in ("x", "dt", "B", "C", "z"):
            k = NAMES.index(name)
            tol = (1e-3, 1e-4) if name in ("x", "dt", "z") else (1e-3, 1e-3)
            assert_close_report(g[k][:, s0:s1], gs[k], *tol, f"d{name}[{i}]")
        for k in sums:
            sums[k] += gs[NAMES.index(k)]
    for k, v in sums.items():
        assert_close_report(g[NAMES.index(k)], v, 1e-3, 1e-3, f"d{k}")


VARLEN = {
    # name: (seqlen, cu_seqlens)
    "inside-chunks": (200, [0, 30, 100, 150, 200]),
    "chunk-edges": (260, [0, 64, 128, 192, 260]),
    "empty-and-one-step": (130, [0, 0, 1, 65, 65, 130]),
    "first-ends-in-chunk-0": (150, [0, 20, 150]),
}


def _varlen_ops(c, cu, seq, chunk_pass=0, softplus=True):
    d = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    if d["D"] is not None and d["D"].dim() == 1:
        d["D"] = d["D"][:, None].expand(d["x"].shape[2:]).contiguous()
    args = (d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["z"], d["dt_bias"], d["initial_states"],
            softplus, 0.0, float("inf"))
    sq = torch.as_tensor(seq, dtype=torch.int32).to(DEV)
    out, fin, saved, _ = torch.ops.mamba_cpu.ssd_fwd(*args, False, 0, chunk_pass, seq_idx=sq)
    var = torch.ops.mamba_cpu.ssd_varlen_states(*args, saved, torch.as_tensor(cu, dtype=torch.int32).to(DEV), 0,
                                                chunk_pass, seq_idx=sq)
    torch.cuda.synchronize()
    return var, fin


@pytest.mark.parametrize("layout", list(VARLEN), ids=list(VARLEN))
@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_varlen_states_match_oracle(layout, chunk_pass):
    """Per-sequence final states (return_varlen_states) against the oracle:
    zeros for empty sequences; the initial state reaches the id-0 first
    sequence, also when it ends inside the first chunk; the last entry is
    the final state."""
    l, cu = VARLEN[layout]
    seq = np.repeat(np.arange(len(cu) - 1), np.diff(cu))[None].astype(np.int32)
    c = case(1, l, 4, 32, 2, 64, seed=7 + l, init=True)
    print(f" {layout} chunk_pass {chunk_pass} cu {cu}", flush=True)
    var, fin = _varlen_ops(c, cu, seq, chunk_pass)
    want = S.ssd_varlen_states(c["x"], c["dt"], c["A"], c["B"], c["C"], cu, dt_bias=c["dt_bias"],
                               initial_states=c["initial_states"], dt_softplus=True, seq_idx=seq)
    assert_close_report(var, want, 1e-4, 1e-5, "varlen_states")
    for i in np.flatnonzero(np.diff(cu) == 0):
        assert not var[i].any()
    assert_close_report(var[-1], fin[0], 1e-4, 1e-5, "last = final")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_states_low_precision(dtype):
    cu = [0, 50, 64, 190, 300]
    seq = np.repeat(np.arange(4), np.diff(cu))[None].astype(np.int32)
    c = case(1, 300, 8, 64, 1, 128, seed=3, init=True, dtype=dtype)
    want = S.ssd_varlen_states(c["x"], c["dt"], c["A"], c["B"], c["C"], cu, dt_bias=c["dt_bias"],
                               initial_states=c["initial_states"], dt_softplus=True, seq_idx=seq)
    for cp in (1, 2):
        var, _ = _varlen_ops(c, cu, seq, cp)
        assert_close_report(var, want, 2e-2, 2e-2, f"varlen_states cp{cp}")


def test_varlen_states_through_the_function():
    """mamba_chunk_scan_combined(..., return_final_states=True,
    return_varlen_states=True) returns (out, final, varlen) with autograd on
    the inputs; varlen carries no gradient; the same results without
    autograd; out and final as without cu_seqlens."""
    cu = [0, 40, 41, 140]
    seq = torch.as_tensor(np.repeat(np.arange(3), np.diff(cu))[None], device=DEV)
    c = case(1, 140, 4, 32, 1, 32, seed=12, init=True)
    dev = {k: None if v is None else v.to(DEV).requires_grad_(True) for k, v in c.items()}
    kw = dict(chunk_size=256, dt_softplus=True, seq_idx=seq, return_final_states=True)
    out, fin, var = mamba_cpu.mamba_chunk_scan_combined(
        **dev, cu_seqlens=torch.as_tensor(cu, device=DEV), return_varlen_states=True, **kw)
    assert not var.requires_grad and out.requires_grad
    (out.sum() + fin.sum()).backward()
    with torch.no_grad():
        out2, fin2, var2 = mamba_cpu.mamba_chunk_scan_combined(
            **dev, cu_seqlens=torch.as_tensor(cu, device=DEV), return_varlen_states=True, **kw)
        out3, fin3 = mamba_cpu.mamba_chunk_scan_combined(**dev, **kw)
    assert torch.equal(out, out2) and torch.equal(fin, fin2) and torch.equal(var, var2)
    assert torch.equal(out, out3) and torch.equal(fin, fin3)
    want = S.ssd_varlen_states(c["x"], c["dt"], c["A"], c["B"], c["C"], cu, dt_bias=c["dt_bias"],
                               initial_states=c["initial_states"], dt_softplus=True, seq_idx=seq.cpu().numpy())
    assert_close_report(var, want, 1e-4, 1e-5, "varlen_states")
    with pytest.raises(ValueError, match="seq_idx"):
        mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=64, cu_seqlens=torch.as_tensor(cu, device=DEV),
                                            return_varlen_states=True)


def test_opcheck_with_seq_idx_and_varlen_states():
    """opcheck of ssd_fwd / ssd_bwd with seq_idx and of ssd_varlen_states."""
    cu = [0, 30, 31, 70]
    c = case(1, 70, 2, 16, 1, 16, seed=9, init=True)
    d = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    seq = torch.as_tensor(np.repeat(np.arange(3), np.diff(cu))[None], dtype=torch.int32, device=DEV)
    args = (d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["z"], d["dt_bias"], d["initial_states"],
            True, 0.0, float("inf"))
    torch.library.opcheck(torch.ops.mamba_cpu.ssd_fwd.default, args + (True,), dict(seq_idx=seq))
    out, fin, saved, ysave = torch.ops.mamba_cpu.ssd_fwd(*args, True, seq_idx=seq)
    bargs = (torch.randn_like(out), torch.randn_like(fin)) + args + (saved, ysave)
    torch.library.opcheck(torch.ops.mamba_cpu.ssd_bwd.default, bargs, dict(seq_idx=seq))
    cut = torch.as_tensor(cu, dtype=torch.int32, device=DEV)
    torch.library.opcheck(torch.ops.mamba_cpu.ssd_varlen_states.default, args + (saved, cut), dict(seq_idx=seq))

"""mamba_chunk_scan_combined (Mamba-2's SSD scan) on the GPU against the
float64 oracle (oracle/ssd.py, pinned by tests/test_oracle_ssd.py).

Cases: sequence lengths that are and are not multiples of the 64-step chunk
(one chunk, several, a ragged tail, 2048 steps), headdim 16-64, dstate
16-128, 1, 2 or 4 groups, D per head or per channel, with and without z,
dt_bias, softplus, a dt_limit clamp, initial states and final states;
float32, bfloat16 and float16 storage; every gradient; workgroups walking
1, 2, 4 or 8 heads of a group; chunk states carried by two launches or by
the in-order kernels; opcheck of the two operators; an empty sequence.
Tolerances (unscaled, |got - want| <= atol + rtol |want|): float32 outputs
and final states rtol 1e-4 / atol 1e-5; float32 gradients rtol 1e-3 with
atol 1e-4 for per-element gradients (dx, ddt, dz) and 1e-3 for sums (dA,
dB, dC, dD, ddt_bias, dinitial_states); 16-bit storage 2e-2 / 2e-2, against
the oracle on the same rounded inputs and upstream gradients.
"""

import math

import numpy as np
import pytest
import torch

from conftest import assert_close_report
from oracle import ssd as S

import mamba_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "initial_states")


def case(b, l, h, p, g, n, seed=0, D="hp", z=True, bias=True, init=False, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    c = dict(x=r(b, l, h, p).to(dtype), dt=r(b, l, h) * 0.5 - 1.0,
             A=-torch.exp(torch.rand(h, generator=gen) * math.log(8)),
             B=r(b, l, g, n).to(dtype), C=r(b, l, g, n).to(dtype))
    c["D"] = None if D is None else r(*((h, p) if D == "hp" else (h,)))
    c["z"] = r(b, l, h, p).to(dtype) if z else None
    c["dt_bias"] = torch.rand(h, generator=gen) * 0.5 if bias else None
    c["initial_states"] = r(b, h, p, n) if init else None
    return c


def run(c, grads=True, softplus=True, limit=(0.0, float("inf")), seed=1):
    """out, final states and the gradients of sum(out W) + sum(final V) on
    the GPU, and W, V."""
    dev = {k: None if v is None else v.to(DEV).requires_grad_(grads) for k, v in c.items()}
    out, fin = mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=256, dt_softplus=softplus,
                                                   dt_limit=limit, return_final_states=True)
    gen = torch.Generator().manual_seed(seed)
    W = torch.randn(out.shape, generator=gen).to(out.dtype)
    V = torch.randn(fin.shape, generator=gen)
    got = {}
    if grads:
        ((out.float() * W.to(DEV).float()).sum() + (fin * V.to(DEV)).sum()).backward()
        got = {k: v.grad for k, v in dev.items() if v is not None}
    torch.cuda.synchronize()
    return out.detach(), fin.detach(), got, W, V


def check(c, out, fin, got, W, V, softplus=True, limit=(0.0, float("inf")), low=False):
    kw = dict(dt_softplus=softplus, dt_limit=limit)
    want, want_fin = S.ssd_fwd(**c, **kw)
    o_tol = (2e-2, 2e-2) if low else (1e-4, 1e-5)
    assert_close_report(out, want, *o_tol, "out")
    assert_close_report(fin, want_fin, *((2e-2, 2e-2) if low else (1e-4, 1e-5)), "final_states")
    if not got:
        return
    grads = S.ssd_bwd(**c, **kw, dout=W.float(), dfinal_states=V)
    for name, w in zip(NAMES, grads):
        if c[name] is None:
            assert w is None, name
            continue
        if low:
            tol = (2e-2, 2e-2)
        else:
            tol = (1e-3, 1e-4) if name in ("x", "dt", "z") else (1e-3, 1e-3)
        assert_close_report(got[name], w, *tol, f"d{name}")


SHAPES = [
    # b, l, h, p, g, n
    (2, 64, 2, 16, 1, 16),
    (1, 100, 4, 32, 2, 32),
    (2, 130, 4, 64, 1, 128),
    (1, 200, 8, 16, 4, 64),
    (1, 37, 2, 64, 2, 48),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "b{}l{}h{}p{}g{}n{}".format(*s))
def test_forward_and_gradients_match_oracle(shape):
    c = case(*shape, seed=sum(shape))
    check(c, *run(c))


@pytest.mark.parametrize("opts", [
    dict(D="h", z=False, bias=False, init=True),
    dict(D=None, z=True, bias=True, init=True),
    dict(D="hp", z=False, bias=True, init=False),
], ids=["Dh-noz-init", "noD-z-init", "noz-bias"])
@pytest.mark.parametrize("softplus,limit", [(True, (0.0, float("inf"))), (True, (0.05, 0.6)),
                                            (False, (0.0, float("inf")))], ids=["sp", "sp-clamp", "raw"])
def test_options_match_oracle(opts, softplus, limit):
    c = case(2, 90, 4, 32, 2, 32, seed=5, **opts)
    if not softplus:
        c["dt"] = c["dt"].abs() * 0.3 + 0.05  # a positive step without softplus
    check(c, *run(c, softplus=softplus, limit=limit), softplus=softplus, limit=limit)


def test_raw_negative_steps_are_clamped():
    """Without softplus, a negative raw step is clamped to the default
    dt_limit (0, inf): step 0 and no raw-dt gradient there (mamba_ssm's and
    transformers' semantics; the oracle is pinned against transformers'
    mamba2_chunk_scan in tests/test_oracle_ssd.py)."""
    c = case(2, 150, 4, 32, 2, 32, seed=6, init=True)
    c["dt"] = c["dt"] + 0.8  # about half of dt + dt_bias below 0
    out, fin, got, W, V = run(c, softplus=False)
    check(c, out, fin, got, W, V, softplus=False)
    neg = (c["dt"] + c["dt_bias"][None, None]) < 0
    assert 0.2 < neg.float().mean().item() < 0.8
    assert torch.all(got["dt"].cpu()[neg] == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_storage(dtype):
    c = case(2, 150, 4, 64, 2, 64, seed=9, dtype=dtype)
    out, fin, got, W, V = run(c)
    assert out.dtype == dtype and got["x"].dtype == dtype and got["B"].dtype == dtype
    check(c, out, fin, got, W, V, low=True)


def test_long_sequence_2048_steps():
    """32 chunks: the state passing over many chunks, forward and backward."""
    c = case(1, 2048, 4, 64, 1, 64, seed=13, init=True)
    check(c, *run(c))


def test_no_grad_forward_equals_training_forward():
    c = case(1, 130, 4, 32, 2, 32, seed=3)
    dev = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    with torch.no_grad():
        a = mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=64, dt_softplus=True)
    b = mamba_cpu.mamba_chunk_scan_combined(**{k: None if v is None else v.requires_grad_() for k, v in dev.items()},
                                            chunk_size=64, dt_softplus=True)
    assert torch.equal(a, b.detach())


def test_empty_sequence_passes_the_initial_state_through():
    c = case(2, 0, 2, 16, 1, 16, seed=4, init=True)
    dev = {k: None if v is None else v.to(DEV).requires_grad_() for k, v in c.items()}
    out, fin = mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=64, return_final_states=True)
    assert out.shape == (2, 0, 2, 16)
    assert torch.equal(fin, dev["initial_states"])
    V = torch.randn_like(fin)
    (out.sum() + (fin * V).sum()).backward()
    assert torch.equal(dev["initial_states"].grad, V)
    for k in ("A", "D", "dt_bias"):
        assert torch.count_nonzero(dev[k].grad) == 0, k


def test_rejects_unsupported_shapes_and_options():
    c = case(1, 16, 2, 16, 1, 16)
    dev = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    seq = torch.zeros(1, 16, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="cu_seqlens"):
        mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=64, seq_idx=seq, return_varlen_states=True)
    with pytest.raises(ValueError, match="seq_idx"):
        mamba_cpu.mamba_chunk_scan_combined(**dev, chunk_size=64, seq_idx=seq[:, :8])
    bad = dict(dev, x=torch.randn(1, 16, 2, 24, device=DEV), z=None, D=None)
    with pytest.raises(NotImplementedError, match="headdim"):
        mamba_cpu.mamba_chunk_scan_combined(**bad, chunk_size=64)
    with pytest.raises(ValueError):
        mamba_cpu.mamba_chunk_scan_combined(**{k: None if v is None else v.cpu() for k, v in dev.items()},
                                            chunk_size=64)


def run_ops(c, head_block=0, chunk_pass=0, softplus=True, limit=(0.0, float("inf")), seed=1, seq=None):
    """Forward and backward through the operators with the chunk kernels'
    head block and the way chunk states are carried pinned: out, final
    states, the nine gradients of sum(out W) + sum(final V), and W, V.
    seq: packed-sequence ids (batch, seqlen) or None."""
    d = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    if d["D"] is not None and d["D"].dim() == 1:   # the operator takes D per channel
        d["D"] = d["D"][:, None].expand(d["x"].shape[2:]).contiguous()
    args = (d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["z"], d["dt_bias"], d["initial_states"],
            softplus, float(limit[0]), float(limit[1]))
    sq = None if seq is None else torch.as_tensor(seq, dtype=torch.int32).to(DEV)
    out, fin, saved, ysave = torch.ops.mamba_cpu.ssd_fwd(*args, True, head_block, chunk_pass, seq_idx=sq)
    gen = torch.Generator().manual_seed(seed)
    W = torch.randn(out.shape, generator=gen).to(out.dtype)
    V = torch.randn(fin.shape, generator=gen)
    g = torch.ops.mamba_cpu.ssd_bwd(W.to(DEV), V.to(DEV), *args, saved, ysave, head_block, chunk_pass,
                                    seq_idx=sq)
    torch.cuda.synchronize()
    return out, fin, g, W, V


@pytest.mark.parametrize("shape,blocks", [
    ((2, 130, 8, 32, 1, 64), (1, 2, 4, 8)),
    ((1, 200, 8, 16, 2, 32), (2, 4)),
    ((3, 70, 4, 64, 1, 128), (2, 4)),
], ids=["h8g1", "h8g2", "h4n128"])
def test_head_blocks_match_oracle(shape, blocks):
    """Workgroups walking 2, 4 or 8 heads of a group (C B^T shared, dB/dC
    summed over the block's heads in the accumulators, partials per head
    block): every head-block size against the oracle, and the forward
    bitwise equal across sizes (each head's arithmetic is the same)."""
    c = case(*shape, seed=sum(shape) + 1, init=True)
    want = S.ssd_fwd(**c, dt_softplus=True)
    first = None
    for hb in blocks:
        out, fin, g, W, V = run_ops(c, head_block=hb)
        print(f" head_block {hb}")
        assert_close_report(out, want[0], 1e-4, 1e-5, "out")
        assert_close_report(fin, want[1], 1e-4, 1e-5, "final_states")
        wg = S.ssd_bwd(**c, dt_softplus=True, dout=W.float(), dfinal_states=V)
        for name, got, w in zip(NAMES, g, wg):
            tol = (1e-3, 1e-4) if name in ("x", "dt", "z") else (1e-3, 1e-3)
            assert_close_report(got, w, *tol, f"d{name}")
        if first is None:
            first = (out, fin)
        else:
            assert torch.equal(out, first[0]) and torch.equal(fin, first[1])


def check_ops(c, got, softplus=True, limit=(0.0, float("inf")), low=False, seq=None):
    out, fin, g, W, V = got
    kw = dict(dt_softplus=softplus, dt_limit=limit, seq_idx=seq)
    want = S.ssd_fwd(**c, **kw)
    tol = (2e-2, 2e-2) if low else (1e-4, 1e-5)
    assert_close_report(out, want[0], *tol, "out")
    assert_close_report(fin, want[1], *tol, "final_states")
    wg = S.ssd_bwd(**c, **kw, dout=W.float(), dfinal_states=V)
    for name, got_g, w in zip(NAMES, g, wg):
        if c[name] is None:
            continue
        if name == "D" and c["D"].dim() == 1:   # per-channel dD back to the per-head D
            got_g = got_g.sum(-1)
        if low:
            tol = (2e-2, 2e-2)
        else:
            tol = (1e-3, 1e-4) if name in ("x", "dt", "z") else (1e-3, 1e-3)
        assert_close_report(got_g, w, *tol, f"d{name}")


@pytest.mark.parametrize("shape,opts", [
    ((2, 130, 4, 64, 1, 128), dict(init=True)),
    ((1, 200, 8, 16, 4, 64), dict(z=False)),
    ((3, 70, 4, 32, 2, 48), dict(init=True, D="h")),
    ((1, 37, 2, 64, 2, 16), dict(bias=False)),
    ((2, 300, 4, 48, 1, 32), dict(init=True, z=False, D=None)),
], ids=["n128-init", "p16-noz", "n48-init", "n16-short", "p48-noD"])
@pytest.mark.parametrize("chunk_pass", [1, 2], ids=["two-launch", "in-order"])
def test_chunk_passes_match_oracle(shape, opts, chunk_pass):
    """Chunk states carried by the two-launch form (chunk-end states for
    every chunk, then a passing launch) and by the in-order kernels (one
    workgroup per batch row, head and 64-state column block walking the
    chunks, column blocks of 64, 48 and 16 states): forward, final states and
    every gradient against the oracle, with and without initial states, z,
    D and dt_bias."""
    c = case(*shape, seed=sum(shape) + chunk_pass, **opts)
    check_ops(c, run_ops(c, chunk_pass=chunk_pass))


def test_chunk_passes_in_bf16_and_clamped():
    c = case(2, 130, 8, 64, 2, 64, seed=5, init=True, dtype=torch.bfloat16)
    for cp in (1, 2):
        check_ops(c, run_ops(c, chunk_pass=cp, limit=(0.05, 2.0)), limit=(0.05, 2.0), low=True)


def test_chunk_pass_must_be_known():
    c = case(1, 64, 2, 16, 1, 16)
    with pytest.raises(ValueError, match="chunk_pass"):
        run_ops(c, chunk_pass=3)


def test_head_block_must_divide_the_group():
    c = case(1, 64, 6, 16, 2, 16)
    with pytest.raises(ValueError, match="head_block"):
        run_ops(c, head_block=2)   # 3 heads per group


def test_opcheck_ssd_ops():
    c = case(1, 70, 2, 16, 1, 16, seed=6, init=True)
    d = {k: None if v is None else v.to(DEV) for k, v in c.items()}
    if d["D"] is not None and d["D"].dim() == 1:   # the operator takes D per channel
        d["D"] = d["D"][:, None].expand(d["x"].shape[2:]).contiguous()
    args = (d["x"], d["dt"], d["A"], d["B"], d["C"], d["D"], d["z"], d["dt_bias"], d["initial_states"],
            True, 0.0, float("inf"), True)
    torch.library.opcheck(torch.ops.mamba_cpu.ssd_fwd.default, args)
    out, fin, saved, ysave = torch.ops.mamba_cpu.ssd_fwd(*args)
    bargs = (torch.randn_like(out), torch.randn_like(fin)) + args[:12] + (saved, ysave)
    torch.library.opcheck(torch.ops.mamba_cpu.ssd_bwd.default, bargs)

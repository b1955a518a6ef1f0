"""Empty inputs (no steps, no batch rows) through every op on the GPU.

The reference's ops take them as they come: its scan kernels loop over zero
steps or rows (csrc/selective_scan.cpp:120-145, 168-248) and its conv
concatenates the initial states in front of x (ops/causal_conv1d.py:16-53).
The expected values are closed forms: with no steps the scan's state stays
at its zero start, so last_state = 0 whatever the inputs and every parameter
gradient is 0; a convolution over no steps hands its initial states through
as its final states (cat(initial_states, x)[..., -(width - 1):] with x
empty), so the final states' gradient reaches initial_states unchanged.
Nothing here may launch a kernel with an empty grid.
"""

import pytest
import torch

from mamba_cpu import (
    causal_conv1d_fn,
    causal_conv1d_update,
    mamba_chunk_scan_combined,
    selective_scan_fn,
    selective_state_update,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _scan_inputs(batch, dim, seqlen, dstate):
    g = torch.Generator().manual_seed(0)
    t = {
        "u": torch.randn(batch, dim, seqlen, generator=g),
        "delta": torch.rand(batch, dim, seqlen, generator=g),
        "A": -0.5 - torch.rand(dim, dstate, generator=g),
        "B": torch.randn(batch, dstate, seqlen, generator=g),
        "C": torch.randn(batch, dstate, seqlen, generator=g),
        "D": torch.randn(dim, generator=g),
        "z": torch.randn(batch, dim, seqlen, generator=g),
        "delta_bias": torch.rand(dim, generator=g),
    }
    return {k: v.to(DEV).requires_grad_() for k, v in t.items()}


@pytest.mark.parametrize("batch,dim,seqlen", [(2, 8, 0), (0, 8, 5), (0, 8, 0)])
def test_scan_without_steps_or_rows(batch, dim, seqlen):
    dstate = 4
    t = _scan_inputs(batch, dim, seqlen, dstate)
    print(f"scan batch {batch} dim {dim} seqlen {seqlen}", flush=True)
    out, last = selective_scan_fn(**t, delta_softplus=True, return_last_state=True)
    assert out.shape == (batch, dim, seqlen) and last.shape == (batch, dim, dstate)
    assert torch.count_nonzero(last).item() == 0
    w = torch.randn(batch, dim, dstate, device=DEV)
    ((last * w).sum() + out.sum()).backward()
    for name in ("u", "delta", "z", "B", "C"):
        assert t[name].grad.shape == t[name].shape, name
    for name in ("A", "D", "delta_bias"):
        assert t[name].grad.shape == t[name].shape, name
        assert torch.count_nonzero(t[name].grad).item() == 0, name
    torch.cuda.synchronize()


@pytest.mark.parametrize("with_init", [False, True])
def test_conv_without_steps_hands_initial_states_through(with_init):
    batch, dim, width = 2, 8, 4
    x = torch.randn(batch, dim, 0, device=DEV, requires_grad=True)
    w = torch.randn(dim, width, device=DEV, requires_grad=True)
    b = torch.randn(dim, device=DEV, requires_grad=True)
    init = torch.randn(batch, dim, width - 1, device=DEV, requires_grad=True) if with_init else None
    print(f"conv seqlen 0 with_init {with_init}", flush=True)
    out, final = causal_conv1d_fn(x, w, b, initial_states=init, return_final_states=True, activation="silu")
    assert out.shape == (batch, dim, 0) and final.shape == (batch, dim, width - 1)
    want = init.detach() if with_init else torch.zeros(batch, dim, width - 1, device=DEV)
    torch.testing.assert_close(final, want, rtol=0, atol=0)
    dfinal = torch.randn_like(final)
    (final * dfinal).sum().backward()
    assert torch.count_nonzero(w.grad).item() == 0 and torch.count_nonzero(b.grad).item() == 0
    assert x.grad is None or x.grad.shape == x.shape
    if with_init:
        torch.testing.assert_close(init.grad, dfinal, rtol=0, atol=0)


def test_conv_without_rows():
    x = torch.randn(0, 8, 10, device=DEV, requires_grad=True)
    w = torch.randn(8, 4, device=DEV, requires_grad=True)
    b = torch.randn(8, device=DEV, requires_grad=True)
    print("conv batch 0", flush=True)
    out = causal_conv1d_fn(x, w, b, activation="silu")
    assert out.shape == (0, 8, 10)
    out.sum().backward()
    assert torch.count_nonzero(w.grad).item() == 0 and torch.count_nonzero(b.grad).item() == 0


def test_decode_ops_without_rows():
    print("conv update and state update, batch 0", flush=True)
    x = torch.randn(0, 8, device=DEV)
    state = torch.randn(0, 8, 3, device=DEV)
    w = torch.randn(8, 4, device=DEV)
    assert causal_conv1d_update(x, state, w, activation="silu").shape == (0, 8)
    ssm = torch.randn(0, 8, 4, device=DEV)
    dt = torch.rand(0, 8, device=DEV)
    A = -torch.rand(8, 4, device=DEV)
    Bv, Cv = torch.randn(0, 4, device=DEV), torch.randn(0, 4, device=DEV)
    out = selective_state_update(ssm, x, dt, A, Bv, Cv, D=torch.randn(8, device=DEV), dt_softplus=True)
    assert out.shape == (0, 8)
    torch.cuda.synchronize()


def test_ssd_without_rows():
    batch, seqlen, nheads, headdim, dstate = 0, 96, 2, 16, 16
    g = torch.Generator().manual_seed(0)
    x = torch.randn(batch, seqlen, nheads, headdim, generator=g).to(DEV).requires_grad_()
    dt = torch.rand(batch, seqlen, nheads, generator=g).to(DEV).requires_grad_()
    A = (-torch.rand(nheads, generator=g)).to(DEV).requires_grad_()
    B = torch.randn(batch, seqlen, 1, dstate, generator=g).to(DEV).requires_grad_()
    C = torch.randn(batch, seqlen, 1, dstate, generator=g).to(DEV).requires_grad_()
    D = torch.randn(nheads, generator=g).to(DEV).requires_grad_()
    bias = torch.rand(nheads, generator=g).to(DEV).requires_grad_()
    print("ssd batch 0", flush=True)
    out, final = mamba_chunk_scan_combined(x, dt, A, B, C, 64, D=D, dt_bias=bias, dt_softplus=True,
                                           return_final_states=True)
    assert out.shape == x.shape and final.shape == (batch, nheads, headdim, dstate)
    out.sum().backward()
    for t in (A, D, bias):
        assert t.grad.shape == t.shape and torch.count_nonzero(t.grad).item() == 0
    torch.cuda.synchronize()

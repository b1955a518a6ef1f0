"""selective_state_update on the GPU.

Mirrors the reference's tests/test_selective_state_update.py (L single steps
equal the full scan; Mamba-2 head layout equals the flattened Mamba-1 layout)
and adds direct comparisons with the float64 oracle for both layouts, grouped
B/C, a bf16 state and state_batch_indices (which the reference rejects).
Tolerance rtol/atol 1e-5 (float32).
"""

import numpy as np
import pytest
import torch

from oracle import numerics as O

from mamba_cpu import selective_scan_fn, selective_state_update

pytestmark = pytest.mark.gpu
DEV = "cuda"


def close(got, want, rtol, atol, name=""):
    np.testing.assert_allclose(got.detach().float().cpu().numpy().astype(np.float64), want,
                               rtol=rtol, atol=atol, err_msg=name)


def test_steps_match_full_scan():
    torch.manual_seed(0)
    batch, dim, seqlen, dstate = 2, 16, 10, 8
    u = torch.randn(batch, dim, seqlen, device=DEV)
    delta = torch.rand(batch, dim, seqlen, device=DEV) * 0.5
    A = -torch.rand(dim, dstate, device=DEV) - 0.5
    B = torch.randn(batch, dstate, seqlen, device=DEV)
    C = torch.randn(batch, dstate, seqlen, device=DEV)
    D = torch.randn(dim, device=DEV)
    z = torch.randn(batch, dim, seqlen, device=DEV)
    dt_bias = torch.rand(dim, device=DEV) * 0.1

    full, last = selective_scan_fn(u, delta, A, B, C, D, z, dt_bias, True, return_last_state=True)
    want, want_last = O.selective_scan_fwd(u, delta, A, B, C, D, z, dt_bias, True)

    state = torch.zeros(batch, dim, dstate, device=DEV)
    steps = [
        selective_state_update(
            state, u[..., t], delta[..., t], A, B[..., t], C[..., t], D, z[..., t], dt_bias, True
        )
        for t in range(seqlen)
    ]
    torch.testing.assert_close(torch.stack(steps, -1), full, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(state, last, rtol=1e-5, atol=1e-5)
    close(torch.stack(steps, -1), want, 1e-5, 1e-5)
    close(state, want_last, 1e-5, 1e-5)


def test_multihead_matches_flattened():
    # Mamba-2 layout with ngroups=1 is Mamba-1 with dim = nheads * headdim.
    torch.manual_seed(0)
    batch, nheads, headdim, dstate = 2, 4, 3, 8
    state = torch.randn(batch, nheads, headdim, dstate, device=DEV)
    x = torch.randn(batch, nheads, headdim, device=DEV)
    dt = torch.rand(batch, nheads, headdim, device=DEV)
    A = -torch.rand(nheads, headdim, dstate, device=DEV)
    B = torch.randn(batch, 1, dstate, device=DEV)
    C = torch.randn(batch, 1, dstate, device=DEV)
    D = torch.randn(nheads, headdim, device=DEV)

    flat_state = state.reshape(batch, -1, dstate).clone()
    out = selective_state_update(state, x, dt, A, B, C, D)
    flat_out = selective_state_update(
        flat_state, x.reshape(batch, -1), dt.reshape(batch, -1), A.reshape(-1, dstate),
        B[:, 0], C[:, 0], D.reshape(-1),
    )
    torch.testing.assert_close(out.reshape(batch, -1), flat_out)
    torch.testing.assert_close(state.reshape(batch, -1, dstate), flat_state)


@pytest.mark.parametrize("multihead", [False, True])
def test_matches_oracle(multihead):
    torch.manual_seed(0)
    b, n = 2, 16
    lead = (4, 8) if multihead else (32,)
    state = torch.randn(b, *lead, n, device=DEV)
    x, dt, z = (torch.randn(b, *lead, device=DEV), torch.rand(b, *lead, device=DEV),
                torch.randn(b, *lead, device=DEV))
    A = -torch.rand(*lead, n, device=DEV) - 0.5
    B = torch.randn(b, 2, n, device=DEV) if multihead else torch.randn(b, n, device=DEV)
    C = torch.randn_like(B)
    D, dt_bias = torch.randn(*lead, device=DEV), torch.rand(*lead, device=DEV)
    want, want_state = O.selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, True)
    out = selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, True)
    close(out, want, 1e-5, 1e-5, "out")
    close(state, want_state, 1e-5, 1e-5, "state")


def test_bf16_state_and_inputs():
    torch.manual_seed(0)
    b, d, n = 3, 40, 16
    state = torch.randn(b, d, n, device=DEV).bfloat16()
    x, dt, z = (torch.randn(b, d, device=DEV).bfloat16(), torch.rand(b, d, device=DEV).bfloat16(),
                torch.randn(b, d, device=DEV).bfloat16())
    A = -torch.rand(d, n, device=DEV) - 0.5
    B, C = torch.randn(b, n, device=DEV), torch.randn(b, n, device=DEV)
    D = torch.randn(d, device=DEV)
    want, want_state = O.selective_state_update(state, x, dt, A, B, C, D, z, None, True)
    out = selective_state_update(state, x, dt, A, B, C, D, z, None, True)
    assert out.dtype == torch.bfloat16 and state.dtype == torch.bfloat16
    close(out, want, 2e-2, 2e-2)
    close(state, want_state, 2e-2, 2e-2)


@pytest.mark.parametrize("heads", [False, True])
def test_state_batch_indices_match_oracle(heads):
    """state_batch_indices (rows of a larger state, one out of range), which
    the reference rejects, against the oracle's restatement of mamba_ssm's
    semantics."""
    torch.manual_seed(5)
    b, h, p, n, rows = 3, 2, 8, 16, 7
    lead = (b, h, p) if heads else (b, h * p)
    prm = (h, p) if heads else (h * p,)
    state = torch.randn((rows,) + lead[1:] + (n,), device=DEV)
    x, z = torch.randn(lead, device=DEV), torch.randn(lead, device=DEV)
    dt = torch.rand(lead, device=DEV)
    A = -torch.rand(prm + (n,), device=DEV) - 0.5
    B = torch.randn((b, 1, n) if heads else (b, n), device=DEV)
    C = torch.randn((b, 1, n) if heads else (b, n), device=DEV)
    D, dtb = torch.randn(prm, device=DEV), torch.rand(prm, device=DEV) * 0.1
    idx = torch.tensor([5, 1, -1], dtype=torch.int32, device=DEV)
    want, want_state = O.selective_state_update(state, x, dt, A, B, C, D, z, dtb, True,
                                                state_batch_indices=idx.cpu().numpy())
    out = selective_state_update(state, x, dt, A, B, C, D, z, dtb, True, state_batch_indices=idx)
    close(out, want, 1e-5, 1e-5, "out")
    close(state, want_state, 1e-5, 1e-5, "state")


def test_rejects_malformed_state_batch_indices():
    s = torch.zeros(1, 4, 2, device=DEV)
    with pytest.raises(ValueError):
        selective_state_update(s, torch.zeros(1, 4, device=DEV), torch.zeros(1, 4, device=DEV),
                               torch.zeros(4, 2, device=DEV), torch.zeros(1, 2, device=DEV),
                               torch.zeros(1, 2, device=DEV),
                               state_batch_indices=torch.zeros(2, dtype=torch.int32, device=DEV))

"""Tensors past 4 GiB: the kernels address a tile with a 32-bit offset from a
64-bit, wave-uniform base, so rows that start beyond byte 2^32 must read and
write the same values as a small call on those rows alone.

Each case runs one call over float32 tensors of 4.3 GB each (the scan and
the conv: batch 2, dim 8208, seqlen 65536; the SSD scan: batch 2, seqlen
65600, 128 heads x 64, dstate 128), whose last rows start past byte 2^32, and
one call over the last 16 channels (heads) of batch row 1 only, then compares
those rows of every per-row result. The small call is pinned to the float64
oracle by the other tests; the two differ only in how the work is cut (time
chunks of the scan, head blocks and the state-passing form of the SSD scan),
which moves float32 results by a few ulps. Tolerances: rtol 1e-4 / atol 1e-5 on outputs and states, conftest's
gradient bounds on gradients.
"""

import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL, assert_close_report

from mamba_cpu import causal_conv1d_fn, mamba_chunk_scan_combined, selective_scan_fn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BATCH, DIM, SEQLEN, DSTATE = 2, 8208, 65536, 16
ROWS = slice(DIM - 16, DIM)


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_scan_rows_past_4_gib():
    assert BATCH * DIM * SEQLEN * 4 > 2**32
    g = torch.Generator(device=DEV).manual_seed(0)
    big = {
        "u": torch.randn(BATCH, DIM, SEQLEN, device=DEV, generator=g),
        "delta": 0.1 * torch.rand(BATCH, DIM, SEQLEN, device=DEV, generator=g),
        "A": -0.5 - torch.rand(DIM, DSTATE, device=DEV, generator=g),
        "B": torch.randn(BATCH, DSTATE, SEQLEN, device=DEV, generator=g),
        "C": torch.randn(BATCH, DSTATE, SEQLEN, device=DEV, generator=g),
        "D": torch.randn(DIM, device=DEV, generator=g),
        "z": torch.randn(BATCH, DIM, SEQLEN, device=DEV, generator=g),
        "delta_bias": 0.1 * torch.rand(DIM, device=DEV, generator=g),
    }
    dout = torch.randn(BATCH, DIM, SEQLEN, device=DEV, generator=g)
    per_row = ("u", "delta", "z")
    for k in per_row:
        big[k].requires_grad_()
    print(f"scan forward + backward over ({BATCH}, {DIM}, {SEQLEN}) float32", flush=True)
    out, last = selective_scan_fn(**big, delta_softplus=True, return_last_state=True)
    out.backward(dout)
    got = {"out": out[1:, ROWS].detach().clone(), "last": last[1:, ROWS].clone()}
    got.update({"d" + k: big[k].grad[1:, ROWS].clone() for k in per_row})
    del out, last
    small = {}
    for k, v in big.items():
        if k in per_row:
            small[k] = v.detach()[1:, ROWS].clone().requires_grad_()
        elif k in ("B", "C"):
            small[k] = v[1:].clone()
        else:
            small[k] = v[ROWS].clone()
    small_dout = dout[1:, ROWS].clone()
    del big, dout
    _free()
    print("scan over the last 16 channels of batch row 1", flush=True)
    out, last = selective_scan_fn(**small, delta_softplus=True, return_last_state=True)
    out.backward(small_dout)
    assert_close_report(got["out"], out.detach(), 1e-4, 1e-5, "out")
    assert_close_report(got["last"], last, 1e-4, 1e-5, "last_state")
    for k in per_row:
        assert_close_report(got["d" + k], small[k].grad, GRAD_RTOL, GRAD_ATOL[k], "d" + k)
    del got, small, out, last
    _free()


def test_conv_rows_past_4_gib():
    width = 4
    g = torch.Generator(device=DEV).manual_seed(1)
    x = torch.randn(BATCH, DIM, SEQLEN, device=DEV, generator=g).requires_grad_()
    w = torch.randn(DIM, width, device=DEV, generator=g) / 2
    b = torch.randn(DIM, device=DEV, generator=g) / 10
    dout = torch.randn(BATCH, DIM, SEQLEN, device=DEV, generator=g)
    print(f"conv forward + backward over ({BATCH}, {DIM}, {SEQLEN}) float32", flush=True)
    out = causal_conv1d_fn(x, w, b, activation="silu")
    out.backward(dout)
    got_out, got_dx = out[1:, ROWS].detach().clone(), x.grad[1:, ROWS].clone()
    xs = x.detach()[1:, ROWS].clone().requires_grad_()
    ds = dout[1:, ROWS].clone()
    del x, out, dout
    _free()
    print("conv over the last 16 channels of batch row 1", flush=True)
    out = causal_conv1d_fn(xs, w[ROWS].clone(), b[ROWS].clone(), activation="silu")
    out.backward(ds)
    assert_close_report(got_out, out.detach(), 1e-5, 1e-5, "conv out")
    assert_close_report(got_dx, xs.grad, 1e-5, 1e-5, "conv dx")
    del got_out, got_dx, xs, out
    _free()


def test_ssd_rows_past_4_gib():
    batch, seqlen, nheads, headdim, dstate = 2, 65600, 128, 64, 128
    assert batch * seqlen * nheads * headdim * 4 > 2**32
    heads = slice(nheads - 16, nheads)
    g = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(batch, seqlen, nheads, headdim, device=DEV, generator=g).requires_grad_()
    dt = (0.1 * torch.rand(batch, seqlen, nheads, device=DEV, generator=g)).requires_grad_()
    A = -0.5 - torch.rand(nheads, device=DEV, generator=g)
    B = torch.randn(batch, seqlen, 1, dstate, device=DEV, generator=g) / 8
    C = torch.randn(batch, seqlen, 1, dstate, device=DEV, generator=g) / 8
    D = torch.randn(nheads, device=DEV, generator=g)
    dout = torch.randn(batch, seqlen, nheads, headdim, device=DEV, generator=g)
    print(f"ssd forward + backward over ({batch}, {seqlen}, {nheads}, {headdim}) float32, dstate {dstate}",
          flush=True)
    out, final = mamba_chunk_scan_combined(x, dt, A, B, C, 64, D=D, return_final_states=True)
    out.backward(dout)
    got = {"out": out[1:, :, heads].detach().clone(), "final": final[1:, heads].clone(),
           "dx": x.grad[1:, :, heads].clone(), "ddt": dt.grad[1:, :, heads].clone()}
    xs = x.detach()[1:, :, heads].clone().requires_grad_()
    dts = dt.detach()[1:, :, heads].clone().requires_grad_()
    small = dict(A=A[heads].clone(), B=B[1:].clone(), C=C[1:].clone(), D=D[heads].clone())
    ds = dout[1:, :, heads].clone()
    del x, dt, out, final, dout, A, B, C, D
    _free()
    print("ssd over the last 16 heads of batch row 1", flush=True)
    out, final = mamba_chunk_scan_combined(xs, dts, small["A"], small["B"], small["C"], 64, D=small["D"],
                                           return_final_states=True)
    out.backward(ds)
    assert_close_report(got["out"], out.detach(), 1e-4, 1e-5, "ssd out")
    assert_close_report(got["final"], final.detach(), 1e-4, 1e-5, "ssd final states")
    assert_close_report(got["dx"], xs.grad, GRAD_RTOL, 1e-4, "ssd dx")
    assert_close_report(got["ddt"], dts.grad, GRAD_RTOL, 1e-4, "ssd ddt")
    del got, xs, dts, small, out, final
    _free()

"""Stream semantics of the ops: each runs on torch's current stream and none
waits for the GPU on the host.

The reference's ops are synchronous CPU calls; on the GPU the boundary is
stream-ordered instead: every kernel of a call (the scan's chunk summaries
and partial reduces, the conv's partial reduce, the SSD scan's state passes)
is enqueued on torch.cuda.current_stream() and the call returns without a
host synchronization. Two checks:

- inputs produced on a side stream behind a long queue of other work, then
  consumed there by forward and backward, give exactly the results of the
  same calls on the default stream (a kernel launched on another stream
  would read the inputs before they exist);
- behind that queue, the calls return to the host long before the stream
  drains.
"""

import time

import pytest
import torch

from mamba_cpu import causal_conv1d_fn, mamba_chunk_scan_combined, selective_scan_fn, selective_state_update

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs():
    g = torch.Generator(device=DEV).manual_seed(0)
    b, d, l, n = 2, 64, 700, 16
    scan = {
        "u": torch.randn(b, d, l, device=DEV, generator=g),
        "delta": 0.5 * torch.rand(b, d, l, device=DEV, generator=g),
        "A": -0.5 - torch.rand(d, n, device=DEV, generator=g),
        "B": torch.randn(b, n, l, device=DEV, generator=g),
        "C": torch.randn(b, n, l, device=DEV, generator=g),
        "D": torch.randn(d, device=DEV, generator=g),
        "z": torch.randn(b, d, l, device=DEV, generator=g),
        "delta_bias": 0.1 * torch.rand(d, device=DEV, generator=g),
    }
    conv = {"x": torch.randn(b, d, l, device=DEV, generator=g), "w": torch.randn(d, 4, device=DEV, generator=g),
            "bias": torch.randn(d, device=DEV, generator=g)}
    ssd = {
        "x": torch.randn(b, 300, 4, 32, device=DEV, generator=g),
        "dt": torch.rand(b, 300, 4, device=DEV, generator=g),
        "A": -torch.rand(4, device=DEV, generator=g),
        "B": torch.randn(b, 300, 1, 32, device=DEV, generator=g),
        "C": torch.randn(b, 300, 1, 32, device=DEV, generator=g),
    }
    upd = {"state": torch.randn(b, d, n, device=DEV, generator=g), "x": torch.randn(b, d, device=DEV, generator=g),
           "dt": torch.rand(b, d, device=DEV, generator=g), "B": torch.randn(b, n, device=DEV, generator=g),
           "C": torch.randn(b, n, device=DEV, generator=g)}
    grads = {"scan": torch.randn(b, d, l, device=DEV, generator=g),
             "conv": torch.randn(b, d, l, device=DEV, generator=g),
             "ssd": torch.randn(b, 300, 4, 32, device=DEV, generator=g)}
    return scan, conv, ssd, upd, grads


def _run(scan, conv, ssd, upd, grads, copy):
    """Forward and backward of every op; with copy, each input is first
    recomputed on the current stream (so it exists only once that stream
    reaches it)."""
    c = (lambda t: (t * 1.0).detach()) if copy else (lambda t: t.detach())
    res = {}
    s = {k: c(v).requires_grad_() for k, v in scan.items()}
    out, last = selective_scan_fn(**s, delta_softplus=True, return_last_state=True)
    out.backward(c(grads["scan"]))
    res.update(scan_out=out.detach(), scan_last=last, **{"scan_d" + k: v.grad for k, v in s.items()})
    x, w, bias = (c(conv[k]).requires_grad_() for k in ("x", "w", "bias"))
    out = causal_conv1d_fn(x, w, bias, activation="silu")
    out.backward(c(grads["conv"]))
    res.update(conv_out=out.detach(), conv_dx=x.grad, conv_dw=w.grad, conv_db=bias.grad)
    m = {k: c(v).requires_grad_() for k, v in ssd.items()}
    out = mamba_chunk_scan_combined(m["x"], m["dt"], m["A"], m["B"], m["C"], 64, dt_softplus=True)
    out.backward(c(grads["ssd"]))
    res.update(ssd_out=out.detach(), **{"ssd_d" + k: v.grad for k, v in m.items()})
    state = c(upd["state"]).clone()
    res["upd_out"] = selective_state_update(state, c(upd["x"]), c(upd["dt"]), c(scan["A"]), c(upd["B"]),
                                            c(upd["C"]), D=c(scan["D"]), dt_softplus=True)
    res["upd_state"] = state
    return res


def _busy(n):
    """About n x 11 ms of matrix products queued on the current stream."""
    a = torch.full((8192, 8192), 1.0 / 8192, device=DEV)
    for _ in range(n):
        a = a @ a
    return a


def test_ops_run_on_the_current_stream():
    inputs = _inputs()
    want = _run(*inputs, copy=False)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _busy(16)
        got = _run(*inputs, copy=True)
    torch.cuda.synchronize()
    for k, v in want.items():
        torch.testing.assert_close(got[k], v, rtol=0, atol=0, msg=lambda m, k=k: f"{k}: {m}")


def test_ops_return_before_the_stream_drains():
    inputs = _inputs()
    _run(*inputs, copy=True)  # first calls: library and kernel loading
    _busy(1)
    torch.cuda.synchronize()
    _busy(24)
    t_busy = time.perf_counter()
    _run(*inputs, copy=True)
    t_calls = time.perf_counter()
    torch.cuda.synchronize()
    t_end = time.perf_counter()
    print(f"after the op calls were queued the stream ran {1e3 * (t_end - t_busy):.0f} ms more; the calls "
          f"took {1e3 * (t_calls - t_busy):.1f} ms on the host", flush=True)
    assert t_end - t_busy > 0.1, "the queued products finished too fast to tell"
    assert t_calls - t_busy < 0.5 * (t_end - t_busy)

"""Forward + backward of the scan, the conv and the SSD scan captured into one
HIP graph (torch.cuda.CUDAGraph) and replayed on new inputs.

A training step replayed from a graph runs every kernel of these calls (chunk
summaries, partial reduces, state passes, the fill kernels that clear
partials) with the addresses captured once, so nothing in them may depend on
host work done at call time, synchronize, or clear memory with
hipMemsetAsync (whose graph nodes have given wrong results on replays after
the first). Each replay, with eager work and synchronizations between
replays, must equal the same calls run eagerly on the replay's inputs, bit for
bit (the kernels are deterministic: fixed-order reductions, no atomics).
"""

import pytest
import torch

from mamba_cpu import causal_conv1d_fn, mamba_chunk_scan_combined, selective_scan_fn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _draw(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    b, d, l, n = 2, 64, 1000, 16
    return {
        "u": torch.randn(b, d, l, device=DEV, generator=g),
        "delta": 0.5 * torch.rand(b, d, l, device=DEV, generator=g),
        "A": -0.5 - torch.rand(d, n, device=DEV, generator=g),
        "B": torch.randn(b, n, l, device=DEV, generator=g),
        "C": torch.randn(b, n, l, device=DEV, generator=g),
        "D": torch.randn(d, device=DEV, generator=g),
        "z": torch.randn(b, d, l, device=DEV, generator=g),
        "delta_bias": 0.1 * torch.rand(d, device=DEV, generator=g),
        "dout": torch.randn(b, d, l, device=DEV, generator=g),
        "cx": torch.randn(b, d, l, device=DEV, generator=g),
        "cw": torch.randn(d, 4, device=DEV, generator=g),
        "cb": torch.randn(d, device=DEV, generator=g),
        "sx": torch.randn(b, 200, 4, 32, device=DEV, generator=g),
        "sdt": torch.rand(b, 200, 4, device=DEV, generator=g),
        "sA": -torch.rand(4, device=DEV, generator=g),
        "sB": torch.randn(b, 200, 1, 32, device=DEV, generator=g),
        "sC": torch.randn(b, 200, 1, 32, device=DEV, generator=g),
        "sdout": torch.randn(b, 200, 4, 32, device=DEV, generator=g),
    }


SCAN = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
LEAVES = SCAN + ("cx", "cw", "cb", "sx", "sdt", "sA", "sB", "sC")


def _step(t):
    """Forward and backward of the three ops; gradients land in the leaves'
    .grad; returns the forward outputs."""
    out, last = selective_scan_fn(*(t[k] for k in SCAN), delta_softplus=True, return_last_state=True)
    cout = causal_conv1d_fn(t["cx"], t["cw"], t["cb"], activation="silu")
    sout = mamba_chunk_scan_combined(t["sx"], t["sdt"], t["sA"], t["sB"], t["sC"], 64, dt_softplus=True)
    torch.autograd.backward([out, last, cout, sout],
                            [t["dout"], torch.ones_like(last), t["dout"], t["sdout"]])
    return {"out": out, "last": last, "cout": cout, "sout": sout}


def _results(t, outs):
    r = {k: v.detach().clone() for k, v in outs.items()}
    r.update({"d" + k: t[k].grad.clone() for k in LEAVES})
    return r


def _eager(seed):
    t = _draw(seed)
    for k in LEAVES:
        t[k].requires_grad_()
    return _results(t, _step(t))


def test_training_calls_replay_from_a_graph():
    static = _draw(0)
    for k in LEAVES:
        static[k].requires_grad_()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up outside capture: library loading, allocator pools
            for k in LEAVES:
                static[k].grad = None
            _step(static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for k in LEAVES:
        static[k].grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(static)
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        fresh = _draw(seed)
        with torch.no_grad():
            for k, v in fresh.items():
                static[k].copy_(v)
        graph.replay()
        got = _results(static, outs)
        torch.cuda.synchronize()
        want = _eager(seed)  # eager work between replays
        torch.cuda.synchronize()
        print(f"replay with inputs of seed {seed}", flush=True)
        for k, v in want.items():
            torch.testing.assert_close(got[k], v, rtol=0, atol=0, msg=lambda m, k=k: f"seed {seed}, {k}: {m}")


def _mixer_draw(seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    b, d, l, N, R, Dm, width = 2, 64, 300, 16, 8, 32, 4
    r = lambda *s, sc=1.0: torch.randn(*s, device=DEV, generator=g) * sc  # noqa: E731
    return {
        "xz": r(b, l, 2 * d).transpose(1, 2), "conv_w": r(d, 1, width, sc=0.5), "conv_b": r(d, sc=0.3),
        "x_proj_w": r(R + 2 * N, d, sc=d ** -0.5), "dt_proj_w": r(d, R, sc=R ** -0.5),
        "out_proj_w": r(Dm, d, sc=d ** -0.5), "out_proj_b": r(Dm, sc=0.1),
        "A": -torch.exp(2 * torch.rand(d, N, device=DEV, generator=g)), "D": r(d),
        "delta_bias": torch.rand(d, device=DEV, generator=g) - 3, "dout": r(b, l, Dm),
    }


MIXER = ("xz", "conv_w", "conv_b", "x_proj_w", "dt_proj_w", "out_proj_w", "out_proj_b", "A", "D", "delta_bias")


def _mixer_step(t):
    from mamba_cpu import mamba_inner_fn

    out = mamba_inner_fn(t["xz"], t["conv_w"], t["conv_b"], t["x_proj_w"], t["dt_proj_w"], t["out_proj_w"],
                         t["out_proj_b"], t["A"], D=t["D"], delta_bias=t["delta_bias"], delta_softplus=True)
    out.backward(t["dout"])
    return out


def test_fused_mixer_replays_from_a_graph():
    """The fused Mamba-1 mixer (its x_proj / dt_proj / out_proj products go
    through rocBLAS from C++) captured forward + backward and replayed."""
    static = _mixer_draw(0)
    for k in MIXER:
        static[k] = static[k].detach().requires_grad_()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for k in MIXER:
                static[k].grad = None
            _mixer_step(static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for k in MIXER:
        static[k].grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _mixer_step(static)
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        fresh = _mixer_draw(seed)
        with torch.no_grad():
            for k, v in fresh.items():
                static[k].copy_(v)
        graph.replay()
        got = {"out": out.detach().clone(), **{"d" + k: static[k].grad.clone() for k in MIXER}}
        torch.cuda.synchronize()
        eager = _mixer_draw(seed)
        for k in MIXER:
            eager[k] = eager[k].detach().requires_grad_()
        want = {"out": _mixer_step(eager).detach(), **{"d" + k: eager[k].grad for k in MIXER}}
        torch.cuda.synchronize()
        print(f"mixer replay with inputs of seed {seed}", flush=True)
        for k, v in want.items():
            torch.testing.assert_close(got[k], v, rtol=0, atol=0, msg=lambda m, k=k: f"seed {seed}, {k}: {m}")

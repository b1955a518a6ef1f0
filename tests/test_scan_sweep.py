"""A seeded sweep of selective_scan_fn configurations on the GPU against the
float64 oracle: batch, channels, ragged sequence lengths (including the
16-step block edges), dstate (one to four state lanes), B/C group layouts
(shared, grouped, unequal, input-independent), the optional z / D /
delta_bias, softplus, bf16 storage and channel-contiguous (transposed)
u/delta/z, each forward and every gradient, plus the final state.
Tolerances as in tests/test_selective_scan.py: fp32 outputs rtol 1e-4 /
atol 1e-5 (gradients 1e-3 / 1e-4 after scaling by their magnitude), bf16
1e-2 / 2e-2."""

import numpy as np
import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL
from oracle import numerics as O

from mamba_cpu import selective_scan_fn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def configs(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        groups = ["none", "g1", "g2", "unequal", "2d"][i % 5]
        cfg = dict(
            batch=int(rng.integers(1, 4)),
            seqlen=int(rng.choice([1, 15, 16, 17, 31, 33, 64, 100, 129, 300])),
            dstate=int(rng.choice([1, 3, 8, 16, 17, 32, 40, 64])),
            groups=groups,
            has_z=bool(rng.integers(0, 2)), has_D=bool(rng.integers(0, 2)), has_bias=bool(rng.integers(0, 2)),
            softplus=bool(rng.integers(0, 2)),
            dtype=torch.bfloat16 if i % 6 == 5 else torch.float32,
            channels_last=i % 4 == 3,
            seed=i,
        )
        cfg["dim"] = int(rng.choice([4, 8, 16, 24, 40, 64]))
        out.append(cfg)
    return out


def build(cfg):
    g = torch.Generator().manual_seed(cfg["seed"])
    b, d, l, n = cfg["batch"], cfg["dim"], cfg["seqlen"], cfg["dstate"]
    dt = cfg["dtype"]
    rnd = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    groups = cfg["groups"]
    if groups == "none":
        B, C = rnd(b, n, l), rnd(b, n, l)
    elif groups == "g1":
        B, C = rnd(b, 1, n, l), rnd(b, 1, n, l)
    elif groups == "g2":
        B, C = rnd(b, 2, n, l), rnd(b, 2, n, l)
    elif groups == "unequal":
        B, C = rnd(b, 2, n, l), rnd(b, 4, n, l) if d % 4 == 0 else rnd(b, 1, n, l)
    else:
        B, C = rnd(d, n), rnd(b, n, l)

    def x(*s):
        t = rnd(*s).to(dt)
        return t.transpose(1, 2).contiguous().transpose(1, 2) if cfg["channels_last"] else t

    inp = dict(
        u=x(b, d, l), delta=(torch.rand(b, d, l, generator=g) * 0.5).to(dt), A=-torch.rand(d, n, generator=g) - 0.5,
        B=B, C=C, D=rnd(d) if cfg["has_D"] else None, z=x(b, d, l) if cfg["has_z"] else None,
        delta_bias=torch.rand(d, generator=g) * 0.1 if cfg["has_bias"] else None,
    )
    if cfg["channels_last"]:
        inp["delta"] = inp["delta"].transpose(1, 2).contiguous().transpose(1, 2)
    return {k: None if v is None else v.to(DEV).requires_grad_() for k, v in inp.items()}


def close(got, want, rtol, atol, name):
    np.testing.assert_allclose(got.detach().float().cpu().double().numpy(), want, rtol=rtol, atol=atol,
                               err_msg=name)


@pytest.mark.parametrize("cfg", configs(), ids=lambda c: (
    f"b{c['batch']}d{c['dim']}l{c['seqlen']}n{c['dstate']}-{c['groups']}"
    f"{'-z' if c['has_z'] else ''}{'-D' if c['has_D'] else ''}{'-bias' if c['has_bias'] else ''}"
    f"{'-sp' if c['softplus'] else ''}{'-bf16' if c['dtype'] == torch.bfloat16 else ''}"
    f"{'-cl' if c['channels_last'] else ''}"))
def test_scan_configuration_matches_oracle(cfg):
    inp = build(cfg)
    sp = cfg["softplus"]
    out, last = selective_scan_fn(**inp, delta_softplus=sp, return_last_state=True)
    want, want_last = O.selective_scan_fwd(**inp, delta_softplus=sp)
    f32 = cfg["dtype"] == torch.float32
    close(out, want, *((1e-4, 1e-5) if f32 else (1e-2, 1e-2)), "out")
    close(last, want_last, *((1e-4, 1e-5) if f32 else (1e-2, 1e-2)), "last_state")
    g = torch.Generator().manual_seed(cfg["seed"] + 100)
    W = torch.randn(*inp["u"].shape, generator=g).to(DEV)
    V = torch.randn(*last.shape, generator=g).to(DEV)
    ((out.float() * W).sum() + (last * V).sum()).backward()
    # a bf16 out's upstream gradient is W rounded to bf16: the oracle gets that
    wants = O.selective_scan_bwd(**inp, delta_softplus=sp, dout=W.to(cfg["dtype"]).float(),
                                 dlast_state=V)
    for k, w in zip(["u", "delta", "A", "B", "C", "D", "z", "delta_bias"], wants):
        if inp[k] is None:
            continue
        close(inp[k].grad, w, *((GRAD_RTOL, GRAD_ATOL[k]) if f32 else (2e-2, 2e-2)), k)

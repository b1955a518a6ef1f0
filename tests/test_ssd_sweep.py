"""A seeded sweep of mamba_chunk_scan_combined configurations on the GPU
against the float64 oracle (oracle/ssd.py): batch, ragged sequence lengths
around the 64-step chunk edges, headdim 16-64, dstate 16-128, 1-2 groups of
1-4 heads, D per head or per channel or absent, z, dt_bias, initial states,
softplus and the dt clamp, float32 / bfloat16 / float16 storage, and the
kernel forms pinned through the operators: the chunk states carried by two
launches or by the in-order kernels, and 1 to 4 heads per workgroup of the
chunk kernels. Forward, final states and every gradient; tolerances as in
tests/test_ssd.py (float32 outputs rtol 1e-4 / atol 1e-5, gradients rtol 1e-3
/ atol 1e-4 for x, dt, z and 1e-3 for the sums; 16-bit storage 2e-2)."""

import numpy as np
import pytest
import torch

from test_ssd import DEV, case, check_ops, run_ops

pytestmark = pytest.mark.gpu


def configs(n=24, seed=7):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        groups = int(rng.integers(1, 3))
        hpg = int(rng.choice([1, 2, 3, 4]))
        blocks = [d for d in (1, 2, 3, 4) if hpg % d == 0]
        cfg = dict(
            b=int(rng.integers(1, 4)),
            l=int(rng.choice([1, 17, 63, 64, 65, 100, 129, 200])),
            h=groups * hpg, g=groups,
            p=int(rng.choice([16, 32, 48, 64])),
            n=int(rng.choice([16, 32, 48, 64, 96, 128])),
            D=[None, "h", "hp"][i % 3],
            z=bool(rng.integers(0, 2)), bias=bool(rng.integers(0, 2)), init=bool(rng.integers(0, 2)),
            softplus=bool(rng.integers(0, 2)),
            limit=(0.01, 5.0) if i % 5 == 4 else (0.0, float("inf")),
            dtype=[torch.bfloat16, torch.float16][(i // 6) % 2] if i % 6 == 5 else torch.float32,
            chunk_pass=i % 3,
            head_block=0 if i % 4 == 0 else int(rng.choice(blocks)),
            seed=100 + i,
        )
        out.append(cfg)
    return out


def _id(c):
    return "b{b}l{l}h{h}g{g}p{p}n{n}-cp{chunk_pass}-hb{head_block}".format(**c)


@pytest.mark.parametrize("cfg", configs(), ids=_id)
def test_ssd_sweep(cfg):
    c = case(cfg["b"], cfg["l"], cfg["h"], cfg["p"], cfg["g"], cfg["n"], seed=cfg["seed"], D=cfg["D"],
             z=cfg["z"], bias=cfg["bias"], init=cfg["init"], dtype=cfg["dtype"])
    if not cfg["softplus"]:
        c["dt"] = c["dt"].abs() * 0.3 + 0.05  # a positive step without softplus
    print(f" {_id(cfg)} D={cfg['D']} z={cfg['z']} bias={cfg['bias']} init={cfg['init']} "
          f"softplus={cfg['softplus']} limit={cfg['limit']} {cfg['dtype']}", flush=True)
    got = run_ops(c, head_block=cfg["head_block"], chunk_pass=cfg["chunk_pass"], softplus=cfg["softplus"],
                  limit=cfg["limit"])
    check_ops(c, got, softplus=cfg["softplus"], limit=cfg["limit"], low=cfg["dtype"] != torch.float32)
    assert got[0].device.type == DEV

"""Writes tests/golden/scan_ref_vectors.npz: selective-scan forward/backward
vectors produced by the reference's own CPU kernels (csrc/selective_scan.cpp,
compiled from the reference sources into oracle/_ref/libmcpu_ref.so by
oracle/Makefile). The reference ships no data files, so these are the
known-answer vectors for the scan; a machine without the reference sources
checks against them.

    make -C oracle REF=/root/reference && python tests/golden/make_golden.py

Cases (seeded, float32):
  full   batch 2, dim 16, seqlen 70, dstate 16, 1 group, z + D + delta_bias,
         softplus, dlast_state given  (ragged last 16-step block)
  groups batch 1, dim 8, seqlen 33, dstate 4, 2 groups, no z/D/bias, no softplus
  c1s    batch 1, dim 16, seqlen 160, dstate 16, the forward-only workload's
         input recipe (A = -U(0,1), softplus, no z/bias) at reduced dim/seqlen
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import ref as R  # noqa: E402


def case(name, b, d, l, n, g, full, softplus, dlast, seed, a_recipe="exp"):
    rng = np.random.default_rng(seed)
    f = np.float32
    u = rng.standard_normal((b, d, l)).astype(f)
    # without softplus, delta is the step itself: keep it positive so the scan stays stable
    delta = (rng.standard_normal((b, d, l)) if softplus else rng.random((b, d, l)) * 0.5).astype(f)
    if a_recipe == "exp":
        A = (-np.exp(rng.random((d, n)) * np.log(16))).astype(f)
    else:
        A = (-rng.random((d, n))).astype(f)
    B = rng.standard_normal((b, g, n, l)).astype(f)
    C = rng.standard_normal((b, g, n, l)).astype(f)
    D = rng.standard_normal(d).astype(f) if full else None
    z = rng.standard_normal((b, d, l)).astype(f) if full else None
    bias = (rng.random(d) * 2 - 4).astype(f) if full else None
    dout = rng.standard_normal((b, d, l)).astype(f)
    dls = rng.standard_normal((b, d, n)).astype(f) if dlast else None
    Bk, Ck = R.kernel_bc(B), R.kernel_bc(C)
    out, last = R.scan_fwd(u, delta, A, Bk, Ck, D, z, bias, softplus)
    du, ddelta, dA, dB, dC, dD, dz, dbias = R.scan_bwd(u, delta, A, Bk, Ck, D, z, bias, softplus,
                                                        dout, dls)
    rec = dict(u=u, delta=delta, A=A, B=B, C=C, dout=dout, out=out, last_state=last, du=du,
               ddelta=ddelta, dA=dA, dB=np.swapaxes(dB, -1, -2), dC=np.swapaxes(dC, -1, -2),
               softplus=np.array(softplus))
    for k, v in (("D", D), ("z", z), ("delta_bias", bias), ("dlast_state", dls)):
        if v is not None:
            rec[k] = v
    if D is not None:
        rec["dD"] = dD
    if z is not None:
        rec["dz"] = dz
    if bias is not None:
        rec["ddelta_bias"] = dbias
    return {f"{name}/{k}": v for k, v in rec.items()}


def main():
    if not R.available():
        sys.exit("oracle/_ref/libmcpu_ref.so is not built: make -C oracle REF=/root/reference")
    assert R.set_cpu_isa("default")  # the reference's portable path
    data = {}
    data.update(case("full", 2, 16, 70, 16, 1, True, True, True, seed=1))
    data.update(case("groups", 1, 8, 33, 4, 2, False, False, False, seed=2))
    data.update(case("c1s", 1, 16, 160, 16, 1, False, True, False, seed=0, a_recipe="uniform"))
    np.savez_compressed(os.path.join(HERE, "scan_ref_vectors.npz"), **data)


if __name__ == "__main__":
    main()

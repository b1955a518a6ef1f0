#!/usr/bin/env python
"""Selective-scan forward + backward throughput on one MI355X.

One step = selective_scan_fn forward and backward (torch.autograd.grad) over
the fp32 workload batch 8, dim 1536, seqlen 1024, dstate 16, one B/C group,
with z, D, delta_bias and softplus, on synthetic seeded inputs already in HBM.
The headline value is algorithmic bytes per step (every input read once, every
output written once) divided by the measured step time, in GB/s.

Also reported, on one JSON line:
  roofline      the backward launch sequence (dominant), timed with HIP events
                on the op's stream over the timed region, against 8 TB/s HBM;
  cpu_baseline  the reference's own CPU kernels (oracle/_ref, built from the
                reference sources) on the same workload on this host's cores;
  extra         forward-only time of the same workload, and Mamba-130M
                (random init, 24 layers, d_model 768) prefill tokens/s for
                4 x 1024 tokens through the patched Hugging Face model.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "mamba-cpu_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "selective_scan fwd+bwd HBM GB/s & % peak; Mamba-130M prefill tokens/s"
B_, D_, L_, N_, G_ = 8, 1536, 1024, 16, 1


def algorithmic_bytes(b, d, l, n, g, e=4):
    """Compulsory bytes: each input read once, each output written once.
    Forward reads u, delta, z, B, C, A, D, delta_bias and writes out; backward
    reads u, delta, z, dout, B, C, A, D, delta_bias and writes du, ddelta, dz,
    dB, dC, dA, dD, ddelta_bias."""
    x = b * d * l * e
    bc = b * g * l * n * 4
    params = (d * n + 2 * d) * 4
    fwd = 3 * x + 2 * bc + params + x
    bwd = 4 * x + 2 * bc + params + 3 * x + 2 * bc + params
    return fwd, bwd


def make_inputs(torch, dev):
    g = torch.Generator(device=dev).manual_seed(0)
    u = torch.randn(B_, D_, L_, generator=g, device=dev)
    delta = torch.randn(B_, D_, L_, generator=g, device=dev)
    z = torch.randn(B_, D_, L_, generator=g, device=dev)
    delta_bias = torch.rand(D_, generator=g, device=dev) * 2 - 4          # U(-4, -2)
    A = -torch.exp(torch.rand(D_, N_, generator=g, device=dev) * math.log(16))
    B = torch.randn(B_, G_, N_, L_, generator=g, device=dev)
    C = torch.randn(B_, G_, N_, L_, generator=g, device=dev)
    D = torch.randn(D_, generator=g, device=dev)
    gout = torch.randn(B_, D_, L_, generator=g, device=dev)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=delta_bias), gout


def cpu_baseline(inputs, gout, fwd_bytes, bwd_bytes):
    """The reference's CPU kernels (csrc/selective_scan.cpp, built from source
    into oracle/_ref) on the same workload, warm-up 1 + timed iterations as in
    the reference's benchmarks/bench_selective_scan.py:16-22."""
    from oracle import ref as R

    if not R.available():
        return None
    threads = int(os.environ.get("MCPU_BENCH_CPU_THREADS", min(os.cpu_count() or 1, 16)))
    a = {k: v.detach().float().cpu().numpy() for k, v in inputs.items()}
    Bk, Ck = R.kernel_bc(a["B"]), R.kernel_bc(a["C"])
    dout = gout.cpu().numpy()

    def run():
        R.scan_fwd(a["u"], a["delta"], a["A"], Bk, Ck, a["D"], a["z"], a["delta_bias"], True, threads)
        R.scan_bwd(a["u"], a["delta"], a["A"], Bk, Ck, a["D"], a["z"], a["delta_bias"], True, dout, None,
                   threads)

    run()
    iters = 3
    t0 = time.perf_counter()
    for _ in range(iters):
        run()
    sec = (time.perf_counter() - t0) / iters
    return {
        "value": round((fwd_bytes + bwd_bytes) / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"the full workload (batch {B_}, dim {D_}, seqlen {L_}, dstate {N_}, fp32, fwd+bwd), "
                  f"1 warm-up + {iters} timed iterations, {R.cpu_isa()} kernels; "
                  f"{sec * 1e3:.1f} ms per fwd+bwd",
    }


def prefill_tokens_per_s(torch, dev, iters=3):
    """Random-init Mamba-130M architecture through the patched HF model, fp32."""
    import transformers

    import mamba_cpu.hf

    mamba_cpu.hf.patch_transformers()
    torch.manual_seed(0)
    cfg = transformers.MambaConfig(num_hidden_layers=24, hidden_size=768, state_size=16, expand=2,
                                   conv_kernel=4, vocab_size=50280)
    model = transformers.MambaForCausalLM(cfg).to(dev).eval()
    ids = torch.randint(0, 50280, (4, 1024), device=dev)
    with torch.no_grad():
        model(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            model(ids)
        torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / iters
    del model
    torch.cuda.empty_cache()
    return 4 * 1024 / sec, sec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part of it "
              f"(got --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import torch

    import mamba_cpu
    from mamba_cpu import selective_scan_fn

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inputs, gout = make_inputs(torch, dev)
    leaves = {k: v.clone().requires_grad_() for k, v in inputs.items()}
    order = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]
    fwd_bytes, bwd_bytes = algorithmic_bytes(B_, D_, L_, N_, G_)
    stream = torch.cuda.current_stream(dev)

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        out = selective_scan_fn(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"],
                                leaves["D"], leaves["z"], leaves["delta_bias"], delta_softplus=True)
        if ev is not None:
            ev[1].record(stream)
        grads = torch.autograd.grad(out, [leaves[k] for k in order], gout)
        if ev is not None:
            ev[2].record(stream)
        return grads

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in events) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in events) / args.steps
    gbs = (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e9

    # Forward alone (no autograd), same workload.
    with torch.no_grad():
        for _ in range(3):
            selective_scan_fn(**inputs, delta_softplus=True)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            selective_scan_fn(**inputs, delta_softplus=True)
        e1.record(stream)
        torch.cuda.synchronize()
        fwd_only_ms = e0.elapsed_time(e1) / args.steps

    bwd_gbs = bwd_bytes / (bwd_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "scan_bwd_b8_d1536_l1024_n16_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    extra = {
        "fwd_ms_in_step": round(fwd_ms, 4),
        "bwd_ms_in_step": round(bwd_ms, 4),
        "fwd_only_ms": round(fwd_only_ms, 4),
        "fwd_only_GBps": round(fwd_bytes / (fwd_only_ms * 1e-3) / 1e9, 1),
        "algorithmic_bytes": {"fwd": fwd_bytes, "bwd": bwd_bytes},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "library": mamba_cpu._C.version(),
    }
    if not args.no_prefill:
        try:
            tps, sec = prefill_tokens_per_s(torch, dev)
            extra["mamba130m_prefill_tokens_per_s"] = round(tps, 1)
            extra["mamba130m_prefill_ms"] = round(sec * 1e3, 2)
        except Exception as exc:  # reported, not hidden
            extra["mamba130m_prefill_error"] = repr(exc)

    cpu = None if args.no_cpu_baseline else cpu_baseline(inputs, gout, fwd_bytes, bwd_bytes)

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded normal/uniform inputs of the stated shapes)",
        "config": {
            "workload": "selective_scan_fn forward+backward, fp32, batch 8, dim 1536, seqlen 1024, "
                        "dstate 16, 1 group, z + D + delta_bias, softplus",
            "batch": B_, "dim": D_, "seqlen": L_, "dstate": N_, "ngroups": G_,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "selective-scan backward launch (scan_bwd_kernel + its dB/dC/dA/dD/ddelta_bias reduce kernels)",
            "achieved": round(bwd_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()

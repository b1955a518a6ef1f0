"""Parity at the full sizes of the measured workloads, on the production paths.

Each workload is drawn with its stated recipe on the CPU (seed 0), run on the
GPU through the public API, and compared with the reference's own CPU kernels
(oracle/_ref, built from csrc/selective_scan.cpp; float32) and, where it runs
in seconds, with the float64 oracle:

  scan, forward, fp32        batch 1, dim 1536, seqlen 2048, dstate 16
  scan, fwd+bwd, fp32        batch 8, dim 1536, seqlen 1024, dstate 16, z, D,
                             delta_bias: the training path (forward with block
                             checkpoints and saved y, then the unchunked
                             12-wave backward that reads them)
  scan, fwd+bwd, bf16        batch 1, dim 5120, seqlen 16384, dstate 16: the
                             time-chunked forward and backward
  conv, fwd+bwd, fp32/bf16   batch 8, dim 3072, seqlen 2048, width 4, silu,
                             against the reference's ATen conv path
                             (oracle/cpu_torch.py)
  conv update                state (64, 3072, 3), 256 single-token steps
and the long shapes of the reference's upstream-parity test
(tests/test_upstream.py:57-75) against the float64 oracle.

Tolerances (unscaled, |got - want| <= atol + rtol |want|): float32 outputs
rtol 1e-4 / atol 1e-5 (at the forward-only workload, where float32 itself
cannot meet that, the reference kernels' own error sets the bar: see its
test); float32 gradients conftest.GRAD_RTOL / GRAD_ATOL; bf16-stored results
(out, and the gradients of bf16 inputs: du, ddelta, dB, dC, conv out and dx)
rtol 1e-2 / atol 1e-3, about two bf16 roundings; float32 results computed
from bf16 inputs (last state, dA, dD, conv dweight/dbias) the float32
gradient bounds, since both sides see the same bf16 values widened to
float32.
"""

import math
import os

import numpy as np
import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL, assert_close_report
from oracle import numerics as O
from oracle import ref as R

import mamba_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda"
THREADS = min(os.cpu_count() or 1, 16)
NAMES = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")


def note(msg):
    print(msg, flush=True)


def need_ref():
    if not R.available():
        pytest.skip("oracle/_ref (the reference's CPU kernels) is not built")


def scan_c1():
    """Forward-only workload: u, delta ~ N(0,1) (1, 1536, 2048); A = -U(0,1)
    (1536, 16); B, C ~ N(0,1) (1, 16, 2048); D ~ N(0,1) (1536); softplus."""
    g = torch.Generator().manual_seed(0)
    b, d, l, n = 1, 1536, 2048, 16
    return dict(u=torch.randn(b, d, l, generator=g), delta=torch.randn(b, d, l, generator=g),
                A=-torch.rand(d, n, generator=g), B=torch.randn(b, n, l, generator=g),
                C=torch.randn(b, n, l, generator=g), D=torch.randn(d, generator=g))


def scan_c2():
    """Training-step workload: u, delta, z ~ N(0,1) (8, 1536, 1024);
    delta_bias ~ U(-4,-2); A = -exp(U(0, ln 16)) (1536, 16); B, C ~ N(0,1)
    (8, 1, 16, 1024); D ~ N(0,1); softplus; upstream gradient ~ N(0,1)."""
    g = torch.Generator().manual_seed(0)
    b, d, l, n = 8, 1536, 1024, 16
    inp = dict(u=torch.randn(b, d, l, generator=g), delta=torch.randn(b, d, l, generator=g),
               z=torch.randn(b, d, l, generator=g),
               delta_bias=torch.rand(d, generator=g) * 2 - 4,
               A=-torch.exp(torch.rand(d, n, generator=g) * math.log(16)),
               B=torch.randn(b, 1, n, l, generator=g), C=torch.randn(b, 1, n, l, generator=g),
               D=torch.randn(d, generator=g))
    return inp, torch.randn(b, d, l, generator=g)


def scan_c5():
    """Long-sequence workload: u, delta, B, C in bf16 ~ N(0,1), u/delta
    (1, 5120, 16384), B/C (1, 16, 16384); A = -exp(U(0, ln 16)) and D ~ N(0,1)
    in fp32; softplus; upstream gradient ~ N(0,1) in bf16."""
    g = torch.Generator().manual_seed(0)
    b, d, l, n = 1, 5120, 16384, 16
    bf = torch.bfloat16
    inp = dict(u=torch.randn(b, d, l, generator=g).to(bf), delta=torch.randn(b, d, l, generator=g).to(bf),
               B=torch.randn(b, n, l, generator=g).to(bf), C=torch.randn(b, n, l, generator=g).to(bf),
               A=-torch.exp(torch.rand(d, n, generator=g) * math.log(16)),
               D=torch.randn(d, generator=g))
    return inp, torch.randn(b, d, l, generator=g).to(bf)


def gpu_fwd_bwd(inp, dout, softplus=True):
    """out, last_state and every gradient through selective_scan_fn's
    autograd on the GPU (the training path)."""
    leaves = {k: v.to(DEV).requires_grad_() for k, v in inp.items()}
    out, last = mamba_cpu.selective_scan_fn(**leaves, delta_softplus=softplus, return_last_state=True)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    grads = {k: v.grad for k, v in leaves.items()}
    return out.detach(), last.detach(), grads


def ref_fwd_bwd(inp, dout, softplus=True):
    """The reference's kernels on float32 copies of the same inputs."""
    a = {k: inp.get(k) for k in NAMES}
    Bk, Ck = R.kernel_bc(a["B"]), R.kernel_bc(a["C"])
    out, last = R.scan_fwd(a["u"], a["delta"], a["A"], Bk, Ck, a["D"], a["z"], a["delta_bias"], softplus,
                           THREADS)
    grads = R.scan_bwd(a["u"], a["delta"], a["A"], Bk, Ck, a["D"], a["z"], a["delta_bias"], softplus,
                       dout, None, THREADS)
    want = {}
    for k, v in zip(NAMES, grads):
        if k in ("B", "C"):
            v = np.swapaxes(v, -1, -2).reshape(inp[k].shape)  # kernel layout -> the input's
        if inp.get(k) is not None:
            want[k] = v
    return out, last, want


def test_forward_fp32_b1_d1536_l2048():
    """The forward-only workload (the time-chunked forward at batch 1) against
    the float64 oracle and the reference's kernels.

    Here A = -U(0, 1) decays slowly, so over 2048 steps the states grow to a
    few hundred and out = <h, C> + D u is a 16-term sum that cancels to
    values near zero: float32 cannot meet atol 1e-5 there. The reference's
    own kernels miss it against float64 on 27 of 3.1 M elements (largest error
    2.6e-4 at |out| up to 309). So the float32 check is: the GPU's error
    against float64 is within 1.5 times the reference kernels' own (the
    largest error, and the count of elements beyond rtol 1e-4 / atol 1e-5),
    and every element meets rtol 1e-4 / atol 1e-3 against both. Measured on
    an MI355X: largest error 2.0e-4, 18 elements beyond (v_exp_f32's slight
    low bias, compounded over the slowly decaying steps, gave 5.4e-4 and 52
    before the chunked forward carried each block's start state with one
    exponential of its summed step)."""
    need_ref()
    inp = scan_c1()
    note("scan fwd fp32 (1, 1536, 2048, 16): GPU")
    out, last = mamba_cpu.selective_scan_fn(**{k: v.to(DEV) for k, v in inp.items()}, delta_softplus=True,
                                            return_last_state=True)
    torch.cuda.synchronize()
    out, last = out.cpu().double().numpy(), last.cpu().double().numpy()
    note("  reference kernels")
    Bk, Ck = R.kernel_bc(inp["B"]), R.kernel_bc(inp["C"])
    rout, rlast = R.scan_fwd(inp["u"], inp["delta"], inp["A"], Bk, Ck, inp["D"], None, None, True, THREADS)
    note("  float64 oracle")
    wout, wlast = O.selective_scan_fwd(**inp, delta_softplus=True)
    for name, got in (("GPU", out), ("reference", rout)):
        assert_close_report(got, wout, 1e-4, 1e-3, f"out ({name}) vs float64")
    assert_close_report(out, rout, 1e-4, 1e-3, "out vs reference")
    assert_close_report(last, wlast, 1e-4, 1e-5, "last_state vs float64")
    assert_close_report(last, rlast, 1e-4, 1e-5, "last_state vs reference")
    gerr, rerr = np.abs(out - wout), np.abs(rout - wout)
    bound = 1e-5 + 1e-4 * np.abs(wout)
    g_over, r_over = int((gerr > bound).sum()), int((rerr > bound).sum())
    note(f"  largest error vs float64: GPU {gerr.max():.3g}, reference {rerr.max():.3g}; elements beyond "
         f"rtol 1e-4 / atol 1e-5: GPU {g_over}, reference {r_over} of {out.size}")
    assert gerr.max() <= 1.5 * rerr.max()
    assert g_over <= 1.5 * max(r_over, 1)


def test_training_step_fp32_b8_d1536_l1024():
    """The headline training step: forward with checkpoints and saved y, then
    the backward the library picks for this shape: 12-wave workgroups (checked
    through the workspace size, which is the 12-wave one) in a single time
    chunk, reading y back. Against the float64 oracle and the reference's
    kernels."""
    import ctypes

    from mamba_cpu import _C
    from scan_abi import scan_args

    need_ref()
    inp, dout = scan_c2()
    # The production choice for this shape, as the library sizes it.
    dev_inp = {k: v.to(DEV) for k, v in inp.items()}
    Bk, Ck = (dev_inp[k].transpose(-1, -2) for k in ("B", "C"))
    a = scan_args(dev_inp["u"], dev_inp["delta"], dev_inp["A"], Bk, Ck, dev_inp["D"], dev_inp["z"],
                  dev_inp["delta_bias"], True)
    a.ckpt = 64

    def ws(waves):
        a.bwd_waves = waves
        return _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a))

    assert ws(0) == ws(12) != ws(4)
    del dev_inp, Bk, Ck
    note("scan fwd+bwd fp32 (8, 1536, 1024, 16) z/D/bias: GPU")
    out, last, got = gpu_fwd_bwd(inp, dout)
    note("  reference kernels")
    rout, rlast, rgrads = ref_fwd_bwd(inp, dout.numpy())
    assert_close_report(out, rout, 1e-4, 1e-5, "out vs reference")
    assert_close_report(last, rlast, 1e-4, 1e-5, "last_state vs reference")
    for k, w in rgrads.items():
        assert_close_report(got[k], w, GRAD_RTOL, GRAD_ATOL[k], f"d{k} vs reference")
    note("  float64 oracle (about half a minute)")
    wout, wlast = O.selective_scan_fwd(**inp, delta_softplus=True)
    assert_close_report(out, wout, 1e-4, 1e-5, "out vs float64")
    assert_close_report(last, wlast, 1e-4, 1e-5, "last_state vs float64")
    wgrads = O.selective_scan_bwd(**inp, delta_softplus=True, dout=dout)
    for k, w in zip(NAMES, wgrads):
        assert_close_report(got[k], w, GRAD_RTOL, GRAD_ATOL[k], f"d{k} vs float64")


def test_long_sequence_bf16_b1_d5120_l16384():
    """The long bf16 sequence, time-chunked in both directions, against the
    reference's kernels on float32 copies of the same bf16 values."""
    need_ref()
    inp, dout = scan_c5()
    note("scan fwd+bwd bf16 (1, 5120, 16384, 16): GPU")
    out, last, got = gpu_fwd_bwd(inp, dout)
    # each gradient comes back in its input's dtype: bf16 for u, delta, B, C
    for k in ("u", "delta", "B", "C"):
        assert got[k].dtype == torch.bfloat16, k
    assert out.dtype == torch.bfloat16 and got["A"].dtype == got["D"].dtype == torch.float32
    note("  reference kernels")
    rout, rlast, rgrads = ref_fwd_bwd(inp, dout.float().numpy())
    assert_close_report(out, rout, 1e-2, 1e-3, "out (bf16) vs reference")
    assert_close_report(last, rlast, GRAD_RTOL, 1e-4, "last_state vs reference")
    for k, w in rgrads.items():
        if got[k].dtype == torch.bfloat16:
            assert_close_report(got[k], w, 1e-2, 1e-3, f"d{k} (bf16) vs reference")
        else:
            assert_close_report(got[k], w, GRAD_RTOL, GRAD_ATOL[k], f"d{k} vs reference")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_conv_fwd_bwd_b8_d3072_l2048(dtype):
    """causal_conv1d_fn forward and backward at the conv workload against the
    reference's ATen path (F.pad + depthwise F.conv1d in the weight's dtype +
    silu, autograd) on the same values."""
    from oracle import cpu_torch as CT

    g = torch.Generator().manual_seed(0)
    b, d, l, w = 8, 3072, 2048, 4
    x = torch.randn(b, d, l, generator=g).to(dtype)
    wt = torch.randn(d, w, generator=g) * 0.5
    bias = torch.randn(d, generator=g) * 0.1 ** 0.5
    dout = torch.randn(b, d, l, generator=g).to(dtype)
    note(f"conv fwd+bwd {dtype} (8, 3072, 2048, 4) silu: GPU")
    gx, gw, gb = (t.to(DEV).requires_grad_() for t in (x, wt, bias))
    out = mamba_cpu.causal_conv1d_fn(gx, gw, gb, activation="silu")
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    note("  reference ATen path")
    cx, cw, cb = (t.clone().requires_grad_() for t in (x, wt, bias))
    prev = torch.get_num_threads()
    torch.set_num_threads(THREADS)
    try:
        cout = CT.causal_conv1d_fn(cx, cw, cb, activation="silu")
        cout.backward(dout)
    finally:
        torch.set_num_threads(prev)
    if dtype == torch.float32:
        assert_close_report(out, cout, 1e-4, 1e-5, "out")
        assert_close_report(gx.grad, cx.grad, GRAD_RTOL, 1e-4, "dx")
    else:
        assert out.dtype == torch.bfloat16 and gx.grad.dtype == torch.bfloat16
        assert_close_report(out, cout, 1e-2, 1e-3, "out (bf16)")
        assert_close_report(gx.grad, cx.grad, 1e-2, 1e-3, "dx (bf16)")
    assert_close_report(gw.grad, cw.grad, GRAD_RTOL, 1e-3, "dweight")
    assert_close_report(gb.grad, cb.grad, GRAD_RTOL, 1e-3, "dbias")


def test_conv_update_b64_d3072_256_steps():
    """256 single-token causal_conv1d_update steps on a (64, 3072, 3) state:
    every step's output and the final state against the reference's ATen
    update path."""
    from oracle import cpu_torch as CT

    g = torch.Generator().manual_seed(0)
    b, d, w, steps = 64, 3072, 4, 256
    state = torch.randn(b, d, w - 1, generator=g)
    xs = torch.randn(steps, b, d, generator=g)
    wt = torch.randn(d, w, generator=g) * 0.5
    bias = torch.randn(d, generator=g) * 0.1 ** 0.5
    note("conv update (64, 3072, 3) x 256 steps: GPU")
    gs, gxs, gw, gb = (t.to(DEV) for t in (state, xs, wt, bias))
    outs = torch.stack([mamba_cpu.causal_conv1d_update(gxs[i], gs, gw, gb, activation="silu")
                        for i in range(steps)])
    torch.cuda.synchronize()
    note("  reference ATen path")
    cs = state.clone()
    couts = torch.stack([CT.causal_conv1d_update(xs[i], cs, wt, bias, activation="silu")
                         for i in range(steps)])
    assert_close_report(outs, couts, 1e-4, 1e-5, "outputs")
    assert_close_report(gs, cs, 0, 0, "final state")  # a shift of the inputs: exact


def upstream_case(batch, dim, seqlen, dstate, ngroups, full):
    """The reference's upstream-parity inputs (tests/test_upstream.py:37-54):
    u, B, C, D, z ~ N(0,1); delta ~ U(0, 0.5); A ~ -U(0.5, 16.5);
    delta_bias ~ U(0, 0.1); D, z and delta_bias only when full."""
    g = torch.Generator().manual_seed(0)
    bc = (batch, dstate, seqlen) if ngroups is None else (batch, ngroups, dstate, seqlen)
    inp = {"u": torch.randn(batch, dim, seqlen, generator=g),
           "delta": torch.rand(batch, dim, seqlen, generator=g) * 0.5,
           "A": -16 * torch.rand(dim, dstate, generator=g) - 0.5,
           "B": torch.randn(*bc, generator=g), "C": torch.randn(*bc, generator=g)}
    if full:
        inp["D"] = torch.randn(dim, generator=g)
        inp["z"] = torch.randn(batch, dim, seqlen, generator=g)
        inp["delta_bias"] = torch.rand(dim, generator=g) * 0.1
    return inp


@pytest.mark.parametrize("batch,dim,seqlen,dstate", [(1, 16, 1, 4), (2, 64, 257, 16), (1, 32, 2100, 16)])
@pytest.mark.parametrize("ngroups", [None, 1, 2])
@pytest.mark.parametrize("full,softplus", [(True, True), (False, False)])
def test_upstream_parity_shapes(batch, dim, seqlen, dstate, ngroups, full, softplus):
    """The shapes the reference checks against upstream mamba_ssm, here
    against the float64 oracle: outputs, last state and every gradient of
    sum(out * w), unscaled."""
    inp = upstream_case(batch, dim, seqlen, dstate, ngroups, full)
    wgt = torch.randn(batch, dim, seqlen, generator=torch.Generator().manual_seed(1))
    out, last, got = gpu_fwd_bwd(inp, wgt, softplus)
    wout, wlast = O.selective_scan_fwd(**inp, delta_softplus=softplus)
    assert_close_report(out, wout, 1e-4, 1e-5, "out")
    assert_close_report(last, wlast, 1e-4, 1e-5, "last_state")
    wgrads = O.selective_scan_bwd(**inp, delta_softplus=softplus, dout=wgt)
    for k, w in zip(NAMES, wgrads):
        if k in inp:
            assert_close_report(got[k], w, GRAD_RTOL, GRAD_ATOL[k], f"d{k}")

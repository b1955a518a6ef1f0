"""mcpu_selective_scan_bwd_noalloc: the backward without allocation or a
caller workspace, its scratch in the library's fixed per-device array.

Through the C ABI, its results equal mcpu_selective_scan_bwd's (the same
kernels and the same fixed summation order: bitwise) on calls in a row that
reuse the array: the training-step shape (batch 8, dim 1536, seqlen 1024,
dstate 16, with the forward's checkpoints and saved y), then a smaller,
time-chunked one (batch 1, dim 48, seqlen 4000, no checkpoints, so the
array also holds them), then the first again over the second's leftovers.
Shapes whose scratch exceeds the array are refused before any device work.

The array lives in a code object of its own, loaded when the first call on
a device looks up its address: this file's first test measures the device's
free memory around the first and second calls (64 MiB and more taken by the
first, nothing by the second), so it runs before any other noalloc call in
the process.
"""

import ctypes

import pytest
import torch

from conftest import GRAD_ATOL, GRAD_RTOL, assert_close_report
from oracle import numerics as O

NAMES = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")


def case(batch, dim, seqlen, seed):
    g = torch.Generator().manual_seed(seed)
    dev = "cuda"
    u = torch.randn(batch, dim, seqlen, generator=g).to(dev)
    delta = (torch.rand(batch, dim, seqlen, generator=g) * 0.5).to(dev)
    A = (-torch.rand(dim, 16, generator=g) - 0.5).to(dev)
    B = torch.randn(batch, 16, seqlen, generator=g).to(dev)
    C = torch.randn(batch, 16, seqlen, generator=g).to(dev)
    D = torch.randn(dim, generator=g).to(dev)
    z = torch.randn(batch, dim, seqlen, generator=g).to(dev)
    bias = (torch.rand(dim, generator=g) * 0.1).to(dev)
    dout = torch.randn(batch, dim, seqlen, generator=g).to(dev)
    dlast = torch.randn(batch, dim, 16, generator=g).to(dev)
    args = (u, delta, A, B[:, None].transpose(-1, -2), C[:, None].transpose(-1, -2), D, z, bias, True)
    return args, (B, C), dout, dlast


SCRATCH_BYTES = 64 << 20  # MCPU_NOALLOC_SCRATCH_BYTES in include/mamba_hip.h


@pytest.mark.gpu
def test_first_call_reserves_the_array():
    from mamba_cpu import _C
    from scan_abi import bwd as abi_bwd

    noalloc = _C.lib.mcpu_selective_scan_bwd_noalloc
    taken = []

    def entry(a, stream):
        torch.cuda.synchronize()
        before = torch.cuda.mem_get_info()[0]
        rc = noalloc(a, stream)
        torch.cuda.synchronize()
        taken.append(before - torch.cuda.mem_get_info()[0])
        return rc

    entry.__name__ = "mcpu_selective_scan_bwd_noalloc"
    args, _, dout, dlast = case(1, 64, 100, 3)
    for _ in range(2):
        abi_bwd(*args, dout, dlast, None, None, entry=entry)
    print(f"free device memory taken: first call {taken[0] / 2**20:.1f} MiB, second {taken[1] / 2**20:.1f} MiB")
    assert taken[0] >= SCRATCH_BYTES
    assert taken[1] == 0


@pytest.mark.gpu
def test_noalloc_backward_equals_the_workspace_backward():
    from mamba_cpu import _C
    from scan_abi import bwd as abi_bwd

    noalloc = _C.lib.mcpu_selective_scan_bwd_noalloc
    cases = [("training step (8, 1536, 1024), checkpoints given", (8, 1536, 1024, 0), True),
             ("smaller, time-chunked (1, 48, 4000), no checkpoints", (1, 48, 4000, 1), False),
             ("training step again", (8, 1536, 1024, 0), True)]
    for label, (b, d, l, seed), with_ckpt in cases:
        print(f"noalloc backward: {label}", flush=True)
        args, (B, C), dout, dlast = case(b, d, l, seed)
        ckpt = ysave = None
        if with_ckpt:
            _, _, ckpt, ysave = torch.ops.mamba_cpu.selective_scan_fwd_ckpt(*args)
        want = abi_bwd(*args, dout, dlast, ckpt, ysave)
        # the array still holds the previous case's partials: a partial the
        # kernels failed to rewrite would show as a difference here
        got = abi_bwd(*args, dout, dlast, ckpt, ysave, entry=noalloc)
        torch.cuda.synchronize()
        for name, g, w in zip(NAMES, got, want):
            assert torch.equal(g, w), f"{label}: d{name} differs from mcpu_selective_scan_bwd"
        if b == 1:
            # and against the float64 oracle, as the workspace path is tested
            oracle = O.selective_scan_bwd(args[0], args[1], args[2], B, C, args[5], args[6], args[7], True,
                                          dout=dout, dlast_state=dlast)
            for name, g, w in zip(NAMES, got, oracle):
                w = w.swapaxes(-1, -2)[:, None] if name in ("B", "C") else w
                assert_close_report(g, w, GRAD_RTOL, GRAD_ATOL[name], f"d{name}")


def test_noalloc_backward_refuses_shapes_beyond_its_array():
    """Host-side check, no device work: a shape whose scratch exceeds the
    64 MiB array is refused with MCPU_ERR_UNSUPPORTED and a message that names
    the workspace entry point."""
    from mamba_cpu import _C

    a = _C.ScanArgs()
    a.u = a.delta = a.A = a.B = a.C = 16
    a.du = a.ddelta = a.dA = a.dB = a.dC = 16
    a.batch, a.dim, a.seqlen, a.dstate, a.ngroups = 8, 1536, 8192, 16, 1
    a.dtype = _C.MCPU_F32
    a.u_stride[:] = a.delta_stride[:] = (1536 * 8192, 8192, 1)
    a.B_stride[:] = a.C_stride[:] = (8192 * 16, 8192 * 16, 16, 1)
    need = _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a))
    assert need > 64 << 20
    rc = _C.lib.mcpu_selective_scan_bwd_noalloc(ctypes.byref(a), None)
    msg = _C.lib.mcpu_last_error().decode()
    assert rc == _C.MCPU_ERR_UNSUPPORTED and "mcpu_selective_scan_bwd" in msg, msg

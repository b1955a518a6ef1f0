"""Direct C-ABI calls of the selective scan for the tests (ctypes over
libmamba_hip.so, torch tensors only as device memory). The tests use them
where the torch operators do not reach: pinning the backward's workgroup
width, and entry points the operators do not call."""

import ctypes

import torch

from mamba_cpu import _C


def scan_args(u, delta, A, Bk, Ck, D=None, z=None, delta_bias=None, softplus=False):
    """An mcpu_scan_args block for (batch, dim, seqlen) u/delta/z and
    kernel-layout (batch, ngroups, seqlen, dstate) B/C views (any strides)."""
    a = _C.ScanArgs()
    a.u, a.delta, a.A, a.B, a.C = (u.data_ptr(), delta.data_ptr(), A.data_ptr(), Bk.data_ptr(),
                                   Ck.data_ptr())
    a.D, a.z, a.delta_bias = _C.ptr(D), _C.ptr(z), _C.ptr(delta_bias)
    a.batch, a.dim, a.seqlen = u.shape
    a.ngroups, a.dstate = Bk.shape[1], Bk.shape[3]
    a.delta_softplus = int(bool(softplus))
    a.dtype = _C.DTYPES[u.dtype]
    a.u_stride[:] = u.stride()
    a.delta_stride[:] = delta.stride()
    a.z_stride[:] = _C.strides3(z)
    a.B_stride[:] = Bk.stride()
    a.C_stride[:] = Ck.stride()
    return a


def bwd(u, delta, A, Bk, Ck, D, z, delta_bias, softplus, dout, dlast=None, ckpt=None, ysave=None,
        waves=0, entry=None):
    """mcpu_selective_scan_bwd (or `entry`, a function of (args, stream) that
    allocates nothing) with its workspace; returns (du, ddelta, dA, dB, dC,
    dD, dz, ddelta_bias), None for absent D / z / delta_bias."""
    a = scan_args(u, delta, A, Bk, Ck, D, z, delta_bias, softplus)
    a.bwd_waves = waves
    a.dout = dout.data_ptr()
    a.dout_stride[:] = dout.stride()
    a.dlast_state = _C.ptr(dlast)
    a.ckpt = _C.ptr(ckpt)
    a.ysave = _C.ptr(ysave) if ysave is not None and ysave.numel() else 0
    du, ddelta = torch.empty_like(u), torch.empty_like(delta)
    dz = torch.empty_like(z) if z is not None else None
    dA = torch.empty_like(A)
    dB = torch.empty(Bk.shape, device=u.device)
    dC = torch.empty(Ck.shape, device=u.device)
    dD = torch.empty_like(D) if D is not None else None
    dbias = torch.empty_like(delta_bias) if delta_bias is not None else None
    a.du, a.ddelta, a.dz = du.data_ptr(), ddelta.data_ptr(), _C.ptr(dz)
    a.dA, a.dB, a.dC, a.dD, a.ddelta_bias = (dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), _C.ptr(dD),
                                             _C.ptr(dbias))
    stream = _C.stream_of(u)
    if entry is None:
        n = _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=u.device)
        _C.check(_C.lib.mcpu_selective_scan_bwd(ctypes.byref(a), ws.data_ptr() if n else None, n, stream),
                 "mcpu_selective_scan_bwd")
    else:
        _C.check(entry(ctypes.byref(a), stream), entry.__name__)
    return du, ddelta, dA, dB, dC, dD, dz, dbias

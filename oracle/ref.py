"""ctypes access to oracle/_ref/libmcpu_ref.so — TEST INFRASTRUCTURE ONLY.

The library is the reference's own CPU selective-scan kernels
(csrc/selective_scan.cpp, compiled unchanged from the reference checkout by
oracle/Makefile) behind the plain-C shim oracle/ref_shim.cpp. It is used as a
parity checker and as the timed CPU baseline; the product never loads it.

Arrays are numpy float32. B/C use the reference's kernel layout
(batch, ngroups, seqlen, dstate) (csrc/selective_scan.h:14-20).
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_ref", "libmcpu_ref.so")
_lib = None


def available():
    return os.path.exists(LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        if not available():
            raise FileNotFoundError(f"{LIB_PATH} not built (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.mcpu_ref_selective_scan_fwd_f32.argtypes = [P] * 10 + [I64] * 5 + [I, I]
        L.mcpu_ref_selective_scan_fwd_f32.restype = None
        L.mcpu_ref_selective_scan_bwd_f32.argtypes = [P] * 18 + [I64] * 5 + [I, I]
        L.mcpu_ref_selective_scan_bwd_f32.restype = None
        L.mcpu_ref_cpu_isa.restype = ctypes.c_char_p
        L.mcpu_ref_set_cpu_isa.argtypes = [ctypes.c_char_p]
        L.mcpu_ref_set_cpu_isa.restype = I
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c32(a):
    if a is None:
        return None
    if hasattr(a, "detach"):
        a = a.detach().cpu().float().numpy()
    return np.ascontiguousarray(a, dtype=np.float32)


def cpu_isa():
    return lib().mcpu_ref_cpu_isa().decode()


def set_cpu_isa(name):
    return bool(lib().mcpu_ref_set_cpu_isa(name.encode()))


def kernel_bc(X):
    """(b, n, l) | (b, g, n, l) -> contiguous float32 (b, g, l, n)."""
    X = _c32(X)
    if X.ndim == 3:
        X = X[:, None]
    return np.ascontiguousarray(np.swapaxes(X, -1, -2))


def scan_fwd(u, delta, A, Bk, Ck, D=None, z=None, delta_bias=None, delta_softplus=False,
             num_threads=1):
    """Reference forward with kernel-layout Bk/Ck. Returns (out, last_state) float32."""
    u, delta, A, Bk, Ck = map(_c32, (u, delta, A, Bk, Ck))
    D, z, delta_bias = map(_c32, (D, z, delta_bias))
    b, d, l = u.shape
    g, n = Bk.shape[1], Bk.shape[3]
    out = np.empty_like(u)
    last = np.empty((b, d, n), np.float32)
    lib().mcpu_ref_selective_scan_fwd_f32(
        _p(u), _p(delta), _p(A), _p(Bk), _p(Ck), _p(D), _p(z), _p(delta_bias), _p(out), _p(last),
        b, d, l, n, g, int(bool(delta_softplus)), int(num_threads))
    return out, last


def scan_bwd(u, delta, A, Bk, Ck, D, z, delta_bias, delta_softplus, dout, dlast_state=None,
             num_threads=1):
    """Reference backward. Returns (du, ddelta, dA, dB, dC, dD, dz, ddelta_bias) float32
    with the per-batch partials summed (as selective_scan_interface.py:87 does);
    dz is None when z is None."""
    u, delta, A, Bk, Ck = map(_c32, (u, delta, A, Bk, Ck))
    D, z, delta_bias, dout, dlast_state = map(_c32, (D, z, delta_bias, dout, dlast_state))
    b, d, l = u.shape
    g, n = Bk.shape[1], Bk.shape[3]
    du, ddelta = np.empty_like(u), np.empty_like(u)
    dA_part = np.empty((b, d, n), np.float32)
    dB, dC = np.zeros_like(Bk), np.zeros_like(Ck)
    dD_part = np.empty((b, d), np.float32)
    dz = np.empty_like(u) if z is not None else None
    dbias_part = np.empty((b, d), np.float32)
    lib().mcpu_ref_selective_scan_bwd_f32(
        _p(u), _p(delta), _p(A), _p(Bk), _p(Ck), _p(D), _p(z), _p(delta_bias), _p(dout),
        _p(dlast_state), _p(du), _p(ddelta), _p(dA_part), _p(dB), _p(dC), _p(dD_part), _p(dz),
        _p(dbias_part), b, d, l, n, g, int(bool(delta_softplus)), int(num_threads))
    return du, ddelta, dA_part.sum(0), dB, dC, dD_part.sum(0), dz, dbias_part.sum(0)

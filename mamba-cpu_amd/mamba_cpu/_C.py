"""Binding of libmamba_hip.so, the gfx950 kernel library, through its C ABI.

This module plays the role of the reference's nanobind module `mamba_cpu._C`
(csrc/bindings.cpp:17-84). It loads the two native libraries:
  libmamba_hip.so    the kernels behind the C ABI of include/mamba_hip.h
                     (raw device pointers and element strides, no torch types),
                     also bound here through ctypes: the argument blocks mirror
                     the header field for field and their sizes are checked
                     against the library at load time;
  libmamba_torch.so  the torch operators mamba_cpu::* (csrc/torch_ops.cpp), C++
                     over that C ABI, which the ops modules call.

There is no fallback: if the library is missing or was built for another
architecture, importing mamba_cpu fails or the first op raises.
"""

import ctypes
import os

import torch  # loads torch's HIP runtime first, so the library binds to the same one

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmamba_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"mamba_cpu: {LIB_PATH} is not built. Build it with `make -C mamba-cpu_amd` "
        "(hipcc, gfx950). There is no CPU fallback."
    )

lib = ctypes.CDLL(LIB_PATH)

# The torch operators (mamba_cpu::*), C++ over the same C ABI.
OPS_PATH = os.path.join(_HERE, "libmamba_torch.so")
if not os.path.exists(OPS_PATH):
    raise ImportError(f"mamba_cpu: {OPS_PATH} is not built. Build it with `make -C mamba-cpu_amd`.")
torch.ops.load_library(OPS_PATH)

MCPU_OK, MCPU_ERR_INVALID, MCPU_ERR_UNSUPPORTED, MCPU_ERR_DEVICE, MCPU_ERR_HIP = range(5)
MCPU_F32, MCPU_BF16, MCPU_F16 = range(3)

DTYPES = {torch.float32: MCPU_F32, torch.bfloat16: MCPU_BF16, torch.float16: MCPU_F16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_S3 = ctypes.c_int64 * 3
_S4 = ctypes.c_int64 * 4
_S2 = ctypes.c_int64 * 2


class ScanArgs(ctypes.Structure):
    _fields_ = [
        ("u", _P), ("delta", _P), ("A", _P), ("B", _P), ("C", _P), ("D", _P), ("z", _P),
        ("delta_bias", _P),
        ("batch", _I64), ("dim", _I64), ("seqlen", _I64), ("dstate", _I64), ("ngroups", _I64),
        ("delta_softplus", _I32), ("dtype", _I32),
        ("u_stride", _S3), ("delta_stride", _S3), ("z_stride", _S3), ("B_stride", _S4),
        ("C_stride", _S4),
        ("out", _P), ("last_state", _P), ("ckpt", _P), ("ysave", _P),
        ("dout", _P), ("dout_stride", _S3), ("dlast_state", _P),
        ("du", _P), ("ddelta", _P), ("dz", _P), ("dA", _P), ("dB", _P), ("dC", _P), ("dD", _P),
        ("ddelta_bias", _P),
        ("out_stride", _S3), ("du_stride", _S3), ("ddelta_stride", _S3), ("dz_stride", _S3),
        ("complex_a", _I32), ("bwd_waves", _I32),
    ]


class ConvArgs(ctypes.Structure):
    _fields_ = [
        ("x", _P), ("weight", _P), ("bias", _P), ("initial_states", _P),
        ("batch", _I64), ("dim", _I64), ("seqlen", _I64), ("width", _I64),
        ("silu", _I32), ("dtype", _I32),
        ("x_stride", _S3), ("init_stride", _S3),
        ("out", _P), ("out_stride", _S3), ("final_states", _P),
        ("dout", _P), ("dout_stride", _S3), ("dfinal_states", _P),
        ("dx", _P), ("dx_stride", _S3), ("dweight", _P), ("dbias", _P), ("dinitial_states", _P),
        ("seq_idx", _P),
    ]


class ConvUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("x", _P), ("conv_state", _P), ("weight", _P), ("bias", _P), ("out", _P),
        ("batch", _I64), ("dim", _I64), ("seqlen", _I64), ("width", _I64), ("state_len", _I64),
        ("silu", _I32), ("dtype", _I32),
        ("x_stride", _S3), ("state_stride", _S3), ("out_stride", _S3),
        ("cache_seqlens", _P), ("conv_state_indices", _P), ("state_batch", _I64),
    ]


class StateUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("state", _P), ("x", _P), ("dt", _P), ("A", _P), ("B", _P), ("C", _P), ("D", _P),
        ("z", _P), ("dt_bias", _P), ("out", _P),
        ("batch", _I64), ("nheads", _I64), ("headdim", _I64), ("dstate", _I64), ("ngroups", _I64),
        ("dt_softplus", _I32), ("dtype", _I32), ("state_dtype", _I32), ("_pad", _I32),
        ("state_stride", _S3), ("x_stride", _S3), ("dt_stride", _S3), ("z_stride", _S3),
        ("B_stride", _S2), ("C_stride", _S2),
        ("state_batch_indices", _P), ("state_batch", _I64),
        ("param_strides", _I32), ("_pad2", _I32), ("A_stride", _S3), ("D_stride", _S2),
        ("dt_bias_stride", _S2),
    ]


class SsdArgs(ctypes.Structure):
    _fields_ = [
        ("x", _P), ("dt", _P), ("A", _P), ("B", _P), ("C", _P), ("D", _P), ("z", _P), ("dt_bias", _P),
        ("initial_states", _P),
        ("batch", _I64), ("seqlen", _I64), ("nheads", _I64), ("headdim", _I64), ("ngroups", _I64),
        ("dstate", _I64),
        ("dtype", _I32), ("dt_softplus", _I32), ("dt_limit_lo", ctypes.c_float),
        ("dt_limit_hi", ctypes.c_float),
        ("out", _P), ("final_states", _P), ("ysave", _P),
        ("dout", _P), ("dfinal_states", _P),
        ("dx", _P), ("ddt", _P), ("dA", _P), ("dB", _P), ("dC", _P), ("dD", _P), ("dz", _P),
        ("ddt_bias", _P), ("dinitial_states", _P), ("head_block", _I32), ("chunk_pass", _I32), ("seq_idx", _P),
    ]


class MixerStepArgs(ctypes.Structure):
    _fields_ = [
        ("hidden", _P), ("norm_weight", _P), ("in_w", _P), ("in_b", _P), ("conv_w", _P), ("conv_b", _P),
        ("conv_state", _P), ("x_w", _P), ("dt_w", _P), ("dt_b", _P), ("A", _P), ("D", _P),
        ("ssm_state", _P), ("out_w", _P), ("out_b", _P), ("out", _P),
        ("batch", _I64), ("d_model", _I64), ("d_inner", _I64), ("dt_rank", _I64), ("dstate", _I64),
        ("width", _I64), ("state_len", _I64),
        ("norm_eps", ctypes.c_float), ("add_residual", _I32), ("residual_in_fp32", _I32), ("dtype", _I32),
        ("hidden_dtype", _I32), ("state_dtype", _I32), ("out_dtype", _I32), ("_pad", _I32),
    ]


class NormLinearArgs(ctypes.Structure):
    _fields_ = [
        ("hidden", _P), ("norm_weight", _P), ("weight", _P), ("bias", _P), ("out", _P),
        ("batch", _I64), ("d_in", _I64), ("d_out", _I64),
        ("norm_eps", ctypes.c_float), ("dtype", _I32), ("hidden_dtype", _I32), ("out_dtype", _I32),
    ]


class Mamba2StepArgs(ctypes.Structure):
    _fields_ = [
        ("hidden", _P), ("norm_weight", _P), ("in_w", _P), ("in_b", _P), ("conv_w", _P), ("conv_b", _P),
        ("conv_state", _P), ("dt_bias", _P), ("A", _P), ("D", _P), ("ssm_state", _P), ("gate_norm_weight", _P),
        ("out_w", _P), ("out_b", _P), ("out", _P),
        ("batch", _I64), ("d_model", _I64), ("d_inner", _I64), ("nheads", _I64), ("headdim", _I64),
        ("ngroups", _I64), ("dstate", _I64), ("width", _I64), ("state_len", _I64),
        ("norm_eps", ctypes.c_float), ("gate_norm_eps", ctypes.c_float), ("add_residual", _I32),
        ("residual_in_fp32", _I32), ("dtype", _I32), ("hidden_dtype", _I32), ("state_dtype", _I32),
        ("out_dtype", _I32),
    ]


_BLOCKS = (("scan", ScanArgs), ("conv", ConvArgs), ("conv_update", ConvUpdateArgs),
           ("state_update", StateUpdateArgs), ("ssd", SsdArgs), ("mixer_step", MixerStepArgs),
           ("norm_linear", NormLinearArgs), ("mamba2_step", Mamba2StepArgs))
_ARGP = {n: ctypes.POINTER(c) for n, c in _BLOCKS}

lib.mcpu_last_error.restype = ctypes.c_char_p
lib.mcpu_version.restype = ctypes.c_char_p
lib.mcpu_check_device.restype = ctypes.c_int
lib.mcpu_args_size.argtypes = [ctypes.c_char_p]
lib.mcpu_args_size.restype = ctypes.c_size_t
lib.mcpu_selective_scan_ckpt_size.argtypes = [_ARGP["scan"]]
lib.mcpu_selective_scan_ckpt_size.restype = ctypes.c_size_t
lib.mcpu_selective_scan_fwd_workspace_size.argtypes = [_ARGP["scan"]]
lib.mcpu_selective_scan_fwd_workspace_size.restype = ctypes.c_size_t
lib.mcpu_selective_scan_fwd.argtypes = [_ARGP["scan"], _P, ctypes.c_size_t, _P]
lib.mcpu_selective_scan_fwd.restype = ctypes.c_int
lib.mcpu_selective_scan_bwd_workspace_size.argtypes = [_ARGP["scan"]]
lib.mcpu_selective_scan_bwd_workspace_size.restype = ctypes.c_size_t
lib.mcpu_selective_scan_bwd.argtypes = [_ARGP["scan"], _P, ctypes.c_size_t, _P]
lib.mcpu_selective_scan_bwd.restype = ctypes.c_int
lib.mcpu_selective_scan_bwd_noalloc.argtypes = [_ARGP["scan"], _P]
lib.mcpu_selective_scan_bwd_noalloc.restype = ctypes.c_int
lib.mcpu_causal_conv1d_fwd.argtypes = [_ARGP["conv"], _P]
lib.mcpu_causal_conv1d_fwd.restype = ctypes.c_int
lib.mcpu_causal_conv1d_bwd_workspace_size.argtypes = [_ARGP["conv"]]
lib.mcpu_causal_conv1d_bwd_workspace_size.restype = ctypes.c_size_t
lib.mcpu_causal_conv1d_bwd.argtypes = [_ARGP["conv"], _P, ctypes.c_size_t, _P]
lib.mcpu_causal_conv1d_bwd.restype = ctypes.c_int
lib.mcpu_causal_conv1d_update.argtypes = [_ARGP["conv_update"], _P]
lib.mcpu_causal_conv1d_update.restype = ctypes.c_int
lib.mcpu_selective_state_update.argtypes = [_ARGP["state_update"], _P]
lib.mcpu_selective_state_update.restype = ctypes.c_int
lib.mcpu_ssd_saved_size.argtypes = [_ARGP["ssd"]]
lib.mcpu_ssd_saved_size.restype = ctypes.c_size_t
lib.mcpu_ssd_fwd.argtypes = [_ARGP["ssd"], _P, ctypes.c_size_t, _P]
lib.mcpu_ssd_fwd.restype = ctypes.c_int
lib.mcpu_ssd_bwd_workspace_size.argtypes = [_ARGP["ssd"]]
lib.mcpu_ssd_bwd_workspace_size.restype = ctypes.c_size_t
lib.mcpu_ssd_bwd.argtypes = [_ARGP["ssd"], _P, ctypes.c_size_t, _P, ctypes.c_size_t, _P]
lib.mcpu_ssd_bwd.restype = ctypes.c_int
lib.mcpu_ssd_varlen_states.argtypes = [_ARGP["ssd"], _P, ctypes.c_size_t, _P, ctypes.c_int64, _P, _P]
lib.mcpu_ssd_varlen_states.restype = ctypes.c_int
lib.mcpu_mixer_step_workspace_size.argtypes = [_ARGP["mixer_step"]]
lib.mcpu_mixer_step_workspace_size.restype = ctypes.c_size_t
lib.mcpu_mixer_step.argtypes = [_ARGP["mixer_step"], _P, ctypes.c_size_t, _P]
lib.mcpu_mixer_step.restype = ctypes.c_int
lib.mcpu_norm_linear.argtypes = [_ARGP["norm_linear"], _P]
lib.mcpu_norm_linear.restype = ctypes.c_int
lib.mcpu_mamba2_step_workspace_size.argtypes = [_ARGP["mamba2_step"]]
lib.mcpu_mamba2_step_workspace_size.restype = ctypes.c_size_t
lib.mcpu_mamba2_step.argtypes = [_ARGP["mamba2_step"], _P, ctypes.c_size_t, _P]
lib.mcpu_mamba2_step.restype = ctypes.c_int

for _name, _cls in _BLOCKS:
    _want = lib.mcpu_args_size(_name.encode())
    if _want != ctypes.sizeof(_cls):
        raise ImportError(f"mamba_cpu: {_name} argument block is {ctypes.sizeof(_cls)} bytes here "
                          f"but {_want} in {LIB_PATH}; rebuild the library")


def version():
    return lib.mcpu_version().decode()


def ptr(t):
    """Device pointer of a tensor, 0 (NULL) for None."""
    return 0 if t is None else t.data_ptr()


def strides3(t):
    return (0, 0, 0) if t is None else tuple(t.stride())


def stream_of(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def check(rc, what):
    """Map a C-ABI status to the exception types the reference raises."""
    if rc == MCPU_OK:
        return
    msg = f"{what}: {lib.mcpu_last_error().decode()}"
    if rc == MCPU_ERR_INVALID:
        raise ValueError(msg)
    if rc == MCPU_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


class device_of:
    """Makes t's device current for the duration of a library call."""

    def __init__(self, t):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        if self.idx is not None:
            cur = torch.cuda.current_device()
            if cur != self.idx:
                self.prev = cur
                torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def call(fn, args, what, *extra):
    check(fn(ctypes.byref(args), *extra), what)

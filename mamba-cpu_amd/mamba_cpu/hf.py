"""Hugging Face transformers' Mamba-family models on this package's GPU ops.

    import mamba_cpu.hf
    mamba_cpu.hf.patch_transformers()
    model = transformers.MambaForCausalLM(config).to("cuda")

How transformers (>= 5) reaches its kernels: each Mamba-family modeling
module defines five kernel functions as module globals (mamba_selective_scan,
mamba_selective_state_update, causal_conv1d_fn, causal_conv1d_update,
mamba_inner_fn) and its mixers look them up by name on every call. The
reference hooks the same five globals (src/mamba_cpu/hf.py:63-112), which is
why the hook points, the three public names and the parameter lists below are
what they are.

Mamba-2 models (modeling_mamba2) look up their own set the same way:
mamba2_chunk_scan (mamba_ssm's mamba_chunk_scan_combined),
mamba2_selective_state_update, causal_conv1d_fn and causal_conv1d_update,
routed here to mamba_chunk_scan_combined and the ops above. Their fifth,
mamba2_split_conv1d_scan_combined (the fused layer), is left alone: without
mamba_ssm it answers None and the mixer takes its unfused path through the
four routed functions. Following mamba_ssm, a seq_idx that reaches these
functions packs sequences (transformers' own torch functions ignore it).

patch_transformers() puts a DeviceRoute in each global: a call whose leading
tensor is on a ROCm GPU (torch's "cuda" device type) runs this package's op,
any other call the function the route replaced, so CPU models keep
transformers' own path. mamba_inner_fn, which the reference answers with
None so that mixers take their unfused path, is the fused mixer of
mamba_cpu.ops.mamba_inner for float32 Mamba models in training, and None
where that mixer does not apply.
"""

import importlib

import torch

from mamba_cpu.ops import (
    causal_conv1d_fn,
    causal_conv1d_update,
    mamba_chunk_scan_combined,
    selective_scan_fn,
    selective_state_update,
)
from mamba_cpu.ops.mamba_inner import fused_path_supported, mamba_inner_fn

MAMBA1_FAMILIES = ("mamba", "falcon_mamba", "jamba")
MAMBA2_FAMILIES = ("mamba2",)
SUPPORTED_MODELS = MAMBA1_FAMILIES + MAMBA2_FAMILIES


# GPU bodies of transformers' kernel globals. Each takes the parameter list of
# the function it stands in for (transformers' modeling_mamba.py defines
# them); keywords that only choose among transformers' own torch fallbacks
# (use_mambapy, use_associative_scan, ...) arrive in **options and are moot
# here.


def gpu_selective_scan(hidden_states, dt, A, B, C, D=None, z=None, delta_bias=None,
                       delta_softplus=False, return_last_state=False, **options):
    return selective_scan_fn(hidden_states, dt, A, B, C, D=D, z=z, delta_bias=delta_bias,
                             delta_softplus=delta_softplus, return_last_state=return_last_state)


def gpu_selective_state_update(state, hidden_states, dt, A, B, C, D=None, dt_bias=None,
                               dt_softplus=False, z=None, **options):
    # transformers orders (D, dt_bias, dt_softplus, z); the op's own order is (D, z, dt_bias, dt_softplus)
    return selective_state_update(state, hidden_states, dt, A, B, C, D=D, z=z, dt_bias=dt_bias,
                                  dt_softplus=dt_softplus)


def gpu_causal_conv1d(hidden_states, weight, bias=None, activation=None, seq_idx=None, **options):
    return causal_conv1d_fn(hidden_states, weight, bias, seq_idx=seq_idx, activation=activation)


def gpu_causal_conv1d_update(hidden_states, conv_state, weight, bias=None, activation=None, **options):
    return causal_conv1d_update(hidden_states, conv_state, weight, bias, activation=activation)


def gpu_mamba_inner(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                    out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                    delta_softplus=True, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                    b_c_dt_rms_eps=1e-6, **options):
    """The fused mixer where it applies; None otherwise, which sends the mixer
    down its unfused path (through the four ops above).

    FalconMamba passes RMS-norm weights: its unfused path normalises dt
    before dt_proj, where the fused mixer's norms (mamba_ssm's) normalise
    delta after it. Such calls answer None, so that model computes what the
    reference computes."""
    if b_rms_weight is not None or c_rms_weight is not None or dt_rms_weight is not None:
        return None
    if not fused_path_supported(xz, conv1d_weight, x_proj_weight, delta_proj_weight, out_proj_weight,
                                A, B, C):
        return None
    return mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                          out_proj_weight, out_proj_bias, A, D=D, delta_bias=delta_bias,
                          delta_softplus=delta_softplus)


def gpu_chunk_scan(hidden_states, dt, A, B, C, chunk_size, D=None, dt_bias=None, initial_states=None,
                   dt_softplus=False, dt_limit=(0.0, float("inf")), return_final_states=False, z=None,
                   seq_idx=None, cu_seqlens=None, return_varlen_states=False, **options):
    """mamba2_chunk_scan: (batch, seqlen, nheads, headdim) x, (batch, seqlen,
    nheads) dt, (nheads,) A and D, (batch, seqlen, ngroups, dstate) B and C;
    out in x's dtype (transformers' torch function returns float32)."""
    return mamba_chunk_scan_combined(hidden_states, dt, A, B, C, chunk_size, D=D, z=z, dt_bias=dt_bias,
                                     initial_states=initial_states, seq_idx=seq_idx, cu_seqlens=cu_seqlens,
                                     dt_softplus=dt_softplus, dt_limit=dt_limit,
                                     return_final_states=return_final_states,
                                     return_varlen_states=return_varlen_states)


# transformers global -> the GPU body that routes take for it: Mamba-1
# families, then Mamba-2 families
KERNEL_GLOBALS = {
    "mamba_selective_scan": gpu_selective_scan,
    "mamba_selective_state_update": gpu_selective_state_update,
    "causal_conv1d_fn": gpu_causal_conv1d,
    "causal_conv1d_update": gpu_causal_conv1d_update,
    "mamba_inner_fn": gpu_mamba_inner,
}
MAMBA2_KERNEL_GLOBALS = {
    "mamba2_chunk_scan": gpu_chunk_scan,
    "mamba2_selective_state_update": gpu_selective_state_update,
    "causal_conv1d_fn": gpu_causal_conv1d,
    "causal_conv1d_update": gpu_causal_conv1d_update,
}


def kernel_globals(family):
    """The globals table of a model family."""
    return MAMBA2_KERNEL_GLOBALS if family in MAMBA2_FAMILIES else KERNEL_GLOBALS


class DeviceRoute:
    """Stands in for one of transformers' kernel globals. A call whose first
    positional argument is a tensor on a ROCm GPU goes to `gpu`; every other
    call goes to `fallback`, the function this route replaced (reachable as
    __wrapped__ too)."""

    def __init__(self, fallback, gpu):
        self.fallback = fallback
        self.gpu = gpu
        self.__wrapped__ = fallback
        self.__name__ = getattr(fallback, "__name__", gpu.__name__)
        self.__doc__ = getattr(fallback, "__doc__", None)

    def __call__(self, *args, **kwargs):
        lead = args[0] if args else None
        on_gpu = isinstance(lead, torch.Tensor) and lead.device.type == "cuda"
        return (self.gpu if on_gpu else self.fallback)(*args, **kwargs)

    def __repr__(self):
        return f"DeviceRoute({self.__name__}: ROCm GPU -> mamba_cpu, else -> transformers)"


def _modeling(family):
    return importlib.import_module(f".modeling_{family}", f"transformers.models.{family}")


def patch_transformers(models=SUPPORTED_MODELS):
    """Route ROCm-GPU calls of the given model families' kernels to this
    package. Calling it again changes nothing. Raises RuntimeError, and
    patches nothing, if a family's modeling module lacks one of the globals
    of its table (transformers older than 5)."""
    modules = [(_modeling(family), kernel_globals(family)) for family in models]
    gaps = []
    for module, table in modules:
        absent = [name for name in table if not hasattr(module, name)]
        if absent:
            gaps.append(f"{module.__name__} ({', '.join(absent)})")
    if gaps:
        raise RuntimeError("mamba_cpu.hf works with transformers >= 5, whose Mamba modeling modules "
                           "define the kernel globals it routes; missing in " + "; ".join(gaps))
    for module, table in modules:
        for name, body in table.items():
            current = getattr(module, name)
            if not isinstance(current, DeviceRoute):
                setattr(module, name, DeviceRoute(current, body))


def unpatch_transformers(models=SUPPORTED_MODELS):
    """Put back the functions patch_transformers() replaced."""
    for family in models:
        module = _modeling(family)
        for name in kernel_globals(family):
            current = getattr(module, name, None)
            if isinstance(current, DeviceRoute):
                setattr(module, name, current.fallback)

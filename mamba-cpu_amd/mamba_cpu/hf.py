"""Run Hugging Face transformers Mamba models on mamba_cpu's MI355X ops.

    import mamba_cpu.hf
    mamba_cpu.hf.patch_transformers()
    model = transformers.MambaForCausalLM(config).to("cuda")

Same mechanism and surface as the reference's src/mamba_cpu/hf.py:26-112:
transformers (>= 5) resolves `mamba_selective_scan`,
`mamba_selective_state_update`, `causal_conv1d_fn`, `causal_conv1d_update` and
`mamba_inner_fn` from module globals at call time, and patch_transformers()
wraps those globals. The wrappers route calls whose first tensor is on a ROCm
GPU ("cuda" device type) to this package's gfx950 custom ops; tensors on other
devices keep transformers' own path. `mamba_inner_fn`, which the reference
answers with None (so its mixers always take their unfused path), is the
fused mixer of mamba_cpu.ops.mamba_inner for float32 models on the GPU, and
None otherwise.
"""

import functools
import importlib

from mamba_cpu.ops import (
    causal_conv1d_fn,
    causal_conv1d_update,
    selective_scan_fn,
    selective_state_update,
)
from mamba_cpu.ops.mamba_inner import fused_path_supported, mamba_inner_fn

SUPPORTED_MODELS = ("mamba", "falcon_mamba", "jamba")
_DEVICE_TYPE = "cuda"  # ROCm GPUs report the "cuda" device type in PyTorch


def _scan(
    hidden_states,
    dt,
    A,
    B,
    C,
    D=None,
    z=None,
    delta_bias=None,
    delta_softplus=False,
    return_last_state=False,
    **kwargs,  # use_mambapy, use_associative_scan select transformers' own fallbacks
):
    return selective_scan_fn(
        hidden_states, dt, A, B, C, D, z, delta_bias, delta_softplus, return_last_state
    )


def _state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False, **kwargs):
    return selective_state_update(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus)


def _conv(x, weight, bias=None, activation=None, **kwargs):
    return causal_conv1d_fn(x, weight, bias, activation=activation)


def _conv_update(x, conv_state, weight, bias=None, activation=None, **kwargs):
    return causal_conv1d_update(x, conv_state, weight, bias, activation)


def _inner(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
           out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, delta_softplus=True,
           b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None, b_c_dt_rms_eps=1e-6, **kwargs):
    # The fused mixer (mamba_cpu.ops.mamba_inner) where it applies; None
    # otherwise, and the mixer takes its unfused path, which calls the four
    # ops above (the reference always answers None, hf.py:59-60).
    # FalconMamba passes norm weights: its unfused path normalises dt before
    # dt_proj and ignores the weights, where mamba_inner_fn's norms (as in
    # mamba_ssm) normalise delta after it, so that model keeps the unfused
    # path, which is the computation the reference runs.
    if any(w is not None for w in (b_rms_weight, c_rms_weight, dt_rms_weight)):
        return None
    if not fused_path_supported(xz, conv1d_weight, x_proj_weight, delta_proj_weight, out_proj_weight,
                                A, B, C):
        return None
    return mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                          out_proj_weight, out_proj_bias, A, D=D, delta_bias=delta_bias,
                          delta_softplus=delta_softplus, b_rms_weight=b_rms_weight,
                          c_rms_weight=c_rms_weight, dt_rms_weight=dt_rms_weight,
                          b_c_dt_rms_eps=b_c_dt_rms_eps)


_OPS = {
    "mamba_selective_scan": _scan,
    "mamba_selective_state_update": _state_update,
    "causal_conv1d_fn": _conv,
    "causal_conv1d_update": _conv_update,
    "mamba_inner_fn": _inner,
}


def _dispatch(original, native):
    @functools.wraps(original)
    def wrapper(first, *args, **kwargs):
        fn = native if first.device.type == _DEVICE_TYPE else original
        return fn(first, *args, **kwargs)

    wrapper._mamba_cpu_original = original
    return wrapper


def _modeling_module(name):
    return importlib.import_module(f"transformers.models.{name}.modeling_{name}")


def patch_transformers(models=SUPPORTED_MODELS):
    """Route ROCm-GPU execution of the given transformers model families
    through mamba_cpu. Safe to call repeatedly."""
    modules = [_modeling_module(name) for name in models]
    for module in modules:
        missing = [op for op in _OPS if not hasattr(module, op)]
        if missing:
            raise RuntimeError(
                f"{module.__name__} has no {', '.join(missing)}; mamba_cpu.hf needs transformers >= 5"
            )
    for module in modules:
        for op, native in _OPS.items():
            original = getattr(module, op)
            if not hasattr(original, "_mamba_cpu_original"):
                setattr(module, op, _dispatch(original, native))


def unpatch_transformers(models=SUPPORTED_MODELS):
    """Undo patch_transformers."""
    for name in models:
        module = _modeling_module(name)
        for op in _OPS:
            original = getattr(getattr(module, op), "_mamba_cpu_original", None)
            if original is not None:
                setattr(module, op, original)

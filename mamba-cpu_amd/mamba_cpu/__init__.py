"""Mamba-1 op set on AMD MI355X (gfx950), with the public API of mamba-cpu.

The four ops are torch.library custom ops over hand-written HIP kernels in
libmamba_hip.so; they take ROCm GPU tensors. `mamba_chunk_scan_combined` is
Mamba-2's SSD scan (mamba_ssm's function of that name) over the same library. `mamba_inner_fn` is the fused
Mamba-1 mixer over them (transformers' training path). `mamba_cpu.hf.patch_transformers()`
routes Hugging Face Mamba / FalconMamba / Jamba / Mamba-2 models on the GPU to them.
"""

from mamba_cpu.ops import (
    causal_conv1d_fn,
    causal_conv1d_update,
    mamba_chunk_scan_combined,
    mamba_inner_fn,
    selective_scan_fn,
    selective_state_update,
)
from mamba_cpu.reference import causal_conv1d_ref, selective_scan_ref

__version__ = "0.3.0"

__all__ = [
    "causal_conv1d_fn",
    "causal_conv1d_ref",
    "causal_conv1d_update",
    "mamba_chunk_scan_combined",
    "mamba_inner_fn",
    "selective_scan_fn",
    "selective_scan_ref",
    "selective_state_update",
]

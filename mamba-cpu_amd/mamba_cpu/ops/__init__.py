from mamba_cpu.ops.causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from mamba_cpu.ops.mamba_inner import mamba_inner_fn
from mamba_cpu.ops.selective_scan_interface import selective_scan_fn
from mamba_cpu.ops.selective_state_update import selective_state_update
from mamba_cpu.ops.ssd_combined import mamba_chunk_scan_combined

__all__ = [
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "mamba_chunk_scan_combined",
    "mamba_inner_fn",
    "selective_scan_fn",
    "selective_state_update",
]

"""mamba2_jax.ops -- the per-token ops around the SSD (HIP) and the naive SSD
formulation.

Same names as the reference's ops/__init__.py:5-15: the decode step
(selective_state_update), the depthwise causal conv before the SSD
(causal_conv1d, causal_conv1d_update) and the gated RMSNorm after it
(rms_norm_gated).
"""

from .causal_conv1d import causal_conv1d, causal_conv1d_update
from .rms_norm import rms_norm_gated
from .selective_state_update import selective_state_update
from .ssd_naive import mamba_chunk_scan_combined_naive

__all__ = ["selective_state_update", "mamba_chunk_scan_combined_naive", "causal_conv1d",
           "causal_conv1d_update", "rms_norm_gated"]

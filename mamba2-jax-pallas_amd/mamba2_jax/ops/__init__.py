"""mamba2_jax.ops -- the decode step (HIP) and the naive SSD formulation.

Same names as the reference's ops/__init__.py:5-15 for the hot path;
causal_conv1d and rms_norm_gated (the steps before and after the SSD) are not
part of this build.
"""

from .selective_state_update import selective_state_update
from .ssd_naive import mamba_chunk_scan_combined_naive

__all__ = ["selective_state_update", "mamba_chunk_scan_combined_naive"]

"""mamba2_jax.modules -- the SSD dispatch of modules/mamba2.py (the Flax block
around it is outside this build)."""

from .mamba2 import _ssd_combined_fwd

__all__ = ["_ssd_combined_fwd"]

"""mamba2_jax.modules -- the Mamba2 mixer layer (prefill and decode step) over
the HIP kernels, and the SSD dispatch of reference modules/mamba2.py."""

from .mamba2 import Mamba2, _ssd_combined_fwd, allocate_inference_cache

__all__ = ["Mamba2", "_ssd_combined_fwd", "allocate_inference_cache"]

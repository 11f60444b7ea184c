"""mamba2_jax.models -- the Mamba2 language model's forward and decode loop
over the HIP kernels (reference models/mamba2_lm.py)."""

from .mamba2_lm import Mamba2Config, Mamba2LMHeadModel, init_params, rms_norm

__all__ = ["Mamba2Config", "Mamba2LMHeadModel", "init_params", "rms_norm"]

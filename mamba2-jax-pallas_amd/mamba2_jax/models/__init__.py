"""mamba2_jax.models -- the Mamba2 language model's forward and decode loop
over the HIP kernels (reference models/mamba2_lm.py)."""

from .mamba2_lm import (MAMBA2_CONFIGS, Mamba2Config, Mamba2LMHeadModel, init_params,
                        load_from_pretrained, load_from_torch_checkpoint, read_state_dict, rms_norm)

__all__ = ["MAMBA2_CONFIGS", "Mamba2Config", "Mamba2LMHeadModel", "init_params",
           "load_from_pretrained", "load_from_torch_checkpoint", "read_state_dict", "rms_norm"]

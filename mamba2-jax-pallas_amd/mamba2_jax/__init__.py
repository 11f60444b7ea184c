"""mamba2_jax -- MI355X-native Mamba2 SSD forward and decode step.

The reference's (AlexG1105/mamba2-jax-pallas) Python API for this path --
mamba2_jax.kernels.*, mamba2_jax.ops.selective_state_update,
mamba2_jax.modules.mamba2._ssd_combined_fwd and the package-root exports
(mamba_chunk_scan_combined_fwd, Mamba2; reference src/mamba2_jax/__init__.py:5-11)
-- over hand-written HIP kernels
for gfx950 in libm2ssd.so (C ABI: include/m2ssd.h).  Arrays are torch tensors
on the GPU.
"""

from .kernels.ssd_combined import mamba_chunk_scan_combined_fwd
from .modules.mamba2 import Mamba2

__all__ = ["mamba_chunk_scan_combined_fwd", "Mamba2"]

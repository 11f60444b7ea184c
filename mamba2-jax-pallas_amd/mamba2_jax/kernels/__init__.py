"""mamba2_jax.kernels -- the SSD stage operators and the combined forward, as
hand-written HIP kernels for MI355X (gfx950) in libm2ssd.so.

Same names as the reference's kernels/__init__.py:6-32.
"""

from .chunk_cumsum_fwd import (
    chunk_cumsum_fwd,
    chunk_cumsum_fwd_mosaic,
    chunk_cumsum_fwd_pallas,
    chunk_cumsum_fwd_naive_jax,
)
from .chunk_state_fwd import chunk_state_fwd, chunk_state_fwd_mosaic, chunk_state_varlen_mosaic
from .state_passing_fwd import state_passing_fwd, state_passing_fwd_mosaic
from .bmm_chunk_fwd import bmm_chunk_fwd, bmm_chunk_fwd_mosaic
from .chunk_scan_fwd import chunk_scan_fwd, chunk_scan_fwd_mosaic
from .ssd_combined import mamba_chunk_scan_combined_fwd

__all__ = [
    "chunk_cumsum_fwd",
    "chunk_cumsum_fwd_mosaic",
    "chunk_cumsum_fwd_pallas",
    "chunk_cumsum_fwd_naive_jax",
    "chunk_state_fwd",
    "chunk_state_fwd_mosaic",
    "chunk_state_varlen_mosaic",
    "state_passing_fwd",
    "state_passing_fwd_mosaic",
    "bmm_chunk_fwd",
    "bmm_chunk_fwd_mosaic",
    "chunk_scan_fwd",
    "chunk_scan_fwd_mosaic",
    "mamba_chunk_scan_combined_fwd",
]

"""Dispatch for the SSD forward and the decode step.

Mirrors reference modules/mamba2.py:42-74 (``_ssd_combined_fwd``) and the
decode call at :510-521.  ``use_pallas=True`` (the default) runs the HIP
kernels; ``use_pallas=False`` runs the naive formulation on the GPU.  Unlike
the reference, a failure of the HIP path is raised, never swallowed into a
silent fallback: a fallback would hide parity and performance failures.
"""

from __future__ import annotations

from ..kernels.ssd_combined import mamba_chunk_scan_combined_fwd as _hip_fwd
from ..ops.selective_state_update import selective_state_update
from ..ops.ssd_naive import mamba_chunk_scan_combined_naive


def _ssd_combined_fwd(use_pallas: bool = True, **kwargs):
    """The SSD layer forward: the HIP kernels, or the naive path if use_pallas=False."""
    if use_pallas:
        return _hip_fwd(**kwargs)
    return mamba_chunk_scan_combined_naive(**kwargs)


__all__ = ["_ssd_combined_fwd", "selective_state_update"]

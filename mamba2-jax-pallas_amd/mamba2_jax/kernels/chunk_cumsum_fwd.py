"""chunk_cumsum_fwd on MI355X: dt processing + per-chunk dA cumsum.

Drop-in for reference kernels/chunk_cumsum_fwd.py (chunk_cumsum_fwd :288-302,
chunk_cumsum_fwd_mosaic :194-235, chunk_cumsum_fwd_pallas :99-187,
chunk_cumsum_fwd_naive_jax :242-281).  All four names run the same HIP
wavefront-scan kernel (libm2ssd.so: m2_chunk_cumsum); tile / warp keyword
arguments are accepted and ignored.
"""

from __future__ import annotations

import math

import torch

from .. import _lib as L


def chunk_cumsum_fwd(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                     dt_limit=(0.0, float("inf"))):
    """dt (batch, seqlen, nheads) -> (dA_cumsum, dt_out), each float32
    (batch, nheads, nchunks, chunk_size).

    dt' = clip(softplus?(dt + dt_bias), *dt_limit), 0 past the end of the
    sequence; dA_cumsum = per-chunk inclusive cumsum of dt' * A.
    """
    dev = L.device_of(dt, A, dt_bias)
    L.require(dt.dim() == 3, f"dt must be (batch, seqlen, nheads), got {tuple(dt.shape)}")
    batch, seqlen, nheads = dt.shape
    L.require(tuple(A.shape) == (nheads,), f"A.shape={tuple(A.shape)} != ({nheads},)")
    if dt_bias is not None:
        L.require(tuple(dt_bias.shape) == (nheads,),
                  f"dt_bias.shape={tuple(dt_bias.shape)} != ({nheads},)")
    chunk_size = int(chunk_size)
    L.require(chunk_size > 0, "chunk_size must be positive")
    nc = math.ceil(seqlen / chunk_size)
    dt_c = L.dev_contig(dt)
    code = L.dtype_code(dt_c, "chunk_cumsum_fwd: dt")
    A_c = L.dev_contig(A, torch.float32)
    bias_c = L.dev_contig(dt_bias, torch.float32)
    dA = torch.empty((batch, nheads, nc, chunk_size), dtype=torch.float32, device=dev)
    dto = torch.empty_like(dA)
    args = L.ChunkCumsumArgs(
        dt=L.ptr(dt_c), A=L.ptr(A_c), dt_bias=L.ptr(bias_c), dA_cumsum=L.ptr(dA),
        dt_out=L.ptr(dto), batch=batch, seqlen=seqlen, nheads=nheads, chunk_size=chunk_size,
        dt_dtype=code, dt_softplus=int(bool(dt_softplus)), dt_min=float(dt_limit[0]),
        dt_max=float(dt_limit[1]))
    with torch.cuda.device(dev):
        L.call("m2_chunk_cumsum", args, L.stream_of(dev))
    return dA, dto


def chunk_cumsum_fwd_mosaic(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                            dt_limit=(0.0, float("inf"))):
    """Same as chunk_cumsum_fwd (reference name kept)."""
    return chunk_cumsum_fwd(dt, A, chunk_size, dt_bias, dt_softplus, dt_limit)


def chunk_cumsum_fwd_pallas(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                            dt_limit=(0.0, float("inf")), block_size_h=8, num_warps=4):
    """Same as chunk_cumsum_fwd; block_size_h / num_warps are ignored."""
    return chunk_cumsum_fwd(dt, A, chunk_size, dt_bias, dt_softplus, dt_limit)


def chunk_cumsum_fwd_naive_jax(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                               dt_limit=(0.0, float("inf"))):
    """Same as chunk_cumsum_fwd (the kernel multiplies by A before the cumsum)."""
    return chunk_cumsum_fwd(dt, A, chunk_size, dt_bias, dt_softplus, dt_limit)

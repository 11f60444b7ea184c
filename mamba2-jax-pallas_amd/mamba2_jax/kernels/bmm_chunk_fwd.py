"""bmm_chunk_fwd on MI355X: per-chunk C @ B^T as an MFMA kernel whose fragments
are loaded straight from HBM (libm2ssd.so: m2_bmm_chunk).

Drop-in for reference kernels/bmm_chunk_fwd.py (bmm_chunk_fwd :381-400,
bmm_chunk_fwd_mosaic :293-374).  Tile keyword arguments are accepted and
ignored.
"""

from __future__ import annotations

import math

import torch

from .. import _lib as L
from . import _shapes as S
from .chunk_state_fwd import _io_dtype, _seq_idx


def bmm_chunk_fwd(a, b, chunk_size, seq_idx=None, causal=False, output_dtype=None,
                  BM=64, BK=64, BN=64, num_stages=2):
    """a, b (batch, seqlen, ngroups, k) -> (batch, nchunks, ngroups, Q, Q):
    out[.., c, g] = a_c @ b_c^T, optionally causal- and seq_idx-masked."""
    dev = L.device_of(a, b, seq_idx)
    L.require(a.dim() == 4 and tuple(b.shape) == tuple(a.shape),
              f"a and b must both be (batch, seqlen, ngroups, k): {tuple(a.shape)} vs {tuple(b.shape)}")
    batch, seqlen, ngroups, k = a.shape
    chunk_size = int(chunk_size)
    L.require(chunk_size > 0, "chunk_size must be positive")
    nc = math.ceil(seqlen / chunk_size)
    out_dtype = L.torch_dtype(output_dtype) or torch.float32
    L.require(out_dtype in (torch.float32, torch.bfloat16),
              f"output_dtype {out_dtype} is not supported (float32 or bfloat16)")
    io = _io_dtype(a, b)
    if k % 32:
        # zero columns of the contraction add nothing (the reference pads k to
        # its tile, kernels/bmm_chunk_fwd.py:209-218); the kernels take k % 32 == 0
        kp = 32 * math.ceil(k / 32)
        a, b = S.pad_last(a, kp), S.pad_last(b, kp)
        k = kp
    a_c, b_c = L.dev_contig(a, io), L.dev_contig(b, io)
    seq = _seq_idx(seq_idx, batch, seqlen)
    out = torch.empty((batch, nc, ngroups, chunk_size, chunk_size), dtype=out_dtype, device=dev)
    args = L.BmmChunkArgs(
        a=L.ptr(a_c), b=L.ptr(b_c), seq_idx=L.ptr(seq), out=L.ptr(out), batch=batch,
        seqlen=seqlen, ngroups=ngroups, k=k, chunk_size=chunk_size,
        dtype=L.dtype_code(a_c, "a"), out_dtype=L.dtype_code(out, "out"), causal=int(bool(causal)))
    with torch.cuda.device(dev):
        L.call("m2_bmm_chunk", args, L.stream_of(dev))
    return out


def bmm_chunk_fwd_mosaic(a, b, chunk_size, seq_idx=None, causal=False, output_dtype=None,
                         BM=64, BK=64, BN=64, num_stages=2):
    """Same as bmm_chunk_fwd (reference name kept)."""
    return bmm_chunk_fwd(a, b, chunk_size, seq_idx=seq_idx, causal=causal,
                         output_dtype=output_dtype)

"""state_passing_fwd on MI355X: the inter-chunk recurrence as an HBM-streaming
HIP kernel (libm2ssd.so: m2_state_passing).

Drop-in for reference kernels/state_passing_fwd.py (state_passing_fwd
:348-363, state_passing_fwd_mosaic :158-341).
"""

from __future__ import annotations

import torch

from .. import _lib as L


def state_passing_fwd(states, dA_chunk_cumsum, initial_states=None, seq_idx=None,
                      chunk_size=None, out_dtype=None):
    """states (batch, nchunks, nheads, dim), dA_chunk_cumsum (batch, nheads, nchunks)
    -> (out (batch, nchunks, nheads, dim) in out_dtype [default states.dtype],
        final_states (batch, nheads, dim) float32).

    out[:, c] is the state entering chunk c; with seq_idx the carried state is
    dropped where the sequence changes between chunk ends.
    """
    dev = L.device_of(states, dA_chunk_cumsum, initial_states, seq_idx)
    L.require(states.dim() == 4, "states must be (batch, nchunks, nheads, dim)")
    batch, nchunks, nheads, dim = states.shape
    L.require(tuple(dA_chunk_cumsum.shape) == (batch, nheads, nchunks),
              f"dA_chunk_cumsum.shape={tuple(dA_chunk_cumsum.shape)} != "
              f"({batch}, {nheads}, {nchunks})")
    if initial_states is not None:
        L.require(tuple(initial_states.shape) == (batch, nheads, dim),
                  f"initial_states.shape={tuple(initial_states.shape)} != ({batch}, {nheads}, {dim})")
    seqlen = 0
    if seq_idx is not None:
        L.require(chunk_size is not None, "chunk_size is required with seq_idx")
        L.require(seq_idx.dim() == 2 and seq_idx.shape[0] == batch, "seq_idx must be (batch, seqlen)")
        seqlen = int(seq_idx.shape[1])
        L.require((nchunks - 1) * int(chunk_size) < seqlen <= nchunks * int(chunk_size),
                  "seq_idx length does not match nchunks * chunk_size")
    out_dtype = L.torch_dtype(out_dtype) or states.dtype
    L.require(out_dtype in (torch.float32, torch.bfloat16),
              f"out_dtype {out_dtype} is not supported (float32 or bfloat16)")
    st = L.dev_contig(states, torch.float32)
    dAc = dA_chunk_cumsum if dA_chunk_cumsum.dtype == torch.float32 else dA_chunk_cumsum.float()
    init = L.dev_contig(initial_states, torch.float32)
    seq = None if seq_idx is None else L.dev_contig(seq_idx, torch.int32)
    out = torch.empty((batch, nchunks, nheads, dim), dtype=out_dtype, device=dev)
    fin = torch.empty((batch, nheads, dim), dtype=torch.float32, device=dev)
    sb, sh, sc = dAc.stride()
    args = L.StatePassingArgs(
        states=L.ptr(st), dA_chunk_cumsum=L.ptr(dAc), dA_stride_batch=sb, dA_stride_head=sh,
        dA_stride_chunk=sc, initial_states=L.ptr(init), seq_idx=L.ptr(seq), out=L.ptr(out),
        final_states=L.ptr(fin), batch=batch, nchunks=nchunks, nheads=nheads, dim=dim,
        seqlen=seqlen, chunk_size=int(chunk_size or 0), out_dtype=L.dtype_code(out, "out"))
    with torch.cuda.device(dev):
        L.call("m2_state_passing", args, L.stream_of(dev))
    return out, fin


def state_passing_fwd_mosaic(states, dA_chunk_cumsum, initial_states=None, seq_idx=None,
                             chunk_size=None, out_dtype=None):
    """Same as state_passing_fwd (reference name kept)."""
    return state_passing_fwd(states, dA_chunk_cumsum, initial_states, seq_idx, chunk_size,
                             out_dtype)

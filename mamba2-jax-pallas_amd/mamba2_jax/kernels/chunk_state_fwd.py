"""chunk_state_fwd / chunk_state_varlen on MI355X (MFMA kernels in libm2ssd.so).

Drop-in for reference kernels/chunk_state_fwd.py (chunk_state_fwd :424-441,
chunk_state_fwd_mosaic :373-421, chunk_state_varlen_mosaic :448-597), for
every head dim and dstate: the reference pads both up to its tiles
(:281-295); here sizes the kernels do not tile run through the exact padding /
head splitting / dstate blocks of kernels/_shapes.py.  Tile keyword
arguments (BM, BK, BN, num_stages) are accepted and ignored: the HIP kernels
pick their own tiles.
"""

from __future__ import annotations

import math

import torch

from .. import _lib as L
from . import _shapes as S


def _io_dtype(*ts):
    """Common element type of x / B / C / z: promoted to float32 on mismatch."""
    dts = {t.dtype for t in ts if t is not None}
    if len(dts) == 1:
        d = dts.pop()
        if d in (torch.float32, torch.bfloat16):
            return d
    return torch.float32


def _seq_idx(seq_idx, batch, seqlen):
    if seq_idx is None:
        return None
    L.require(seq_idx.shape == (batch, seqlen),
              lambda: f"seq_idx.shape={tuple(seq_idx.shape)} != ({batch}, {seqlen})")
    return L.dev_contig(seq_idx, torch.int32)


def chunk_state_fwd(x, B, dt, dA_cumsum, seq_idx=None, BM=64, BK=64, BN=64, num_stages=2):
    """states (batch, nchunks, nheads, headdim, dstate) float32:
    sum over each chunk of exp(dA[-1] - dA[q]) * dt[q] * x[q]^T B[q]."""
    L.device_of(x, B, dt, dA_cumsum, seq_idx)
    L.require(x.dim() == 4 and B.dim() == 4, "x must be (b, L, H, P) and B (b, L, G, N)")
    batch, seqlen, nheads, headdim = x.shape
    _, _, ngroups, dstate = B.shape
    L.require(tuple(B.shape[:2]) == (batch, seqlen), "B and x disagree on (batch, seqlen)")
    L.require(dt.dim() == 4 and dt.shape[0] == batch and dt.shape[1] == nheads,
              f"dt must be (batch, nheads, nchunks, chunk_size), got {tuple(dt.shape)}")
    nchunks, chunk_size = int(dt.shape[2]), int(dt.shape[3])
    L.require(tuple(dA_cumsum.shape) == tuple(dt.shape), "dA_cumsum.shape != dt.shape")
    L.require(nheads % ngroups == 0, "nheads must be a multiple of ngroups")
    L.require(nchunks == math.ceil(seqlen / chunk_size), "nchunks != ceil(seqlen / chunk_size)")
    return _chunk_state(x, B, dt, dA_cumsum, seq_idx)


def _chunk_state(x, B, dt, dA_cumsum, seq_idx, native=None):
    """chunk_state_fwd for any head dim / dstate (kernels/_shapes.py);
    `native` runs the mapped problem (default: the library)."""
    native = native or _chunk_state_native
    P, N = x.shape[-1], B.shape[-1]
    if N > S.NMAX:
        # states are independent per column: one call per column block
        out = None
        for n0, n1 in S.n_blocks(N):
            r = _chunk_state(x, B[..., n0:n1], dt, dA_cumsum, seq_idx, native)
            if out is None:
                out = r.new_empty(tuple(r.shape[:-1]) + (N,))
            out[..., n0:n1] = r
        return out
    Pp, k = S.p_plan_stage(P)
    Np = S.n_pad(N)
    if (Pp, k, Np) == (P, 1, N):
        return native(x, B, dt, dA_cumsum, seq_idx)
    out = native(S.split_heads(S.pad_last(x, Pp), 2, k), S.pad_last(B, Np),
                 S.repeat_heads(dt, 1, k), S.repeat_heads(dA_cumsum, 1, k), seq_idx)
    return S.merge_heads(out, 2, k, P, N)


def _chunk_state_native(x, B, dt, dA_cumsum, seq_idx):
    dev = x.device
    batch, seqlen, nheads, headdim = x.shape
    _, _, ngroups, dstate = B.shape
    nchunks, chunk_size = int(dt.shape[2]), int(dt.shape[3])
    io = _io_dtype(x, B)
    x_c, B_c = L.dev_contig(x, io), L.dev_contig(B, io)
    dt_c, dA_c = L.dev_contig(dt, torch.float32), L.dev_contig(dA_cumsum, torch.float32)
    seq = _seq_idx(seq_idx, batch, seqlen)
    out = torch.empty((batch, nchunks, nheads, headdim, dstate), dtype=torch.float32, device=dev)
    args = L.ChunkStateArgs(
        x=L.ptr(x_c), B=L.ptr(B_c), dt=L.ptr(dt_c), dA_cumsum=L.ptr(dA_c), seq_idx=L.ptr(seq),
        states=L.ptr(out), batch=batch, seqlen=seqlen, nheads=nheads, headdim=headdim,
        ngroups=ngroups, dstate=dstate, chunk_size=chunk_size, dtype=L.dtype_code(x_c, "x"))
    with torch.cuda.device(dev):
        L.call("m2_chunk_state", args, L.stream_of(dev))
    return out


def chunk_state_fwd_mosaic(x, B, dt, dA_cumsum, seq_idx=None, BM=64, BK=64, BN=64,
                           num_stages=2):
    """Same as chunk_state_fwd (reference name kept)."""
    return chunk_state_fwd(x, B, dt, dA_cumsum, seq_idx=seq_idx)


def chunk_state_varlen_mosaic(B, x, dt, dA_cumsum, cu_seqlens, chunk_states, BM=64, BK=64,
                              BN=64, num_stages=2):
    """Final state of each packed sequence, (nseq, nheads, headdim, dstate) float32.

    B (total_seqlen, ngroups, dstate), x (total_seqlen, nheads, headdim),
    dt / dA_cumsum (nheads, nchunks, chunk_size), cu_seqlens (nseq + 1,) int32,
    chunk_states (nchunks, nheads, headdim, dstate): the state entering each chunk.
    """
    L.device_of(B, x, dt, dA_cumsum, cu_seqlens, chunk_states)
    L.require(x.dim() == 3 and B.dim() == 3, "x must be (L, H, P) and B (L, G, N)")
    total, nheads, headdim = x.shape
    _, ngroups, dstate = B.shape
    L.require(B.shape[0] == total, "B and x disagree on total_seqlen")
    L.require(dt.dim() == 3 and dt.shape[0] == nheads, "dt must be (nheads, nchunks, chunk_size)")
    nchunks, chunk_size = int(dt.shape[1]), int(dt.shape[2])
    L.require(tuple(dA_cumsum.shape) == tuple(dt.shape), "dA_cumsum.shape != dt.shape")
    L.require(tuple(chunk_states.shape) == (nchunks, nheads, headdim, dstate),
              f"chunk_states.shape={tuple(chunk_states.shape)} != "
              f"({nchunks}, {nheads}, {headdim}, {dstate})")
    L.require(cu_seqlens.dim() == 1 and cu_seqlens.shape[0] >= 2, "cu_seqlens must be (nseq + 1,)")
    L.require(nheads % ngroups == 0, "nheads must be a multiple of ngroups")
    return _varlen(B, x, dt, dA_cumsum, cu_seqlens, chunk_states)


def _varlen(B, x, dt, dA_cumsum, cu_seqlens, chunk_states, native=None):
    """chunk_state_varlen for any head dim / dstate (kernels/_shapes.py);
    `native` runs the mapped problem (default: the library)."""
    native = native or _varlen_native
    P, N = x.shape[-1], B.shape[-1]
    if N > S.NMAX:
        out = None
        for n0, n1 in S.n_blocks(N):
            r = _varlen(B[..., n0:n1], x, dt, dA_cumsum, cu_seqlens, chunk_states[..., n0:n1],
                        native)
            if out is None:
                out = r.new_empty(tuple(r.shape[:-1]) + (N,))
            out[..., n0:n1] = r
        return out
    Pp, k = S.p_plan_stage(P)
    Np = S.n_pad(N)
    if (Pp, k, Np) == (P, 1, N):
        return native(B, x, dt, dA_cumsum, cu_seqlens, chunk_states)
    cs = S.split_heads(S.pad_dim(S.pad_last(chunk_states, Np), 2, Pp), 1, k)
    out = native(S.pad_last(B, Np), S.split_heads(S.pad_last(x, Pp), 1, k),
                 S.repeat_heads(dt, 0, k), S.repeat_heads(dA_cumsum, 0, k), cu_seqlens, cs)
    return S.merge_heads(out, 1, k, P, N)


def _varlen_native(B, x, dt, dA_cumsum, cu_seqlens, chunk_states):
    dev = x.device
    total, nheads, headdim = x.shape
    _, ngroups, dstate = B.shape
    nchunks, chunk_size = int(dt.shape[1]), int(dt.shape[2])
    nseq = int(cu_seqlens.shape[0]) - 1
    io = _io_dtype(x, B)
    x_c, B_c = L.dev_contig(x, io), L.dev_contig(B, io)
    dt_c, dA_c = L.dev_contig(dt, torch.float32), L.dev_contig(dA_cumsum, torch.float32)
    cu = L.dev_contig(cu_seqlens, torch.int32)
    cs = chunk_states
    if cs.dtype not in (torch.float32, torch.bfloat16):
        cs = cs.to(torch.float32)
    cs = L.dev_contig(cs)
    out = torch.empty((nseq, nheads, headdim, dstate), dtype=torch.float32, device=dev)
    args = L.ChunkStateVarlenArgs(
        B=L.ptr(B_c), x=L.ptr(x_c), dt=L.ptr(dt_c), dA_cumsum=L.ptr(dA_c), cu_seqlens=L.ptr(cu),
        chunk_states=L.ptr(cs), out=L.ptr(out), seqlen=total, nseq=nseq, nheads=nheads,
        headdim=headdim, ngroups=ngroups, dstate=dstate, nchunks=nchunks,
        chunk_size=chunk_size, dtype=L.dtype_code(x_c, "x"),
        states_dtype=L.dtype_code(cs, "chunk_states"))
    with torch.cuda.device(dev):
        L.call("m2_chunk_state_varlen", args, L.stream_of(dev))
    return out

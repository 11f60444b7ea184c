"""chunk_scan_fwd on MI355X: the intra-chunk causal scan + carried-state term +
D skip + z gate in one MFMA kernel (libm2ssd.so: m2_chunk_scan).

Drop-in for reference kernels/chunk_scan_fwd.py (chunk_scan_fwd :579-600,
chunk_scan_fwd_mosaic :482-572), for every head dim and dstate: the
reference pads both up to its tiles (:367-390); here sizes the kernels do not
tile run through the exact padding / head splitting / dstate blocks of
kernels/_shapes.py.  Tile keyword arguments are accepted and ignored.
"""

from __future__ import annotations

import math

import torch

from .. import _lib as L
from . import _shapes as S
from .chunk_state_fwd import _io_dtype, _seq_idx


def chunk_scan_fwd(cb, x, dt, dA_cumsum, C, states, D=None, z=None, seq_idx=None,
                   BM=64, BK=64, BN=64, num_stages=2):
    """-> (out, out_x): float32 (batch, seqlen, nheads, headdim); out_x is the
    output before the z gate (None without z).

    cb (batch, nchunks, ngroups, Q, Q), x (batch, seqlen, nheads, headdim),
    dt / dA_cumsum (batch, nheads, nchunks, Q), C (batch, seqlen, ngroups, dstate),
    states (batch, nchunks, nheads, headdim, dstate) = the state entering each
    chunk (rounded to x's dtype before use), D (nheads,) or (nheads, headdim).
    """
    L.device_of(cb, x, dt, dA_cumsum, C, states, D, z, seq_idx)
    L.require(x.dim() == 4, "x must be (batch, seqlen, nheads, headdim)")
    batch, seqlen, nheads, hdim = x.shape
    L.require(C.dim() == 4 and tuple(C.shape[:2]) == (batch, seqlen),
              "C must be (batch, seqlen, ngroups, dstate)")
    _, _, ngroups, dstate = C.shape
    L.require(dt.dim() == 4 and tuple(dt.shape[:2]) == (batch, nheads),
              "dt must be (batch, nheads, nchunks, chunk_size)")
    nchunks, chunk_size = int(dt.shape[2]), int(dt.shape[3])
    L.require(tuple(dA_cumsum.shape) == tuple(dt.shape), "dA_cumsum.shape != dt.shape")
    L.require(nchunks == math.ceil(seqlen / chunk_size), "nchunks != ceil(seqlen / chunk_size)")
    L.require(tuple(cb.shape) == (batch, nchunks, ngroups, chunk_size, chunk_size),
              f"cb.shape={tuple(cb.shape)} != {(batch, nchunks, ngroups, chunk_size, chunk_size)}")
    L.require(tuple(states.shape) == (batch, nchunks, nheads, hdim, dstate),
              f"states.shape={tuple(states.shape)} != {(batch, nchunks, nheads, hdim, dstate)}")
    L.require(nheads % ngroups == 0, "nheads must be a multiple of ngroups")
    if D is not None:
        L.require(tuple(D.shape) in ((nheads,), (nheads, hdim)), f"D.shape={tuple(D.shape)}")
    if z is not None:
        L.require(tuple(z.shape) == tuple(x.shape), "z.shape != x.shape")
    return _chunk_scan(cb, x, dt, dA_cumsum, C, states, D, z, seq_idx)


def _chunk_scan(cb, x, dt, dA_cumsum, C, states, D, z, seq_idx, native=None):
    """chunk_scan_fwd for any head dim / dstate (kernels/_shapes.py);
    `native` runs the mapped problem (default: the library)."""
    native = native or _chunk_scan_native
    P, N = x.shape[-1], C.shape[-1]
    if N > S.NMAX:
        # the inter-chunk term sums over dstate: one call per column block,
        # the outputs before the gate added (CB and D in block 0 only), then
        # the z gate
        out_x = None
        for j, (n0, n1) in enumerate(S.n_blocks(N)):
            o, _ = _chunk_scan(cb if j == 0 else torch.zeros_like(cb), x, dt, dA_cumsum,
                               C[..., n0:n1], states[..., n0:n1], D if j == 0 else None, None,
                               seq_idx, native)
            out_x = o if out_x is None else out_x.add_(o)
        if z is None:
            return out_x, None
        return S.gate(out_x, z), out_x
    Pp, k = S.p_plan_stage(P)
    Np = S.n_pad(N, native=(32,) + S.NATIVE_N)
    if (Pp, k, Np) == (P, 1, N):
        return native(cb, x, dt, dA_cumsum, C, states, D, z, seq_idx)
    st = S.split_heads(S.pad_dim(S.pad_last(states, Np), 3, Pp), 2, k)
    out, out_x = native(cb, S.split_heads(S.pad_last(x, Pp), 2, k), S.repeat_heads(dt, 1, k),
                        S.repeat_heads(dA_cumsum, 1, k), S.pad_last(C, Np), st,
                        S.adapt_D(D, k, Pp), S.split_heads(S.pad_last(z, Pp), 2, k), seq_idx)
    return S.merge_heads(out, 2, k, P), S.merge_heads(out_x, 2, k, P)


def _chunk_scan_native(cb, x, dt, dA_cumsum, C, states, D, z, seq_idx):
    dev = x.device
    batch, seqlen, nheads, hdim = x.shape
    _, _, ngroups, dstate = C.shape
    chunk_size = int(dt.shape[3])
    D_has_hdim = int(D is not None and D.dim() == 2)
    io = _io_dtype(x, C, z)
    x_c, C_c, z_c = L.dev_contig(x, io), L.dev_contig(C, io), L.dev_contig(z, io)
    cb_c = L.dev_contig(cb if cb.dtype in (torch.float32, torch.bfloat16) else cb.float())
    st = L.dev_contig(states if states.dtype in (torch.float32, torch.bfloat16) else states.float())
    dt_c, dA_c = L.dev_contig(dt, torch.float32), L.dev_contig(dA_cumsum, torch.float32)
    D_c = L.dev_contig(D, torch.float32)
    seq = _seq_idx(seq_idx, batch, seqlen)
    out = torch.empty((batch, seqlen, nheads, hdim), dtype=torch.float32, device=dev)
    out_x = torch.empty_like(out) if z is not None else None
    args = L.ChunkScanArgs(
        cb=L.ptr(cb_c), x=L.ptr(x_c), dt=L.ptr(dt_c), dA_cumsum=L.ptr(dA_c), C=L.ptr(C_c),
        states=L.ptr(st), D=L.ptr(D_c), z=L.ptr(z_c), seq_idx=L.ptr(seq), out=L.ptr(out),
        out_x=L.ptr(out_x), batch=batch, seqlen=seqlen, nheads=nheads, headdim=hdim,
        ngroups=ngroups, dstate=dstate, chunk_size=chunk_size, dtype=L.dtype_code(x_c, "x"),
        cb_dtype=L.dtype_code(cb_c, "cb"), states_dtype=L.dtype_code(st, "states"),
        D_has_hdim=D_has_hdim)
    with torch.cuda.device(dev):
        L.call("m2_chunk_scan", args, L.stream_of(dev))
    return out, out_x


def chunk_scan_fwd_mosaic(cb, x, dt, dA_cumsum, C, states, D=None, z=None, seq_idx=None,
                          BM=64, BK=64, BN=64, num_stages=2):
    """Same as chunk_scan_fwd (reference name kept)."""
    return chunk_scan_fwd(cb, x, dt, dA_cumsum, C, states, D=D, z=z, seq_idx=seq_idx)

"""mamba_chunk_scan_combined_fwd on MI355X: the whole SSD layer forward.

Drop-in for reference kernels/ssd_combined.py:46-203, for every head dim and
dstate (sizes the kernels do not tile run through the exact padding / head
splitting / dstate blocks of kernels/_shapes.py).  One call into
libm2ssd.so (m2_ssd_combined) enqueues the five stage kernels
(chunk_cumsum -> chunk_state -> state_passing -> bmm_chunk -> chunk_scan, plus
chunk_state_varlen when varlen states are requested) on the current stream;
the intermediates live in a workspace drawn from torch's caching allocator.
As in the reference, the state entering each chunk is kept in x's dtype,
while the output and the final states are float32.
"""

from __future__ import annotations

import math

import torch

from .. import _lib as L
from . import _shapes as S
from .chunk_state_fwd import _io_dtype, _seq_idx


def _events_array(events):
    """Raw hipEvent_t handles of 7 events: torch.cuda.Event objects (created on
    first record), objects with a raw `cuda_event` handle, or None (that point
    is not recorded)."""
    import ctypes
    if events is None:
        return None, None
    if len(events) != 7:
        raise ValueError("_stage_events needs 7 events")
    for e in events:
        if isinstance(e, torch.cuda.Event) and not e.cuda_event:
            e.record()          # forces creation of the underlying event
    arr = (ctypes.c_void_p * 7)(*[None if e is None else e.cuda_event for e in events])
    return arr, ctypes.cast(arr, ctypes.c_void_p).value


def mamba_chunk_scan_combined_fwd(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                                  initial_states=None, seq_idx=None, cu_seqlens=None,
                                  dt_softplus=False, dt_limit=(0.0, float("inf")),
                                  return_final_states=False, return_varlen_states=False,
                                  *, _stage_events=None):
    """SSD chunked-scan forward.

    x (batch, seqlen, nheads, headdim), dt (batch, seqlen, nheads), A (nheads,),
    B / C (batch, seqlen, ngroups, dstate), D (nheads,) or (nheads, headdim),
    z like x, dt_bias (nheads,), initial_states (batch, nheads, headdim, dstate),
    seq_idx (batch, seqlen) int32, cu_seqlens (nseq + 1,) int32.

    Returns out (float32, like x), then final_states (batch, nheads, headdim,
    dstate) if return_final_states, then varlen_states (nseq, nheads, headdim,
    dstate) if return_varlen_states -- the reference's arity
    (kernels/ssd_combined.py:194-203).

    ``_stage_events`` (optional, 7 events) is a profiling hook: the events are
    recorded before the first and after each of the five stages, and after the
    varlen states when they are requested; None entries are skipped.
    """
    L.device_of(x, dt, A, B, C, D, z, dt_bias, initial_states, seq_idx, cu_seqlens)
    L.require(x.dim() == 4, "x must be (batch, seqlen, nheads, headdim)")
    batch, seqlen, nheads, headdim = x.shape
    L.require(B.dim() == 4 and B.shape[:2] == x.shape[:2],
              "B must be (batch, seqlen, ngroups, dstate)")
    _, _, ngroups, dstate = B.shape
    L.require(C.shape == B.shape, "C.shape != B.shape")
    L.require(dt.shape == x.shape[:3], lambda: f"dt.shape={tuple(dt.shape)}")
    L.require(A.shape == (nheads,), lambda: f"A.shape={tuple(A.shape)} != ({nheads},)")
    L.require(nheads % ngroups == 0, "nheads must be a multiple of ngroups")
    if dt_bias is not None:
        L.require(dt_bias.shape == (nheads,), lambda: f"dt_bias.shape={tuple(dt_bias.shape)}")
    if D is not None:
        L.require(D.shape == (nheads,) or D.shape == (nheads, headdim),
                  lambda: f"D.shape={tuple(D.shape)}")
    if z is not None:
        L.require(z.shape == x.shape, "z.shape != x.shape")
    if initial_states is not None:
        L.require(initial_states.shape == (batch, nheads, headdim, dstate),
                  lambda: f"initial_states.shape={tuple(initial_states.shape)}")
    chunk_size = int(chunk_size)
    L.require(chunk_size > 0, "chunk_size must be positive")
    if not return_varlen_states:
        cu_seqlens = None
    nseq = 0
    if cu_seqlens is not None:
        L.require(batch == 1, "cu_seqlens for varlen states is only supported with batch=1")
        L.require(cu_seqlens.dim() == 1 and cu_seqlens.shape[0] >= 2,
                  "cu_seqlens must be (num_sequences + 1,)")
        nseq = int(cu_seqlens.shape[0]) - 1
    elif return_varlen_states:
        raise L.M2ShapeError("return_varlen_states needs cu_seqlens")

    out, fin, vs = _combined(x, dt, A, B, C, chunk_size, D, z, dt_bias, initial_states, seq_idx,
                             cu_seqlens, nseq, bool(dt_softplus), dt_limit, return_final_states,
                             _stage_events)
    if not return_varlen_states:
        return (out, fin) if return_final_states else out
    return (out, fin, vs) if return_final_states else (out, vs)


def _combined(x, dt, A, B, C, chunk_size, D, z, dt_bias, init, seq_idx, cu_seqlens, nseq,
              dt_softplus, dt_limit, want_final, events, native=None):
    """(out, final or None, varlen or None) for any head dim and dstate: sizes
    the kernels do not tile are mapped onto ones they do (kernels/_shapes.py).
    `native` runs the mapped problem (default: the library; the CPU tests
    pass the oracle to check the mapping)."""
    native = native or _combined_native
    N = B.shape[-1]
    if N > S.NMAX:
        # column blocks: outputs added, states concatenated; D in block 0 only
        out = None
        fins, vss = [], []
        for j, (n0, n1) in enumerate(S.n_blocks(N)):
            o, f, v = _combined(x, dt, A, B[..., n0:n1], C[..., n0:n1], chunk_size,
                                D if j == 0 else None, z, dt_bias,
                                None if init is None else init[..., n0:n1], seq_idx, cu_seqlens,
                                nseq, dt_softplus, dt_limit, want_final, None, native)
            out = o if out is None else out.add_(o)
            fins.append(f)
            vss.append(v)
        fin = torch.cat(fins, dim=-1) if want_final else None
        vs = torch.cat(vss, dim=-1) if cu_seqlens is not None else None
        return out, fin, vs
    P = x.shape[-1]
    Pp, k = S.p_plan_layer(P)
    Np = S.n_pad(N)
    if (Pp, k, Np) == (P, 1, N):
        return native(x, dt, A, B, C, chunk_size, D, z, dt_bias, init, seq_idx, cu_seqlens,
                      nseq, dt_softplus, dt_limit, want_final, events)
    xs = S.split_heads(S.pad_last(x, Pp), 2, k)
    zs = S.split_heads(S.pad_last(z, Pp), 2, k)
    inits = None
    if init is not None:
        inits = S.split_heads(S.pad_dim(S.pad_last(init, Np), 2, Pp), 1, k)
    o, f, v = native(xs, S.repeat_heads(dt, 2, k), S.repeat_heads(A, 0, k), S.pad_last(B, Np),
                     S.pad_last(C, Np), chunk_size, S.adapt_D(D, k, Pp), zs,
                     S.repeat_heads(dt_bias, 0, k), inits, seq_idx, cu_seqlens, nseq, dt_softplus,
                     dt_limit, want_final, events)
    return (S.merge_heads(o, 2, k, P), S.merge_heads(f, 1, k, P, N),
            S.merge_heads(v, 1, k, P, N))


def _combined_native(x, dt, A, B, C, chunk_size, D, z, dt_bias, init, seq_idx, cu_seqlens, nseq,
                     dt_softplus, dt_limit, want_final, events):
    """One m2_ssd_combined call (sizes the kernels take)."""
    dev = x.device
    batch, seqlen, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    D_has_hdim = int(D is not None and D.dim() == 2)
    return_final_states = want_final
    io = _io_dtype(x, B, C, z)
    x_c, B_c, C_c, z_c = (L.dev_contig(t, io) for t in (x, B, C, z))
    dt_c = L.dev_contig(dt if dt.dtype in (torch.float32, torch.bfloat16) else dt.float())
    A_c, D_c, bias_c = (L.dev_contig(t, torch.float32) for t in (A, D, dt_bias))
    init = L.dev_contig(init, torch.float32)
    seq = _seq_idx(seq_idx, batch, seqlen)
    cu = L.dev_contig(cu_seqlens, torch.int32)

    out = torch.empty((batch, seqlen, nheads, headdim), dtype=torch.float32, device=dev)
    fin = (torch.empty((batch, nheads, headdim, dstate), dtype=torch.float32, device=dev)
           if return_final_states else None)
    vs = (torch.empty((nseq, nheads, headdim, dstate), dtype=torch.float32, device=dev)
          if cu is not None else None)
    ev_keep, ev_ptr = _events_array(events)
    args = L.SsdCombinedArgs(
        x=L.ptr(x_c), dt=L.ptr(dt_c), A=L.ptr(A_c), B=L.ptr(B_c), C=L.ptr(C_c), D=L.ptr(D_c),
        z=L.ptr(z_c), dt_bias=L.ptr(bias_c), initial_states=L.ptr(init), seq_idx=L.ptr(seq),
        cu_seqlens=L.ptr(cu), out=L.ptr(out), final_states=L.ptr(fin), varlen_states=L.ptr(vs),
        batch=batch, seqlen=seqlen, nheads=nheads, headdim=headdim, ngroups=ngroups,
        dstate=dstate, chunk_size=chunk_size, nseq=nseq, dtype=L.dtype_code(x_c, "x"),
        dt_dtype=L.dtype_code(dt_c, "dt"), D_has_hdim=D_has_hdim,
        dt_softplus=int(dt_softplus), dt_min=float(dt_limit[0]),
        dt_max=float(dt_limit[1]), stage_events=ev_ptr)
    # the workspace size depends on the sizes, dtypes and flags, on which
    # optional inputs are given and on the library's shape-based choices (the
    # device's CU count, the testing overrides); the library checks the size
    # it is handed against its own again
    key = (dev.index, batch, seqlen, nheads, headdim, ngroups, dstate, chunk_size, nseq,
           args.dtype, args.dt_dtype, D_has_hdim, args.dt_softplus, D_c is not None,
           z_c is not None, bias_c is not None, init is not None, seq is not None,
           cu is not None, fin is not None, L.override_epoch())
    ws_bytes = _ws_cache.get(key)
    if ws_bytes is None:
        import ctypes
        ws_bytes = L.load_library().m2_ssd_combined_workspace_size(ctypes.byref(args))
        L.require(ws_bytes > 0, "m2_ssd_combined_workspace_size rejected the arguments")
        if len(_ws_cache) > 256:
            _ws_cache.clear()
        _ws_cache[key] = ws_bytes
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws_bytes
    if dev.index == torch.cuda.current_device():
        L.call("m2_ssd_combined", args, L.stream_of(dev))
    else:
        with torch.cuda.device(dev):
            L.call("m2_ssd_combined", args, L.stream_of(dev))
    del ev_keep
    return out, fin, vs


_ws_cache = {}

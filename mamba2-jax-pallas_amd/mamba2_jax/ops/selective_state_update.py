"""selective_state_update on MI355X: one decode token as a single fused HIP
kernel that reads and writes the fp32 state once (libm2ssd.so:
m2_selective_state_update).

Drop-in for reference ops/selective_state_update.py:22-123: by default the
caller's ``state`` is left untouched and the updated state is returned as a
new tensor (the reference is functional, and its tests recompute the expected
state from ``state`` after the call, tests/test_mamba2_ops.py:43-56).  The
kernel then reads ``state`` and writes the new tensor: the same HBM bytes as an
in-place update, one extra allocation.  A decode loop that owns its state
passes the keyword-only ``inplace=True``: a float32, contiguous, 16-byte
aligned state is then updated in place and returned (what JAX's
input_output_aliases + buffer donation give), so a step allocates no state.
"""

from __future__ import annotations

import torch

from .. import _lib as L
from ..kernels.chunk_state_fwd import _io_dtype


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False, *, inplace=False):
    """-> (new_state (batch, nheads, headdim, dstate) float32, out (batch, nheads, headdim) float32)

    state (b, H, P, N); x (b, H, P); dt (b, H) or (b, H, P); A (H,) or (H, P, N);
    B, C (b, G, N); D (H,) or (H, P); z (b, H, P); dt_bias (H,) or (H, P).
    dt' = softplus?(dt + dt_bias); state = state * exp(dt' A) + dt' x B;
    out = state @ C + D x; out *= silu(z).  No dt_limit clamp (as the reference).
    """
    dev = L.device_of(state, x, dt, A, B, C, D, z, dt_bias)
    L.require(state.dim() == 4, "state must be (batch, nheads, headdim, dstate)")
    batch, nheads, headdim, dstate = state.shape
    L.require(tuple(x.shape) == (batch, nheads, headdim), f"x.shape={tuple(x.shape)}")
    L.require(B.dim() == 3 and B.shape[0] == batch and B.shape[2] == dstate,
              f"B.shape={tuple(B.shape)}")
    ngroups = int(B.shape[1])
    L.require(tuple(C.shape) == tuple(B.shape), "C.shape != B.shape")
    L.require(nheads % ngroups == 0, "nheads must be a multiple of ngroups")
    if dt.dim() == 2:
        L.require(tuple(dt.shape) == (batch, nheads), f"dt.shape={tuple(dt.shape)}")
        dt_has_hdim = 0
    else:
        L.require(tuple(dt.shape) == (batch, nheads, headdim), f"dt.shape={tuple(dt.shape)}")
        dt_has_hdim = 1
    if A.dim() == 1:
        L.require(tuple(A.shape) == (nheads,), f"A.shape={tuple(A.shape)}")
        A_full = 0
    else:
        L.require(tuple(A.shape) == (nheads, headdim, dstate), f"A.shape={tuple(A.shape)}")
        A_full = 1
    D_has_hdim = bias_has_hdim = 0
    if D is not None:
        D_has_hdim = int(D.dim() == 2)
        L.require(tuple(D.shape) == ((nheads, headdim) if D_has_hdim else (nheads,)),
                  f"D.shape={tuple(D.shape)}")
    if dt_bias is not None:
        bias_has_hdim = int(dt_bias.dim() == 2)
        L.require(tuple(dt_bias.shape) == ((nheads, headdim) if bias_has_hdim else (nheads,)),
                  f"dt_bias.shape={tuple(dt_bias.shape)}")
        # the reference adds them by broadcasting (ops/selective_state_update.py:72),
        # which aligns heads only for dt (b, H) + dt_bias (H,) and dt (b, H, P) +
        # dt_bias (H, P); the mixed pairs fail there (or misalign when sizes coincide)
        L.require(bias_has_hdim == dt_has_hdim,
                  f"dt.shape={tuple(dt.shape)} with dt_bias.shape={tuple(dt_bias.shape)}: "
                  "pass dt (batch, nheads) with dt_bias (nheads,), or dt (batch, nheads, headdim) "
                  "with dt_bias (nheads, headdim)")
    if z is not None:
        L.require(tuple(z.shape) == tuple(x.shape), "z.shape != x.shape")

    direct = state.dtype == torch.float32 and state.is_contiguous() and state.data_ptr() % 16 == 0
    if inplace and direct:
        src = new = state
    else:
        # the kernel reads the caller's state (or a float32 copy of it) and
        # writes a fresh tensor: the caller's state stays untouched
        src = state if direct else state.to(torch.float32).contiguous()
        new = torch.empty((batch, nheads, headdim, dstate), dtype=torch.float32, device=dev)
    io = _io_dtype(x, B, C, z)
    x_c, B_c, C_c, z_c = (L.dev_contig(t, io) for t in (x, B, C, z))
    dt_c = L.dev_contig(dt if dt.dtype in (torch.float32, torch.bfloat16) else dt.float())
    A_c, D_c, bias_c = (L.dev_contig(t, torch.float32) for t in (A, D, dt_bias))
    out = torch.empty((batch, nheads, headdim), dtype=torch.float32, device=dev)
    args = L.SsuArgs(
        state=L.ptr(src), new_state=L.ptr(new), x=L.ptr(x_c), dt=L.ptr(dt_c), A=L.ptr(A_c),
        B=L.ptr(B_c), C=L.ptr(C_c), D=L.ptr(D_c), z=L.ptr(z_c), dt_bias=L.ptr(bias_c), out=L.ptr(out), batch=batch,
        nheads=nheads, headdim=headdim, ngroups=ngroups, dstate=dstate,
        dtype=L.dtype_code(x_c, "x"), dt_dtype=L.dtype_code(dt_c, "dt"),
        dt_has_hdim=dt_has_hdim, A_full=A_full, D_has_hdim=D_has_hdim,
        dt_bias_has_hdim=bias_has_hdim, dt_softplus=int(bool(dt_softplus)))
    with torch.cuda.device(dev):
        L.call("m2_selective_state_update", args, L.stream_of(dev))
    return new, out

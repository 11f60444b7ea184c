"""Head dims and state sizes the HIP kernels do not tile natively, mapped onto
ones they do, so that every operator accepts every size the reference does.

The reference pads headdim and dstate up to its tile sizes in the Python
preprocessing in front of each Pallas call (kernels/chunk_state_fwd.py:281-295,
kernels/chunk_scan_fwd.py:367-390, kernels/bmm_chunk_fwd.py:206-218).  The
kernels here are instantiated for head dim 32 / 64 / 128 (the fused layer
kernels for 64) and dstate 64 / 128 / 256; other sizes reach them through
transformations that leave every result value unchanged:

* dstate zero padding: columns n >= N of B, C, the states and the initial
  state are zero, so they add exact zeros to every product over n (C B^T,
  C state^T) and the padded state columns stay zero; they are sliced off.
* head dim zero padding: rows p >= P of x, z and the states are zero; every
  output row p is a function of row p alone, and the padded rows are sliced
  off.
* head splitting: a head of head dim k * 64 is k heads of head dim 64 that
  share its dt, A, dt_bias and group.  x [b, L, H, k * 64] and
  [b, L, k * H, 64] are the same memory (so are z, out, the states and D
  [H, k * 64]); only the per-head vectors dt, A, dt_bias and D [H] are
  repeated.  Head h * k + j of the split problem falls in group g of head h,
  since (h * k + j) // (k * H / G) == h // (H / G).
* dstate blocks (above 256): states are independent per column, and the
  outputs are sums over columns, so each block of <= 256 columns runs on its
  own and the outputs are added (the D skip and the intra-chunk term counted
  in one block only).  The z gate is linear in the output.  The bf16 rounding
  points of the reference (CB, the inter-chunk product) then fall on each
  block's partial sum instead of the whole sum.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

# dstate sizes the chunk_state / varlen / fused kernels are built for
NATIVE_N = (64, 128, 256)
NMAX = 256
# head dims the stage kernels are built for, and the fused layer's
NATIVE_P_STAGE = (32, 64, 128)
NATIVE_P_LAYER = (32, 64)
SPLIT_P = 64


def n_blocks(N):
    """Column ranges [(n0, n1), ...] of at most NMAX columns covering 0..N."""
    return [(n0, min(n0 + NMAX, N)) for n0 in range(0, N, NMAX)]


def n_pad(N, native=NATIVE_N):
    """dstate the kernels run for N <= NMAX: N itself when native, else the
    next native size."""
    if N in native:
        return N
    for n in NATIVE_N:
        if n >= N:
            return n
    raise ValueError(f"dstate {N} > {NMAX}: split into column blocks first")


def p_plan_stage(P):
    """(padded head dim Pp, split factor k) for the stage operators: the
    kernels run k heads of head dim Pp // k per head.  Up to 128 the next
    native head dim; above, heads of 64."""
    if P in NATIVE_P_STAGE:
        return P, 1
    if P < max(NATIVE_P_STAGE):
        return min(p for p in NATIVE_P_STAGE if p >= P), 1
    Pp = SPLIT_P * math.ceil(P / SPLIT_P)
    return Pp, Pp // SPLIT_P


def p_plan_layer(P):
    """(Pp, k) for the combined forward, whose fused kernels take head dim 64:
    every other head dim but 32 runs as heads of 64 (128 = two heads of 64
    with no copy of x)."""
    if P in NATIVE_P_LAYER:
        return P, 1
    Pp = SPLIT_P * math.ceil(P / SPLIT_P)
    return Pp, Pp // SPLIT_P


def pad_last(t, size):
    """t zero-padded (or kept) to `size` along its last dimension."""
    if t is None or t.shape[-1] == size:
        return t
    return F.pad(t, (0, size - t.shape[-1]))


def pad_dim(t, dim, size):
    """t zero-padded to `size` along dimension `dim`."""
    if t is None or t.shape[dim] == size:
        return t
    dim = dim % t.dim()
    pads = [0, 0] * (t.dim() - dim - 1) + [0, size - t.shape[dim]]
    return F.pad(t, pads)


def split_heads(t, head_dim, k):
    """View [.., H, k * Ps, ..] (heads at `head_dim`, head dim right after) as
    [.., k * H, Ps, ..]; t must be contiguous in those two dimensions."""
    if t is None or k == 1:
        return t
    t = t.contiguous()
    shape = list(t.shape)
    H, Pp = shape[head_dim], shape[head_dim + 1]
    shape[head_dim:head_dim + 2] = [H * k, Pp // k]
    return t.view(shape)


def merge_heads(t, head_dim, k, P, N=None):
    """Inverse of split_heads, then the padding sliced off: [.., k * H, Ps, (Np)]
    -> [.., H, P, (N)] (contiguous)."""
    if t is None:
        return None
    shape = list(t.shape)
    if k > 1:
        Hk, Ps = shape[head_dim], shape[head_dim + 1]
        shape[head_dim:head_dim + 2] = [Hk // k, Ps * k]
        t = t.view(shape)
    sl = [slice(None)] * t.dim()
    sl[head_dim + 1] = slice(0, P)
    if N is not None:
        sl[head_dim + 2] = slice(0, N)
    out = t[tuple(sl)]
    return out if out.is_contiguous() else out.contiguous()


def repeat_heads(t, dim, k):
    """Per-head tensor with each head repeated k times along `dim` (the split
    heads of one head share it)."""
    if t is None or k == 1:
        return t
    return t.repeat_interleave(k, dim=dim)


def adapt_D(D, k, Pp):
    """D (H,) or (H, P) for the split problem: (k * H,) or (k * H, Pp // k)."""
    if D is None:
        return None
    if D.dim() == 1:
        return repeat_heads(D, 0, k)
    return split_heads(pad_last(D, Pp), 0, k)


def gate(out_x, z):
    """out_x * silu(z), silu evaluated in z's dtype (the kernels' gate:
    reference ops/ssd_naive.py:316)."""
    return out_x * F.silu(z).to(out_x.dtype)

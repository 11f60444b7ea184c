"""rms_norm_gated on MI355X: the grouped, SiLU-gated RMSNorm after the SSD as
one HIP kernel in libm2ssd.so (m2_rms_norm_gated).

Drop-in for reference ops/rms_norm.py:15-92: same name, arguments, defaults,
result dtype and rounding points (an intermediate is bf16 exactly when all
its operands are).  x and z may be views whose rows are evenly strided with a
contiguous last dimension (z as a slice of the in-projection output) -- they
are read in place.
"""

from __future__ import annotations

import torch

from .. import _lib as L


def _rows(t, hidden):
    """t (..., hidden) as a (rows, hidden) view with unit last stride, or a copy."""
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    if t.stride(-1) != 1:
        t = t.contiguous()
    try:
        r = t.view(-1, hidden)
    except RuntimeError:
        r = t.reshape(-1, hidden).contiguous()
    if r.shape[0] > 1 and r.stride(0) < hidden:
        r = r.contiguous()
    return r


def _bf(*ts):
    return all(t is None or t.dtype == torch.bfloat16 for t in ts)


def rms_norm_gated(x, weight, z=None, eps=1e-5, group_size=None, norm_before_gate=True, *,
                   out_dtype=None, residual=None):
    """-> out, same shape as x.

    x (..., hidden); weight (hidden,); z (..., hidden) or None.
    z and not norm_before_gate: out = RMSNorm(x * silu(z)) * weight;
    z and norm_before_gate:     out = RMSNorm(x) * weight * silu(z);
    RMS over groups of group_size trailing elements (None: all of hidden).
    out_dtype (keyword only, not in the reference): torch.bfloat16 stores the
    float32 result rounded to bf16 (for a bf16 consumer; no separate cast).
    residual (keyword only, not in the reference; z must be None): a float32
    tensor shaped like x, updated in place to residual + x, whose RMSNorm is
    returned -- a pre-norm block's residual add fused into its norm.
    """
    dev = L.device_of(x, weight, z)
    hidden = int(x.shape[-1])
    gs = hidden if group_size is None else int(group_size)
    L.require(gs > 0 and hidden % gs == 0,
              f"hidden size {hidden} is not a multiple of group_size {gs}")
    L.require(tuple(weight.shape) == (hidden,), f"weight.shape={tuple(weight.shape)}")
    if z is not None:
        L.require(tuple(z.shape) == tuple(x.shape), f"z.shape={tuple(z.shape)} != x.shape")
    xr = _rows(x, hidden)
    zr = None if z is None else _rows(z, hidden)
    w = L.dev_contig(weight if weight.dtype in (torch.float32, torch.bfloat16) else weight.float())
    rows = int(xr.shape[0])
    gate_first = z is not None and not norm_before_gate
    gate_after = z is not None and norm_before_gate
    rr = None
    if residual is not None:
        L.require(z is None, "residual needs z=None")
        L.require(residual.dtype == torch.float32 and tuple(residual.shape) == tuple(x.shape)
                  and residual.is_contiguous() and residual.data_ptr() % 16 == 0,
                  "residual must be a contiguous, 16-byte aligned float32 tensor shaped like x")
        rr = residual.view(-1, hidden)
    # the sum with a float32 residual is float32
    xdt_bf = _bf(xr, zr if gate_first else None) and rr is None
    odt = torch.bfloat16 if xdt_bf and _bf(w, zr if gate_after else None) else torch.float32
    if out_dtype is not None:
        L.require(out_dtype in (odt, torch.bfloat16), f"out_dtype {out_dtype}: the result dtype or bfloat16")
        odt = out_dtype
    out = torch.empty(tuple(x.shape), dtype=odt, device=dev)
    if rows == 0:
        return out
    args = L.RmsNormGatedArgs(
        x=L.ptr(xr), z=L.ptr(zr), weight=L.ptr(w), out=L.ptr(out),
        x_row_stride=xr.stride(0) if rows > 1 else hidden,
        z_row_stride=(zr.stride(0) if rows > 1 else hidden) if zr is not None else 0,
        out_row_stride=hidden, rows=rows, hidden=hidden, group_size=gs, eps=float(eps),
        x_dtype=L.dtype_code(xr, "x"), z_dtype=L.M2_F32 if zr is None else L.dtype_code(zr, "z"),
        w_dtype=L.dtype_code(w, "weight"), out_dtype=L.dtype_code(out, "out"),
        norm_before_gate=int(bool(norm_before_gate)), residual=L.ptr(rr), residual_row_stride=hidden)
    with torch.cuda.device(dev):
        L.call("m2_rms_norm_gated", args, L.stream_of(dev))
    return out


__all__ = ["rms_norm_gated"]

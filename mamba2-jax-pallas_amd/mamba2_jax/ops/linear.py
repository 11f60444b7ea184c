"""Decode-step projections on MI355X: y = x @ w.T (+ bias) for a small batch
(M <= 64 rows) and bf16 weights, as the HIP skinny GEMM in libm2ssd.so
(m2_skinny_gemm).  Not a reference operator: the reference's projections are
XLA GEMMs (modules/mamba2.py:464-469, :538-541; models/mamba2_lm.py:699, :734);
at decode they are bound by reading the weights once per token, which this
kernel does at the HBM rate where hipBLASLt's small-M GEMMs do not.
"""

from __future__ import annotations

import torch

from .. import _lib as L

MAX_ROWS = 64
# rows up to which the decode path uses the skinny kernel (measured on MI355X
# in the 2.7b-shape decode graph at batch 1: in-projection 22 -> 15.9 us,
# out-projection 17 -> 10.5 us per layer; at 64 rows hipBLASLt's tiles are
# faster)
PREFERRED_ROWS = 16


def supported(x, w, max_rows=MAX_ROWS):
    """True when linear_skinny can take these operands."""
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.dim() == 2
            and 1 <= x.shape[0] <= max_rows and w.dim() == 2 and w.shape[1] == x.shape[1]
            and x.shape[1] % 8 == 0 and x.is_cuda and w.is_cuda)


def preferred(x, w):
    """True when the decode path should use linear_skinny for these operands."""
    return supported(x, w, PREFERRED_ROWS)


def preferred_rows(rows, K, w):
    """preferred() for bf16 activations of shape (rows, K) not yet computed:
    lets a caller decide before it rounds them to bf16."""
    return (w.dtype == torch.bfloat16 and w.dim() == 2 and w.shape[1] == K and K % 8 == 0
            and 1 <= rows <= PREFERRED_ROWS and w.is_cuda)


def linear_skinny(x, w, bias=None, out_dtype=torch.bfloat16):
    """x (M, K) bf16, w (N, K) bf16 (the [out, in] layout), bias (N,) -> y (M, N)."""
    dev = L.device_of(x, w, bias)
    L.require(supported(x, w), f"linear_skinny: x {tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} "
                               f"{w.dtype}: need bf16, 1 <= M <= {MAX_ROWS}, K % 8 == 0")
    M, K = x.shape
    N = w.shape[0]
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    w = L.dev_contig(w)
    b = None if bias is None else L.dev_contig(bias if bias.dtype in (torch.float32, torch.bfloat16)
                                               else bias.float())
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    args = L.SkinnyGemmArgs(x=L.ptr(x), w=L.ptr(w), bias=L.ptr(b), y=L.ptr(y), M=M, N=N, K=K,
                            ldx=x.stride(0), ldw=K, ldy=N, x_dtype=L.M2_BF16, w_dtype=L.M2_BF16,
                            bias_dtype=L.M2_F32 if b is None else L.dtype_code(b, "bias"),
                            y_dtype=L.dtype_code(y, "y"))
    with torch.cuda.device(dev):
        L.call("m2_skinny_gemm", args, L.stream_of(dev))
    return y


NORM_MAX_ROWS = 16
# rows up to which the decode layer prefers the normalising projections: each
# workgroup normalises every row itself, one row after another, so the
# prologue's latency grows with the rows (measured on MI355X, 130m shapes:
# 1 row 4.7 us fused vs 6.7 us norm + skinny GEMM; 4 rows 9.1 vs 7.4 us)
NORM_PREFERRED_ROWS = 2
NORM_MAX_ELEMS = 32768      # M * K normalised elements held in LDS
NORM_MAX_GROUPS = 8


def _rows4(t):
    """t (M, K) as rows with unit last stride, 4-element row stride and a
    16-byte aligned base (views such as a slice of the in-projection output
    qualify), or None."""
    if t.stride(1) != 1 or (t.shape[0] > 1 and t.stride(0) % 4) or t.data_ptr() % 16:
        return None
    return t


def norm_supported(x, w, z=None, group_size=None):
    """True when linear_norm can take these operands."""
    if not (w.dtype == torch.bfloat16 and x.dim() == 2 and w.dim() == 2 and x.is_cuda and w.is_cuda):
        return False
    M, K = x.shape
    gs = K if group_size is None else int(group_size)
    return (1 <= M <= NORM_MAX_ROWS and M * K <= NORM_MAX_ELEMS and w.shape[1] == K and K % 8 == 0
            and gs % 4 == 0 and K % gs == 0 and K // gs <= NORM_MAX_GROUPS
            and x.dtype in (torch.float32, torch.bfloat16) and _rows4(x) is not None
            and (z is None or (tuple(z.shape) == (M, K) and z.dtype in (torch.float32, torch.bfloat16)
                               and _rows4(z) is not None)))


def linear_norm(x, norm_weight, w, z=None, group_size=None, eps=1e-5, norm_before_gate=True,
                bias=None, out_dtype=torch.bfloat16, residual=None, store=True, conv_update=None):
    """y = rms_norm_gated(x, norm_weight, z, eps, group_size, norm_before_gate)
    @ w.T (+ bias) in one kernel (m2_skinny_gemm_norm): x (M <= 16, M * K <= 32768), w (N, K)
    bf16.  The normalised rows are bf16, as rms_norm_gated(..., out_dtype=
    torch.bfloat16) gives them.  residual (M, N) float32: the result (rounded
    to out_dtype) is added into it in place; with store=False y is not
    written and None is returned.  conv_update = (args, begin): the decode
    conv update (ops.causal_conv1d.update_from_columns) of output columns
    [begin, begin + args.dim), run on them in the epilogue (width 4, float32
    state in place); those columns of y are then not written."""
    dev = L.device_of(x, norm_weight, w, z, bias, residual)
    L.require(norm_supported(x, w, z, group_size),
              f"linear_norm: x {tuple(x.shape)} {x.dtype}, w {tuple(w.shape)} {w.dtype}: need M <= "
              f"{NORM_MAX_ROWS}, M * K <= {NORM_MAX_ELEMS}, bf16 w, 4-element aligned rows")
    M, K = x.shape
    N = w.shape[0]
    gs = K if group_size is None else int(group_size)
    nw = L.dev_contig(norm_weight if norm_weight.dtype in (torch.float32, torch.bfloat16)
                      else norm_weight.float())
    w = L.dev_contig(w)
    b = None if bias is None else L.dev_contig(bias if bias.dtype in (torch.float32, torch.bfloat16)
                                               else bias.float())
    if residual is not None:
        L.require(residual.dtype == torch.float32 and tuple(residual.shape) == (M, N)
                  and residual.stride(1) == 1, "residual must be float32 (M, N) with unit last stride")
    L.require(store or residual is not None, "linear_norm: nothing to write")
    L.require(out_dtype in (torch.float32, torch.bfloat16), f"out_dtype {out_dtype}")
    y = torch.empty((M, N), dtype=out_dtype, device=dev) if store else None
    args = L.SkinnyGemmNormArgs(
        x=L.ptr(x), z=L.ptr(z), norm_weight=L.ptr(nw),
        x_row_stride=x.stride(0) if M > 1 else K,
        z_row_stride=(z.stride(0) if M > 1 else K) if z is not None else 0, group_size=gs,
        eps=float(eps), x_dtype=L.dtype_code(x, "x"),
        z_dtype=L.M2_F32 if z is None else L.dtype_code(z, "z"),
        norm_weight_dtype=L.dtype_code(nw, "norm_weight"), norm_before_gate=int(bool(norm_before_gate)),
        w=L.ptr(w), bias=L.ptr(b), y=L.ptr(y), residual=L.ptr(residual), M=M, N=N, K=K, ldw=K,
        ldy=N, residual_row_stride=0 if residual is None else (residual.stride(0) if M > 1 else N),
        w_dtype=L.M2_BF16, bias_dtype=L.M2_F32 if b is None else L.dtype_code(b, "bias"),
        y_dtype=L.M2_BF16 if out_dtype == torch.bfloat16 else L.M2_F32)
    if conv_update is not None:
        cargs, begin = conv_update
        L.require(int(cargs.batch) == M and 0 <= begin and begin + int(cargs.dim) <= N,
                  "conv_update: batch M and columns inside N")
        args.with_conv, args.conv_begin, args.conv = 1, int(begin), cargs
    with torch.cuda.device(dev):
        L.call("m2_skinny_gemm_norm", args, L.stream_of(dev))
    return y


__all__ = ["linear_norm", "linear_skinny", "norm_supported", "supported"]

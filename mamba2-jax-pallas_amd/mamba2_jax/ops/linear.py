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


__all__ = ["linear_skinny", "supported"]

"""The decode projections' skinny GEMM (m2_skinny_gemm) against a float32
torch product of the same bf16 operands: y = x w^T (+ bias) for M <= 64.
Tolerance: 1e-5 of the output RMS for f32 outputs (float32 accumulation in
another order), one bf16 ulp of each value plus 1e-5 of the RMS for bf16."""

import numpy as np
import pytest
import torch

from gpu_util import announce
from mamba2_jax import _lib as L
from mamba2_jax.ops.linear import linear_skinny

pytestmark = pytest.mark.gpu

CASES = [(1, 768, 3352), (1, 2560, 10576), (4, 5120, 2560), (16, 40, 17), (17, 64, 33),
         (33, 136, 1000), (64, 2560, 1024), (5, 8, 1), (64, 768, 50288)]


@pytest.mark.parametrize("M,K,N", CASES)
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_skinny_gemm(M, K, N, out):
    announce("skinny_gemm", M, K, N, out)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + K + N)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") / K ** 0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g, device="cuda") if N % 2 else None
    odt = torch.float32 if out == "f32" else torch.bfloat16
    y = linear_skinny(x, w, b, out_dtype=odt)
    ref = x.float() @ w.float().t() + (0 if b is None else b)
    rms = ref.pow(2).mean().sqrt().item()
    err = (y.float() - ref).abs()
    tol = 1e-5 * rms + (2.0 ** -8 * ref.abs() if odt == torch.bfloat16 else 0)
    print(f"  max err {err.max().item():.3e}, rms {rms:.3e}", flush=True)
    assert bool((err <= tol).all()), f"{int((err > tol).sum())} values beyond tolerance"


def test_strided_x_and_errors():
    g = torch.Generator(device="cuda").manual_seed(1)
    xx = torch.randn((8, 1024), generator=g, device="cuda").to(torch.bfloat16)
    x = xx[:, 256:256 + 512]                       # row stride 1024
    w = torch.randn((96, 512), generator=g, device="cuda").to(torch.bfloat16)
    y = linear_skinny(x, w, out_dtype=torch.float32)
    torch.testing.assert_close(y, x.float() @ w.float().t(), rtol=1e-5, atol=1e-4)
    with pytest.raises(AssertionError):
        linear_skinny(torch.zeros((65, 64), device="cuda", dtype=torch.bfloat16), w[:, :64])
    with pytest.raises(AssertionError):
        linear_skinny(torch.zeros((2, 12), device="cuda", dtype=torch.bfloat16),
                      torch.zeros((3, 12), device="cuda", dtype=torch.bfloat16))
    a = L.SkinnyGemmArgs(x=x.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), M=8, N=96, K=512, ldx=1024,
                         ldw=512, ldy=96, x_dtype=L.M2_F32, w_dtype=L.M2_BF16, y_dtype=L.M2_F32)
    with pytest.raises(L.M2Error):
        L.call("m2_skinny_gemm", a, 0)

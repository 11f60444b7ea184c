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


# ---------------------------------------------------------------------------
# m2_skinny_gemm_norm: the rows normalised in the GEMM's prologue
# ---------------------------------------------------------------------------

from mamba2_jax.ops.linear import linear_norm  # noqa: E402
from mamba2_jax.ops.rms_norm import rms_norm_gated  # noqa: E402

NORM_CASES = [
    # M, K, N, x dtype, gated (z slice), group_size, norm_before_gate, bias
    (1, 2560, 10576, "f32", False, None, True, False),     # 2.7b pre-norm + in-projection
    (4, 768, 3352, "f32", False, None, True, True),
    (1, 5120, 2560, "f32", True, None, False, False),      # 2.7b gated norm + out-projection
    (3, 8192, 4096, "f32", True, 1024, False, False),      # nemotron-h-8b: 8 groups
    (2, 1536, 768, "bf16", True, 768, True, True),
    (4, 64, 40, "bf16", False, 16, True, False),
    (16, 768, 3352, "f32", False, None, True, False),     # 130m pre-norm, batch 16
    (11, 1536, 768, "f32", True, 768, False, True),       # 130m-like gated norm, 2 groups
    (2, 1536, 768, "bf16", True, None, True, True),       # one group, bf16 rows, gate after
    (1, 5120, 2560, "f32", True, None, True, False),      # one group, gate after the norm
]


@pytest.mark.parametrize("case", NORM_CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}-{c[3]}-z{int(c[4])}-g{c[5]}"
                                                   f"-nbg{int(c[6])}-b{int(c[7])}" for c in NORM_CASES])
def test_skinny_gemm_norm(case):
    """against the two-kernel composition it replaces (rms_norm_gated storing
    bf16, then the skinny GEMM): the normalised rows may differ by one bf16 ulp
    where the two kernels' sums of squares round differently, so the bound is
    2^-7 of each product's magnitude sum |x'| |w| plus 1e-5 of the RMS;
    with a residual, residual_after == residual_before + y exactly."""
    M, K, N, xdt, gated, gs, nbg, hasb = case
    announce("skinny_gemm_norm", case)
    g = torch.Generator(device="cuda").manual_seed(M + K + N)
    T = {"f32": torch.float32, "bf16": torch.bfloat16}[xdt]
    x = (torch.randn((M, K), generator=g, device="cuda") * 3).to(T)
    z = None
    if gated:
        wide = torch.randn((M, K + 2 * K + 16), generator=g, device="cuda").to(torch.bfloat16)
        z = wide[:, 8:8 + K]                                  # a strided slice, as in the layer
    nw = torch.rand(K, generator=g, device="cuda").add(0.5).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") / K ** 0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g, device="cuda").to(torch.bfloat16) if hasb else None
    res = torch.randn((M, N), generator=g, device="cuda")
    res0 = res.clone()
    y = linear_norm(x, nw, w, z=z, group_size=gs, norm_before_gate=nbg, bias=b, residual=res)
    xn = rms_norm_gated(x, nw, z=z, group_size=gs, norm_before_gate=nbg, out_dtype=torch.bfloat16)
    ref = xn.float() @ w.float().t() + (0 if b is None else b.float())
    mag = xn.float().abs() @ w.float().abs().t()
    err = (y.float() - ref).abs()
    rms = ref.pow(2).mean().sqrt().item()
    tol = 2.0 ** -7 * mag + 2.0 ** -8 * ref.abs() + 1e-5 * rms
    print(f"  max err {err.max().item():.3e}, rms {rms:.3e}", flush=True)
    assert bool((err <= tol).all()), f"{int((err > tol).sum())} values beyond tolerance"
    assert torch.equal(res, res0 + y.float()), "residual += y"
    # residual only (no y): the same sums
    res2 = res0.clone()
    assert linear_norm(x, nw, w, z=z, group_size=gs, norm_before_gate=nbg, bias=b, residual=res2,
                       store=False) is None
    assert torch.equal(res2, res)


def test_skinny_gemm_norm_limits():
    w = torch.zeros((16, 64), device="cuda", dtype=torch.bfloat16)
    nw = torch.ones(64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(AssertionError):                    # 17 rows
        linear_norm(torch.zeros((17, 64), device="cuda"), nw, w)
    with pytest.raises(AssertionError):                    # 16 groups
        linear_norm(torch.zeros((1, 64), device="cuda"), nw, w, group_size=4)
    a = L.SkinnyGemmNormArgs(x=w.data_ptr(), norm_weight=nw.data_ptr(), w=w.data_ptr(), y=0,
                             residual=0, M=1, N=16, K=64, ldw=64, ldy=16, group_size=64,
                             x_dtype=L.M2_BF16, norm_weight_dtype=L.M2_BF16, w_dtype=L.M2_BF16,
                             y_dtype=L.M2_BF16)
    with pytest.raises(L.M2Error):                          # neither y nor residual
        L.call("m2_skinny_gemm_norm", a, 0)


@pytest.mark.parametrize("M,bias", [(1, True), (4, False)])
def test_skinny_gemm_norm_conv_epilogue(M, bias):
    """The decode conv update run in the in-projection's epilogue equals the
    projection followed by causal_conv1d_update (same rounding of the new
    inputs, same conv arithmetic): outputs and the in-place state bit for bit."""
    from mamba2_jax.ops.causal_conv1d import causal_conv1d_update, update_from_columns
    announce("skinny_gemm_norm + conv update", M, bias)
    g = torch.Generator(device="cuda").manual_seed(M + 100)
    K, d_ssm, GN, H = 768, 1536, 128, 24
    conv_dim, N = d_ssm + 2 * GN, 2 * d_ssm + 2 * GN + H
    x = torch.randn((M, K), generator=g, device="cuda")
    nw = torch.rand(K, generator=g, device="cuda").add(0.5).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") / K ** 0.5).to(torch.bfloat16)
    cw = (torch.randn((conv_dim, 4), generator=g, device="cuda") * 0.5).to(torch.bfloat16)
    cb = torch.randn(conv_dim, generator=g, device="cuda").to(torch.bfloat16) if bias else None
    st0 = torch.randn((M, conv_dim, 4), generator=g, device="cuda")
    st_a, st_b = st0.clone(), st0.clone()
    split = (d_ssm, GN, GN)
    y = linear_norm(x, nw, w)
    st_b, want = causal_conv1d_update(y[:, d_ssm:d_ssm + conv_dim], st_b, cw, cb, "silu", split_sizes=split)
    cargs, got = update_from_columns(st_a, cw, cb, "silu", split_sizes=split)
    y2 = linear_norm(x, nw, w, conv_update=(cargs, d_ssm))
    for a_, b_ in zip(got, want):
        assert torch.equal(a_, b_)
    assert torch.equal(st_a, st_b)
    assert torch.equal(y2[:, :d_ssm], y[:, :d_ssm]) and torch.equal(y2[:, -H:], y[:, -H:])

"""Parity of rms_norm_gated (HIP) with the CPU oracle.

* the reference tests' cases (tests/test_mamba2_ops.py:205-296);
* the Mamba2 layer's use: the SSD output y (f32) normalised per group of
  d_ssm / ngroups with z a bf16 slice of the in-projection output, gate
  before the norm (nemotron-h-8b layer shape);
* bf16 inputs (every intermediate rounded as the reference's bf16 arrays),
  both gate orders, z in f32, sizes that are not multiples of 4, groups
  longer than the register-resident size, leading dims of any rank.
Tolerance: f32 results 1e-5 relative to the output RMS; bf16 results 2^-6 of
each value (a one-ulp difference of the bf16 rms moves a whole group by 2^-8
before the final rounding).
"""

import numpy as np
import pytest
import torch

from gpu_util import announce, dev, host
from mamba2_jax.ops.rms_norm import rms_norm_gated
from oracle import ops_oracle as X
from oracle.ssd_oracle import bf16_round

pytestmark = pytest.mark.gpu

NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16"}
T = {"bf16": torch.bfloat16, "f32": torch.float32}


def _close(got, want, is_bf16, what):
    g = host(got)
    assert g.shape == want.shape, (g.shape, want.shape)
    if is_bf16:
        bad = np.abs(g - want) > 2.0 ** -6 * np.abs(want) + 1e-30
        print(f"  {what}: beyond 2^-6: {int(bad.sum())} of {g.size}", flush=True)
        assert not bad.any(), f"{what}: {int(bad.sum())} values"
    else:
        e = np.max(np.abs(g - want)) / max(np.sqrt(np.mean(want ** 2)), 1e-30)
        print(f"  {what}: max|err|/rms = {e:.2e}", flush=True)
        assert e <= 1e-5, f"{what}: {e:.2e}"


def _rnd(a, t):
    return None if a is None else (bf16_round(a) if t == torch.bfloat16 else a.astype(np.float32))


def test_reference_cases():
    """reference tests/test_mamba2_ops.py:205-296 (fp32)."""
    rng = np.random.default_rng(42)
    announce("rms_norm_gated reference cases")
    x = rng.standard_normal((2, 8, 16)).astype(np.float32)
    want, _ = X.rms_norm_gated(x, np.ones(16))
    _close(rms_norm_gated(dev(x), dev(np.ones(16, np.float32))), want, False, "basic")
    x, z, w = (rng.standard_normal(s).astype(np.float32) for s in ((2, 16), (2, 16), (16,)))
    for nbg in (True, False):
        want, _ = X.rms_norm_gated(x, w, z=z, norm_before_gate=nbg)
        _close(rms_norm_gated(dev(x), dev(w), z=dev(z), norm_before_gate=nbg), want, False,
               f"gated, norm_before_gate={nbg}")
    x = rng.standard_normal((2, 32)).astype(np.float32)
    want, _ = X.rms_norm_gated(x, np.ones(32), group_size=8)
    _close(rms_norm_gated(dev(x), dev(np.ones(32, np.float32)), group_size=8), want, False, "grouped")


def test_layer_shape_slice_of_in_projection():
    """nemotron-h-8b: y (1, 4096, 8192) f32, z a bf16 slice of the in-projection
    output (1, 4096, d_in_proj), groups of 1024, gate before the norm."""
    announce("rms_norm_gated, nemotron-h-8b layer")
    rng = np.random.default_rng(7)
    Lq, dssm, dproj, off = 4096, 8192, 8192 * 2 + 2048 + 128, 8192
    y = rng.standard_normal((1, Lq, dssm)).astype(np.float32)
    zx = bf16_round(rng.standard_normal((1, Lq, dproj)).astype(np.float32))
    w = rng.uniform(0.5, 1.5, dssm).astype(np.float32)
    zt = dev(zx, torch.bfloat16)[:, :, off:off + dssm]
    assert not zt.is_contiguous()
    got = rms_norm_gated(dev(y), dev(w), z=zt, group_size=1024, norm_before_gate=False)
    want, dt = X.rms_norm_gated(y, w, z=zx[:, :, off:off + dssm], group_size=1024,
                                norm_before_gate=False, z_dtype="bfloat16")
    assert dt == "float32" and got.dtype == torch.float32
    _close(got, want, False, "f32 y, bf16 z slice")


CASES = [
    # shape, group, dtypes (x, z, w), z, norm_before_gate
    ((3, 64), None, ("bf16", "bf16", "bf16"), True, True),
    ((3, 64), None, ("bf16", "bf16", "bf16"), True, False),
    ((2, 5, 96), 32, ("bf16", "bf16", "f32"), True, False),
    ((4, 256), 64, ("f32", "f32", "f32"), True, True),
    ((4, 256), 64, ("bf16", "f32", "bf16"), True, False),
    ((7, 30), 10, ("f32", "bf16", "f32"), True, False),      # 10 % 4: scalar chunks
    ((3, 30), 15, ("bf16", "bf16", "bf16"), True, True),
    ((2, 12288), None, ("f32", "bf16", "f32"), True, False),  # beyond the resident size
    ((2, 12288), 4096, ("bf16", None, "bf16"), False, True),
    ((2, 3, 4, 40), 20, ("f32", None, "f32"), False, False),
    ((5, 2048), 512, ("bf16", "bf16", "bf16"), True, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-g{c[1]}-{'/'.join(str(d) for d in c[2])}"
                                              f"-z{int(c[3])}-nbg{int(c[4])}" for c in CASES])
def test_norm_cases(case):
    shape, gs, dts, with_z, nbg = case
    announce("rms_norm_gated", case)
    rng = np.random.default_rng(sum(shape) + (gs or 0))
    xdt, zdt, wdt = (None if d is None else T[d] for d in dts)
    hidden = shape[-1]
    x = _rnd(rng.standard_normal(shape) * 2.0, xdt)
    z = _rnd(rng.standard_normal(shape), zdt) if with_z else None
    w = _rnd(rng.uniform(0.5, 1.5, hidden), wdt)
    want, rdt = X.rms_norm_gated(x, w, z=z, group_size=gs, norm_before_gate=nbg,
                                 x_dtype=NAME[xdt], w_dtype=NAME[wdt],
                                 z_dtype=NAME[zdt] if zdt is not None else "float32")
    got = rms_norm_gated(dev(x, xdt), dev(w, wdt), z=None if z is None else dev(z, zdt),
                         group_size=gs, norm_before_gate=nbg)
    assert NAME[got.dtype] == rdt and tuple(got.shape) == shape
    _close(got, want, rdt == "bfloat16", str(case))


def test_errors():
    x = torch.zeros((2, 12), device="cuda")
    with pytest.raises(AssertionError):
        rms_norm_gated(x, torch.ones(12, device="cuda"), group_size=5)
    with pytest.raises(AssertionError):
        rms_norm_gated(x, torch.ones(10, device="cuda"))
    with pytest.raises(ValueError):
        rms_norm_gated(x.cpu(), torch.ones(12))


@pytest.mark.parametrize("hidden,xdt", [(2560, "bf16"), (12288, "bf16"), (768, "f32"), (30, "bf16")])
def test_residual_add_fused(hidden, xdt):
    """residual (f32, in place) += x, then the RMSNorm of the sum: the
    reference's pre-norm block (models/mamba2_lm.py:205-211) in one kernel;
    12288 runs the two-pass path (the second pass must not add again)."""
    announce("rms_norm with residual", hidden, xdt)
    rng = np.random.default_rng(hidden)
    x = _rnd(rng.standard_normal((3, hidden)), T[xdt])
    res = rng.standard_normal((3, hidden)).astype(np.float32)
    w = _rnd(rng.uniform(0.5, 1.5, hidden), torch.bfloat16)
    rt = dev(res)
    got = rms_norm_gated(dev(x, T[xdt]), dev(w, torch.bfloat16), residual=rt, out_dtype=torch.bfloat16)
    summed = res.astype(np.float64) + x
    assert np.array_equal(host(rt), (res + x.astype(np.float32)).astype(np.float64)), "residual += x in f32"
    want, _ = X.rms_norm_gated(summed.astype(np.float32), w, w_dtype="bfloat16")
    _close(got, bf16_round(want), True, "add + norm, bf16 store")


def _sweep_cases(n=20, seed=92):
    """Cases of test_norm_cases' form drawn once from a fixed seed: 1-3 leading
    dims, 1-8 groups of 1-1500 elements (or one group), mixed dtypes, z on and
    off, the norm before or after the gate."""
    rng = np.random.default_rng(seed)
    tys = ("bf16", "f32")
    out = []
    for _ in range(n):
        gs = int(rng.integers(1, 1501))
        ng = int(rng.integers(1, 9))
        lead = tuple(int(v) for v in rng.integers(1, 5, int(rng.integers(1, 3))))
        with_z = bool(rng.random() < 0.7)
        out.append((lead + (gs * ng,), gs if rng.random() < 0.7 else None,
                    (str(rng.choice(tys)), str(rng.choice(tys)) if with_z else None, str(rng.choice(tys))),
                    with_z, bool(rng.random() < 0.5)))
    return out


@pytest.mark.parametrize("case", _sweep_cases())
def test_norm_sweep(case):
    test_norm_cases(case)

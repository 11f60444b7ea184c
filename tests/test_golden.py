"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture.  GPU: the HIP path matches the
fixtures to the parity bar (max|err|/rms <= 1e-3 fp32, 2e-2 bf16).
"""

import os

import numpy as np
import pytest
import torch

from oracle import ssd_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SSD = ["ssd_f32_basic", "ssd_bf16_groups", "ssd_bf16_varlen"]
INPUTS = ("x", "dt", "A", "B", "C", "D", "z", "dt_bias", "initial_states", "seq_idx", "cu_seqlens")


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", SSD)
def test_oracle_reproduces_fixture(name):
    g = load(name)
    kw = {k: g[k] for k in INPUTS if k in g}
    varlen = "want_varlen" in g
    res = O.ssd_combined(chunk_size=int(g["chunk_size"]), dt_softplus=True,
                         return_final_states=True, return_varlen_states=varlen,
                         io_dtype=str(g["io_dtype"]), **kw)
    np.testing.assert_allclose(res[0], g["want_out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(res[1], g["want_final"], rtol=1e-12, atol=1e-12)
    if varlen:
        np.testing.assert_allclose(res[2], g["want_varlen"], rtol=1e-12, atol=1e-12)


def test_oracle_reproduces_ssu_fixture():
    g = load("ssu_bf16_step")
    kw = {k: g[k] for k in ("state", "x", "dt", "A", "B", "C", "D", "z", "dt_bias")}
    new, y = O.selective_state_update(**kw, dt_softplus=True, round_fn=O.round_fn_for("bf16"))
    np.testing.assert_allclose(new, g["want_state"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y, g["want_out"], rtol=1e-12, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("name", SSD)
def test_hip_matches_fixture(name):
    from mamba2_jax.kernels import mamba_chunk_scan_combined_fwd
    g = load(name)
    io = str(g["io_dtype"])
    T = torch.bfloat16 if io == "bf16" else torch.float32
    t = {}
    for k in INPUTS:
        if k not in g:
            continue
        v = torch.from_numpy(g[k]).cuda()
        t[k] = v.to(T) if k in ("x", "dt", "B", "C", "z") else v
    varlen = "want_varlen" in g
    res = mamba_chunk_scan_combined_fwd(chunk_size=int(g["chunk_size"]), dt_softplus=True,
                                        return_final_states=True, return_varlen_states=varlen, **t)
    tol = 1e-3 if io == "f32" else 2e-2
    wants = ["want_out", "want_final"] + (["want_varlen"] if varlen else [])
    for got, key in zip(res, wants):
        e = O.rel_err(got.float().cpu().numpy(), g[key])
        print(f"  {name} {key}: {e:.3e}")
        assert e <= tol, (key, e)


@pytest.mark.gpu
def test_hip_matches_ssu_fixture():
    from mamba2_jax.ops import selective_state_update
    g = load("ssu_bf16_step")
    t = {k: torch.from_numpy(g[k]).cuda() for k in ("state", "x", "dt", "A", "B", "C", "D", "z",
                                                     "dt_bias")}
    for k in ("x", "B", "C", "z"):
        t[k] = t[k].to(torch.bfloat16)
    new, y = selective_state_update(**t, dt_softplus=True)
    assert O.rel_err(new.cpu().numpy(), g["want_state"]) <= 1e-5
    assert O.rel_err(y.cpu().numpy(), g["want_out"]) <= 1e-4

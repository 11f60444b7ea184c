"""Parity of the decode step (selective_state_update) on the GPU.

* one step against the oracle's closed form at the c4 shape and with every
  parameter-shape variant the reference supports;
* 256 consecutive in-place steps against the oracle's float64 trajectory and
  against the HIP prefill over the same tokens (decode == prefill), and the
  full c4 (batch 64, 256 steps) against the oracle one head group at a time;
* functional (default) / in-place semantics, and the reference's own usage
  pattern (expected values computed from the state after the call).
"""

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, host
from mamba2_jax import configs
from mamba2_jax.kernels import mamba_chunk_scan_combined_fwd
from mamba2_jax.ops import selective_state_update
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu


def _step_inputs(rng, b, H, G, P, N, dt_hdim=False, A_full=False, D_hdim=False,
                 bias_hdim=False, with_D=True, with_z=True):
    bf = lambda a: configs.round_to(a.astype(np.float32), "bf16")
    return dict(
        state=(0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32),
        x=bf(rng.standard_normal((b, H, P))),
        dt=rng.standard_normal((b, H, P) if dt_hdim else (b, H)).astype(np.float32),
        A=(-np.exp(rng.uniform(0, np.log(16), (H, P, N) if A_full else H))).astype(np.float32),
        B=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        C=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        D=rng.uniform(0.5, 1.5, (H, P) if D_hdim else H).astype(np.float32) if with_D else None,
        z=bf(rng.standard_normal((b, H, P))) if with_z else None,
        dt_bias=rng.uniform(-4, -2, (H, P) if bias_hdim else H).astype(np.float32),
    )


def _dev(d):
    bfk = ("x", "B", "C", "z")
    return {k: dev(v, torch.bfloat16 if k in bfk else None) for k, v in d.items()}


@pytest.mark.parametrize("b,H,G,P,N,kw", [
    (64, 128, 8, 64, 128, {}),                                  # c4 shape
    (4, 16, 1, 64, 64, dict(dt_hdim=True, bias_hdim=True)),
    (4, 16, 4, 32, 128, dict(A_full=True, D_hdim=True)),
    (2, 8, 2, 128, 256, dict(with_z=False)),
    (3, 6, 3, 64, 32, dict(with_D=False, with_z=False)),
])
@pytest.mark.parametrize("softplus", [True, False])
def test_single_step(b, H, G, P, N, kw, softplus):
    announce("ssu step", b, H, G, P, N, kw, softplus)
    rng = np.random.default_rng(b + H + P + N)
    d = _step_inputs(rng, b, H, G, P, N, **kw)
    if not softplus:
        d["dt"] = np.abs(d["dt"]) * 0.05
        d["dt_bias"] = None
    t = _dev(d)
    new, y = selective_state_update(**t, dt_softplus=softplus)
    ws, wy = O.selective_state_update(**d, dt_softplus=softplus, round_fn=O.round_fn_for("bf16"))
    check(new, ws, 1e-5, "state")
    check(y, wy, 1e-4, "out")


def test_256_steps_trajectory_and_prefill():
    """c4 recurrence (b reduced to 2): 256 in-place steps == the oracle's float64
    trajectory, and == the SSD prefill over the same 256 tokens."""
    cfg = configs.DecodeConfig("c4-small", 2, 128, 8, 64, 128, 256)
    announce("ssu 256 steps", cfg)
    d = configs.make_decode_inputs(cfg)
    state = dev(d["state"])
    s0 = state.clone()
    ys = []
    ref = d["state"].astype(np.float64)
    wys = []
    for t in range(cfg.steps):
        z = dev(d["z"][t], torch.bfloat16)
        new, y = selective_state_update(state, dev(d["x"][t], torch.bfloat16), dev(d["dt"][t]),
                                        dev(d["A"]), dev(d["B"][t], torch.bfloat16),
                                        dev(d["C"][t], torch.bfloat16), D=dev(d["D"]), z=z,
                                        dt_bias=dev(d["dt_bias"]), dt_softplus=True, inplace=True)
        assert new.data_ptr() == state.data_ptr()
        ys.append(y)
        ref, wy = O.selective_state_update(ref, d["x"][t], d["dt"][t], d["A"], d["B"][t],
                                           d["C"][t], D=d["D"], z=d["z"][t],
                                           dt_bias=d["dt_bias"], dt_softplus=True,
                                           round_fn=O.round_fn_for("bf16"))
        wys.append(wy)
    Y = torch.stack(ys, dim=1)                                 # (b, T, H, P)
    check(state, ref, 1e-4, "state after 256 steps")
    check(Y, np.stack(wys, axis=1), 1e-4, "outputs of 256 steps")
    # prefill of the same tokens (bf16 inputs -> bf16 tolerance for the chunked path)
    tok = lambda a: torch.from_numpy(np.ascontiguousarray(np.swapaxes(a, 0, 1)))
    yp, fp = mamba_chunk_scan_combined_fwd(
        tok(d["x"]).to(torch.bfloat16).cuda(), tok(d["dt"]).cuda(), dev(d["A"]),
        tok(d["B"]).to(torch.bfloat16).cuda(), tok(d["C"]).to(torch.bfloat16).cuda(), 64,
        D=dev(d["D"]), z=tok(d["z"]).to(torch.bfloat16).cuda(), dt_bias=dev(d["dt_bias"]),
        initial_states=s0, dt_softplus=True, return_final_states=True)
    check(Y, host(yp), TOL["bf16"], "decode == prefill (outputs)")
    check(state, host(fp), TOL["bf16"], "decode == prefill (final state)")


@pytest.mark.timeout(600)
def test_full_c4_trajectory_by_group():
    """c4 in full: batch 64, 128 heads, all 256 in-place steps on the GPU.  At
    every step the state and the outputs of one head group (16 heads with their
    B / C, independent of the others) are compared with the oracle's float64
    trajectory for that group."""
    cfg = configs.DECODE
    g = 3
    announce("ssu c4 full, 256 steps, group", g, cfg)
    d = configs.make_decode_inputs(cfg)
    hpg = cfg.nheads // cfg.ngroups
    hs = slice(g * hpg, (g + 1) * hpg)
    state = dev(d["state"])
    ref = d["state"][:, hs].astype(np.float64)
    A, D, bias = dev(d["A"]), dev(d["D"]), dev(d["dt_bias"])
    worst_s = worst_y = 0.0
    for t in range(cfg.steps):
        new, y = selective_state_update(state, dev(d["x"][t], torch.bfloat16), dev(d["dt"][t]), A,
                                        dev(d["B"][t], torch.bfloat16), dev(d["C"][t], torch.bfloat16),
                                        D=D, z=dev(d["z"][t], torch.bfloat16), dt_bias=bias,
                                        dt_softplus=True, inplace=True)
        ref, wy = O.selective_state_update(ref, d["x"][t][:, hs], d["dt"][t][:, hs], d["A"][hs],
                                           d["B"][t][:, g:g + 1], d["C"][t][:, g:g + 1],
                                           D=d["D"][hs], z=d["z"][t][:, hs],
                                           dt_bias=d["dt_bias"][hs], dt_softplus=True,
                                           round_fn=O.round_fn_for("bf16"))
        es = O.rel_err(host(state[:, hs]), ref)
        ey = O.rel_err(host(y[:, hs]), wy)
        worst_s, worst_y = max(worst_s, es), max(worst_y, ey)
        assert es <= 1e-4 and ey <= 1e-4, f"step {t}: state {es:.3e}, out {ey:.3e} (tol 1e-4)"
        if t % 32 == 31:
            print(f"  steps 0-{t}: worst state {worst_s:.3e}, out {worst_y:.3e}", flush=True)
    print(f"  worst over {cfg.steps} steps: state {worst_s:.3e}, out {worst_y:.3e} (tol 1e-4)",
          flush=True)


def test_inplace_and_copy_semantics():
    """Default: the caller's state is untouched and a new tensor comes back;
    inplace=True writes through a float32 contiguous state; a state the kernel
    cannot write through (non-contiguous) is never written, inplace or not."""
    announce("ssu in-place / copy")
    rng = np.random.default_rng(5)
    d = _step_inputs(rng, 2, 8, 2, 64, 128)
    t = _dev(d)
    s_before = t["state"].clone()
    new, _ = selective_state_update(**t, dt_softplus=True)
    assert new.data_ptr() != t["state"].data_ptr()
    assert torch.equal(t["state"], s_before), "the default leaves the state alone"
    new2, _ = selective_state_update(**t, dt_softplus=True, inplace=True)
    assert new2.data_ptr() == t["state"].data_ptr()
    assert torch.equal(new2, new)
    st_nc = s_before.transpose(2, 3).contiguous().transpose(2, 3)
    keep = st_nc.clone()
    new3, _ = selective_state_update(**{**t, "state": st_nc}, dt_softplus=True, inplace=True)
    assert new3.data_ptr() != st_nc.data_ptr() and torch.equal(st_nc, keep)
    assert torch.equal(new3, new)


@pytest.mark.parametrize("with_extras", [False, True])
def test_reference_usage_pattern(with_extras):
    """The reference's own tests (tests/test_mamba2_ops.py:25-103) compute the
    expected state from ``state`` AFTER the call, which only works when the
    call leaves it untouched: same shapes (b 2, H 4, P 8, N 16, G 2 / 1), float32
    inputs, the closed form evaluated in float32 torch on the GPU, the
    reference's bounds (state 1e-5, out 1e-5 / 1e-4)."""
    announce("ssu reference usage pattern", with_extras)
    g = torch.Generator(device="cuda").manual_seed(42 + with_extras)
    r = lambda *s: torch.randn(*s, generator=g, device="cuda")
    b, H, P, N = 2, 4, 8, 16
    G = 1 if with_extras else 2
    state, x = r(b, H, P, N), r(b, H, P)
    A = -r(H).abs()
    Bm, Cm = r(b, G, N), r(b, G, N)
    if with_extras:
        dt, D, z, bias = r(b, H), r(H), r(b, H, P), r(H)
        new, out = selective_state_update(state, x, dt, A, Bm, Cm, D=D, z=z, dt_bias=bias,
                                          dt_softplus=True)
        dtr = torch.nn.functional.softplus(dt + bias)
    else:
        dt = torch.rand(b, H, generator=g, device="cuda") * 0.09 + 0.01
        new, out = selective_state_update(state, x, dt, A, Bm, Cm, dt_softplus=False)
        dtr = dt
    Be, Ce = Bm.repeat_interleave(H // G, dim=1), Cm.repeat_interleave(H // G, dim=1)
    dA = torch.exp(dtr[:, :, None, None] * A[None, :, None, None])
    ref_state = state * dA + dtr[:, :, None, None] * Be[:, :, None, :] * x[:, :, :, None]
    ref_out = (ref_state * Ce[:, :, None, :]).sum(-1)
    if with_extras:
        ref_out = (ref_out + D[None, :, None] * x) * torch.nn.functional.silu(z)
    assert (new - ref_state).abs().max().item() < 1e-5
    assert (out - ref_out).abs().max().item() < (1e-4 if with_extras else 1e-5)


def test_mixed_dt_and_bias_layouts_are_rejected():
    """dt (b, H) with dt_bias (H, P), or dt (b, H, P) with dt_bias (H,): the
    reference adds dt and dt_bias by broadcasting (ops/selective_state_update.py
    :72), which fails for these pairs (or misaligns heads when sizes coincide);
    the drop-in raises."""
    from mamba2_jax._lib import M2ShapeError
    rng = np.random.default_rng(3)
    for dt_hdim, bias_hdim in ((False, True), (True, False)):
        d = _step_inputs(rng, 2, 4, 2, 32, 64, dt_hdim=dt_hdim, bias_hdim=bias_hdim)
        with pytest.raises(M2ShapeError):
            selective_state_update(**_dev(d), dt_softplus=True)

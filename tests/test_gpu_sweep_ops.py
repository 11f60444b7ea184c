"""Seeded sweeps of the reference's stage operators and of the decode step.

Shapes and options are drawn once from fixed seeds (every run checks the same
ones) across what each operator accepts: ragged lengths, batch > 1, head dims
32 / 64 / 128, dstate 32-256, chunk 32-256, bf16 and fp32 inputs, sequence
resets, causal masks, initial states, D / z, the parameter-shape variants of
the decode step.  Each case is compared with the CPU oracle at the bars of
the hand-picked tests (tests/test_gpu_stages.py, tests/test_gpu_ssu.py).
"""

import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, seq_idx_from_lengths, tdtype
from mamba2_jax import configs
from mamba2_jax.kernels import bmm_chunk_fwd, chunk_scan_fwd, chunk_state_fwd, state_passing_fwd
from mamba2_jax.ops import selective_state_update
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu


def _lengths(rng, b, L):
    """Per-row sequence lengths (1-3 sequences per row) summing to L."""
    out = []
    for _ in range(b):
        k = int(rng.integers(1, 4))
        cuts = np.sort(rng.choice(np.arange(1, L), size=min(k - 1, L - 1), replace=False)) if L > 1 else []
        edges = [0, *[int(c) for c in cuts], L]
        out.append([edges[i + 1] - edges[i] for i in range(len(edges) - 1)])
    return out


def _ssd_shape(rng):
    dtype = "bf16" if rng.random() < 0.6 else "f32"
    P = int(rng.choice([32, 64, 64, 128]))
    N = int(rng.choice([64, 128, 256]))
    Q = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([2, 4, 6, 8]))
    G = int(rng.choice([g for g in (1, 2, 4) if H % g == 0]))
    b = int(rng.integers(1, 3))
    L = int(rng.integers(2, 600))
    return b, L, H, G, P, N, Q, dtype


# ---------------------------------------------------------------------------
# chunk_state / chunk_scan
# ---------------------------------------------------------------------------

def _state_cases(n=14, seed=77):
    rng = np.random.default_rng(seed)
    return [(_ssd_shape(rng), bool(rng.random() < 0.4), 500 + i) for i in range(n)]


@pytest.mark.parametrize("case", _state_cases())
def test_sweep_chunk_state(case):
    (b, L, H, G, P, N, Q, dtype), use_seq, seed = case
    announce("sweep chunk_state", case)
    cfg = configs.SSDConfig("s", b, L, H, G, P, N, Q, dtype, seed=seed)
    d = configs.make_ssd_inputs(cfg)
    seq = seq_idx_from_lengths(_lengths(np.random.default_rng(seed), b, L)) if use_seq else None
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    T = tdtype(dtype)
    got = chunk_state_fwd(dev(d["x"], T), dev(d["B"], T), dev(wdt), dev(wA), seq_idx=dev(seq))
    want = O.chunk_state(d["B"], d["x"], wdt, wA, seq_idx=seq)
    check(got, want, TOL[dtype], "states")


def _scan_cases(n=14, seed=78):
    rng = np.random.default_rng(seed)
    return [(_ssd_shape(rng), dict(seq=bool(rng.random() < 0.4), D=bool(rng.random() < 0.7),
                                   z=bool(rng.random() < 0.4), Dhp=bool(rng.random() < 0.3)), 600 + i)
            for i in range(n)]


@pytest.mark.parametrize("case", _scan_cases())
def test_sweep_chunk_scan(case):
    (b, L, H, G, P, N, Q, dtype), opt, seed = case
    announce("sweep chunk_scan", case)
    cfg = configs.SSDConfig("s", b, L, H, G, P, N, Q, dtype, seed=seed)
    d = configs.make_ssd_inputs(cfg, with_z=opt["z"])
    rng = np.random.default_rng(seed)
    seq = seq_idx_from_lengths(_lengths(rng, b, L)) if opt["seq"] else None
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    CB = O.bmm_chunk(d["C"], d["B"], Q, seq_idx=seq).astype(np.float32)
    states = (0.5 * rng.standard_normal((b, math.ceil(L / Q), H, P, N))).astype(np.float32)
    D = None
    if opt["D"]:
        D = rng.uniform(0.5, 1.5, (H, P)).astype(np.float32) if opt["Dhp"] else d["D"]
    T = tdtype(dtype)
    out, out_x = chunk_scan_fwd(dev(CB), dev(d["x"], T), dev(wdt), dev(wA), dev(d["C"], T),
                                dev(states), D=dev(D), z=dev(d["z"], T), seq_idx=dev(seq))
    wo, wox = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states, D=D, z=d["z"], seq_idx=seq,
                           round_fn=O.round_fn_for(dtype))
    check(out, wo, TOL[dtype], "out")
    if opt["z"]:
        check(out_x, wox, TOL[dtype], "out_x")


# ---------------------------------------------------------------------------
# bmm_chunk / state_passing
# ---------------------------------------------------------------------------

def _bmm_cases(n=10, seed=79):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        b, L = int(rng.integers(1, 3)), int(rng.integers(2, 1500))
        G, K = int(rng.choice([1, 2, 4, 8])), int(rng.choice([32, 64, 128, 256]))
        Q = int(rng.choice([32, 64, 128, 256]))
        out.append((b, L, G, K, Q, bool(rng.random() < 0.5), bool(rng.random() < 0.4),
                    "bf16" if rng.random() < 0.5 else "f32", 700 + i))
    return out


@pytest.mark.parametrize("case", _bmm_cases())
def test_sweep_bmm_chunk(case):
    b, L, G, K, Q, causal, use_seq, dtype, seed = case
    announce("sweep bmm_chunk", case)
    rng = np.random.default_rng(seed)
    a = configs.round_to(rng.standard_normal((b, L, G, K)).astype(np.float32), dtype)
    bb = configs.round_to(rng.standard_normal((b, L, G, K)).astype(np.float32), dtype)
    seq = seq_idx_from_lengths(_lengths(rng, b, L)) if use_seq else None
    got = bmm_chunk_fwd(dev(a, tdtype(dtype)), dev(bb, tdtype(dtype)), Q, seq_idx=dev(seq),
                        causal=causal)
    want = O.bmm_chunk(a, bb, Q, seq_idx=seq, causal=causal)
    check(got, want, 1e-5 if dtype == "bf16" else 1e-4, "CB")


def _sp_cases(n=10, seed=80):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        b, nc, H = int(rng.integers(1, 3)), int(rng.integers(1, 20)), int(rng.integers(1, 9))
        D = int(rng.choice([64, 200, 2048, 8192]))
        Q = int(rng.choice([32, 64, 128]))
        out.append((b, nc, H, D, Q, bool(rng.random() < 0.5), bool(rng.random() < 0.4),
                    "bf16" if rng.random() < 0.5 else "f32", 800 + i))
    return out


@pytest.mark.parametrize("case", _sp_cases())
def test_sweep_state_passing(case):
    b, nc, H, D, Q, init, use_seq, out_dtype, seed = case
    announce("sweep state_passing", case)
    rng = np.random.default_rng(seed)
    st = rng.standard_normal((b, nc, H, D)).astype(np.float32)
    dAc = -rng.uniform(0.0, 3.0, (b, H, nc)).astype(np.float32)
    s0 = rng.standard_normal((b, H, D)).astype(np.float32) if init else None
    L = nc * Q - int(rng.integers(0, Q))
    seq = seq_idx_from_lengths(_lengths(rng, b, L)) if use_seq else None
    out, fin = state_passing_fwd(dev(st), dev(dAc), dev(s0), seq_idx=dev(seq), chunk_size=Q,
                                 out_dtype=tdtype(out_dtype))
    wo, wf = O.state_passing(st, dAc, s0, seq_idx=seq, chunk_size=Q)
    check(out, wo, 1e-5 if out_dtype == "f32" else TOL["bf16"], "out")
    check(fin, wf, 1e-5, "final")


# ---------------------------------------------------------------------------
# selective_state_update (decode step)
# ---------------------------------------------------------------------------

def _ssu_cases(n=14, seed=81):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H = int(rng.choice([1, 2, 4, 8, 16, 24]))
        G = int(rng.choice([g for g in (1, 2, 4, 8) if H % g == 0]))
        out.append(dict(b=int(rng.integers(1, 17)), H=H, G=G, P=int(rng.choice([32, 64, 128])),
                        N=int(rng.choice([32, 64, 128, 256])),
                        dt_hdim=bool(rng.random() < 0.3), A_full=bool(rng.random() < 0.2),
                        D=int(rng.integers(0, 3)), z=bool(rng.random() < 0.5),
                        bias=bool(rng.random() < 0.7), softplus=bool(rng.random() < 0.7), seed=900 + i))
    return out


@pytest.mark.parametrize("case", _ssu_cases())
def test_sweep_selective_state_update(case):
    announce("sweep selective_state_update", case)
    c = case
    rng = np.random.default_rng(c["seed"])
    b, H, G, P, N = c["b"], c["H"], c["G"], c["P"], c["N"]
    bf = lambda a: configs.round_to(a.astype(np.float32), "bf16")
    d = dict(
        state=(0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32),
        x=bf(rng.standard_normal((b, H, P))),
        dt=rng.standard_normal((b, H, P) if c["dt_hdim"] else (b, H)).astype(np.float32),
        A=(-np.exp(rng.uniform(0, np.log(16), (H, P, N) if c["A_full"] else H))).astype(np.float32),
        B=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        C=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        D=[None, rng.uniform(0.5, 1.5, H), rng.uniform(0.5, 1.5, (H, P))][c["D"]],
        z=bf(rng.standard_normal((b, H, P))) if c["z"] else None,
        # a dt_bias of dt's head layout (the pairs the reference broadcasts)
        dt_bias=rng.uniform(-4, -2, (H, P) if c["dt_hdim"] else H) if c["bias"] else None,
    )
    if d["D"] is not None:
        d["D"] = d["D"].astype(np.float32)
    if d["dt_bias"] is not None:
        d["dt_bias"] = d["dt_bias"].astype(np.float32)
    if not c["softplus"]:
        # dt' = dt + dt_bias stays >= 0 without softplus (as in the hand-picked
        # test): with dt' < 0 and A < 0 a step multiplies the state by up to
        # exp(|dt' A|) ~ e^58 here, where fp32 alone (a NumPy float32 emulation
        # of the step) is 1.5e-4 off the float64 oracle, beyond the 1e-5 bar
        d["dt"] = np.abs(d["dt"]) * 0.05
        if d["dt_bias"] is not None:
            d["dt_bias"] = rng.uniform(0.0, 0.05, d["dt_bias"].shape).astype(np.float32)
    bfk = ("x", "B", "C", "z")
    t = {k: dev(v, torch.bfloat16 if k in bfk else None) for k, v in d.items()}
    new, y = selective_state_update(**t, dt_softplus=c["softplus"])
    ws, wy = O.selective_state_update(**d, dt_softplus=c["softplus"], round_fn=O.round_fn_for("bf16"))
    check(new, ws, 1e-5, "state")
    check(y, wy, 1e-4, "out")

"""Every head dim, dstate and chunk size the reference accepts, on the GPU
against the oracle.

The reference pads headdim and dstate to its tiles and so runs any size
(kernels/chunk_state_fwd.py:281-295, kernels/chunk_scan_fwd.py:367-390,
kernels/bmm_chunk_fwd.py:206-218); selective_state_update has no size limit
(ops/selective_state_update.py:68-123).  Here the combined forward, each stage
operator and the decode step run head dims 16-200 and dstate 4-320 that the
kernels are not built for (through kernels/_shapes.py's padding, head splitting
and dstate blocks, whose exactness tests/test_shapes.py checks on the CPU), and
chunk sizes the combined forward runs as chunks of 128.  Bars: the plain
BASELINE bar for the layer and the stage operators (max|err|/rms <= 1e-3 for
fp32 inputs, 2e-2 for bf16), the decode step's 1e-5 (state) / 1e-4 (output).
"""

import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, tdtype
from mamba2_jax import configs
from mamba2_jax.kernels import (bmm_chunk_fwd, chunk_scan_fwd, chunk_state_fwd,
                                chunk_state_varlen_mosaic, mamba_chunk_scan_combined_fwd)
from mamba2_jax.ops import selective_state_update
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu

COMBINED = [
    # dtype, b, L, H, G, P, N, Q, init, z, D per head dim, packed sequences
    ("bf16", 2, 300, 4, 2, 48, 16, 128, True, True, True, 0),
    ("bf16", 1, 400, 4, 1, 80, 48, 64, False, True, False, 3),
    ("bf16", 2, 257, 6, 2, 96, 96, 256, True, False, True, 0),
    ("bf16", 1, 500, 4, 2, 128, 160, 128, True, True, False, 2),
    ("f32", 2, 300, 4, 2, 48, 96, 128, True, True, True, 0),
    ("f32", 1, 333, 4, 4, 80, 160, 64, False, False, True, 3),
    ("f32", 1, 300, 2, 2, 96, 48, 256, True, True, False, 0),
    ("bf16", 1, 300, 2, 1, 200, 64, 128, True, True, True, 0),    # head dim above 128
    ("bf16", 1, 300, 4, 2, 64, 320, 128, True, True, True, 2),    # dstate above 256
    ("f32", 2, 200, 2, 1, 16, 300, 64, False, True, False, 0),
    ("bf16", 1, 300, 4, 2, 64, 128, 100, True, True, False, 0),   # chunk 100 (runs as 128)
    ("bf16", 1, 700, 4, 2, 64, 128, 512, False, False, False, 2), # chunk 512
    ("f32", 1, 300, 4, 2, 64, 64, 48, True, False, False, 0),     # chunk 48
    ("bf16", 2, 300, 4, 2, 64, 128, 32, True, True, False, 0),    # chunk 32 (runs as 128)
]


@pytest.mark.parametrize("case", COMBINED)
def test_combined_any_size(case):
    dtype, b, L, H, G, P, N, Q, init, z, Dhp, nseq = case
    announce("combined any size", case)
    cfg = configs.SSDConfig("shape", b, L, H, G, P, N, Q, dtype, init_state=init, nseq=nseq,
                            min_seqlen=16, seed=P * 1000 + N + Q)
    d = configs.make_ssd_inputs(cfg, with_z=z)
    if Dhp:
        d["D"] = np.random.default_rng(P + N).uniform(0.5, 1.5, (H, P)).astype(np.float32)
    T = tdtype(dtype)
    t = dict(x=dev(d["x"], T), dt=dev(d["dt"], T), A=dev(d["A"]), B=dev(d["B"], T),
             C=dev(d["C"], T), D=dev(d["D"]), z=dev(d["z"], T), dt_bias=dev(d["dt_bias"]),
             initial_states=dev(d["initial_states"]), seq_idx=dev(d["seq_idx"]),
             cu_seqlens=dev(d["cu_seqlens"]))
    kw = dict(chunk_size=Q, dt_softplus=True, return_final_states=True,
              return_varlen_states=bool(nseq))
    got = mamba_chunk_scan_combined_fwd(**t, **kw)
    want = O.ssd_combined(io_dtype=dtype, **d, **kw)
    assert got[0].shape == (b, L, H, P) and got[1].shape == (b, H, P, N)
    check(got[0], want[0], TOL[dtype], "out")
    check(got[1], want[1], TOL[dtype], "final_states")
    if nseq:
        assert got[2].shape == (nseq, H, P, N)
        check(got[2], want[2], TOL[dtype], "varlen_states")


STAGE = [
    # dtype, P, N
    ("bf16", 48, 16), ("bf16", 80, 48), ("bf16", 96, 96), ("bf16", 64, 160),
    ("f32", 48, 96), ("f32", 96, 160), ("f32", 16, 48),
    ("bf16", 200, 64), ("bf16", 64, 320), ("f32", 130, 300),
]


def _stage_inputs(dtype, P, N, b=2, L=300, H=4, G=2, Q=128, nseq=0):
    cfg = configs.SSDConfig("shape", b, L, H, G, P, N, Q, dtype, nseq=nseq, min_seqlen=16,
                            seed=P * 7 + N)
    d = configs.make_ssd_inputs(cfg, with_z=True)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    return d, dA.astype(np.float32), dto.astype(np.float32)


@pytest.mark.parametrize("dtype,P,N", STAGE)
def test_chunk_state_any_size(dtype, P, N):
    announce("chunk_state any size", dtype, P, N)
    d, dA, dto = _stage_inputs(dtype, P, N)
    seq = np.repeat([[0, 1]], [100, 200], axis=1).astype(np.int32).repeat(2, 0)
    T = tdtype(dtype)
    got = chunk_state_fwd(dev(d["x"], T), dev(d["B"], T), dev(dto), dev(dA), seq_idx=dev(seq))
    want = O.chunk_state(d["B"], d["x"], dto, dA, seq_idx=seq)
    assert tuple(got.shape) == want.shape
    check(got, want, TOL[dtype], "states")


@pytest.mark.parametrize("dtype,P,N", STAGE)
def test_chunk_scan_any_size(dtype, P, N):
    announce("chunk_scan any size", dtype, P, N)
    d, dA, dto = _stage_inputs(dtype, P, N)
    rng = np.random.default_rng(P + N)
    CB = O.bmm_chunk(d["C"], d["B"], 128).astype(np.float32)
    states = (0.5 * rng.standard_normal((2, 3, 4, P, N))).astype(np.float32)
    D = rng.uniform(0.5, 1.5, (4, P)).astype(np.float32)
    T = tdtype(dtype)
    out, out_x = chunk_scan_fwd(dev(CB), dev(d["x"], T), dev(dto), dev(dA), dev(d["C"], T),
                                dev(states), D=dev(D), z=dev(d["z"], T))
    wo, wox = O.chunk_scan(CB, d["x"], dto, dA, d["C"], states, D=D, z=d["z"],
                           round_fn=O.round_fn_for(dtype))
    check(out, wo, TOL[dtype], "out")
    check(out_x, wox, TOL[dtype], "out_x")


@pytest.mark.parametrize("dtype,P,N", STAGE)
def test_varlen_any_size(dtype, P, N):
    announce("chunk_state_varlen any size", dtype, P, N)
    d, dA, dto = _stage_inputs(dtype, P, N, b=1, nseq=3)
    rng = np.random.default_rng(N)
    cs = (0.5 * rng.standard_normal((3, 4, P, N))).astype(np.float32)
    T = tdtype(dtype)
    got = chunk_state_varlen_mosaic(dev(d["B"][0], T), dev(d["x"][0], T), dev(dto[0]), dev(dA[0]),
                                    dev(d["cu_seqlens"]), dev(cs))
    want = O.chunk_state_varlen(d["B"][0], d["x"][0], dto[0], dA[0], d["cu_seqlens"], cs)
    check(got, want, TOL[dtype], "varlen_states")


@pytest.mark.parametrize("dtype,K", [("bf16", 16), ("bf16", 48), ("f32", 80), ("bf16", 320),
                                     ("f32", 100)])
def test_bmm_chunk_any_k(dtype, K):
    announce("bmm_chunk any k", dtype, K)
    rng = np.random.default_rng(K)
    a = configs.round_to(rng.standard_normal((2, 300, 2, K)).astype(np.float32), dtype)
    bb = configs.round_to(rng.standard_normal((2, 300, 2, K)).astype(np.float32), dtype)
    got = bmm_chunk_fwd(dev(a, tdtype(dtype)), dev(bb, tdtype(dtype)), 128, causal=True)
    want = O.bmm_chunk(a, bb, 128, causal=True)
    check(got, want, 1e-5 if dtype == "bf16" else 1e-4, "CB")


SSU = [
    # b, H, G, P, N, variants
    (3, 4, 2, 1024, 4, dict(inplace=True)),        # 1 lane per row, 1024 rows
    (3, 4, 2, 1024, 4, dict(inplace=False)),
    (2, 4, 1, 333, 8, dict(inplace=True, A_full=True)),
    (2, 4, 1, 64, 8, dict(inplace=False, dt_hdim=True)),
    (5, 6, 3, 64, 12, dict(inplace=True)),         # lanes past N idle
    (4, 4, 2, 64, 48, dict(inplace=False, D_hdim=True)),
    (4, 4, 2, 80, 96, dict(inplace=True)),
    (4, 4, 2, 48, 160, dict(inplace=False, A_full=True)),
    (2, 4, 2, 64, 18, dict(inplace=True)),         # dstate not a multiple of 4
    (2, 4, 2, 50, 7, dict(inplace=False, dt_hdim=True, A_full=True)),
    (2, 4, 2, 64, 320, dict(inplace=True)),        # dstate above 256
    (1, 2, 1, 17, 513, dict(inplace=False, D_hdim=True)),
]


@pytest.mark.parametrize("case", SSU)
def test_ssu_any_size(case):
    b, H, G, P, N, kw = case
    announce("selective_state_update any size", case)
    rng = np.random.default_rng(P * N + b)
    bf = lambda a: configs.round_to(a.astype(np.float32), "bf16")
    dt_hdim, A_full, D_hdim = kw.get("dt_hdim", False), kw.get("A_full", False), kw.get("D_hdim", False)
    d = dict(
        state=(0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32),
        x=bf(rng.standard_normal((b, H, P))),
        dt=rng.standard_normal((b, H, P) if dt_hdim else (b, H)).astype(np.float32),
        A=(-np.exp(rng.uniform(0, np.log(16), (H, P, N) if A_full else H))).astype(np.float32),
        B=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        C=bf(rng.standard_normal((b, G, N)) / np.sqrt(N)),
        D=rng.uniform(0.5, 1.5, (H, P) if D_hdim else H).astype(np.float32),
        z=bf(rng.standard_normal((b, H, P))),
        dt_bias=rng.uniform(-4, -2, (H, P) if dt_hdim else H).astype(np.float32),
    )
    bfk = ("x", "B", "C", "z")
    t = {k: dev(v, torch.bfloat16 if k in bfk else None) for k, v in d.items()}
    before = t["state"].clone()
    new, y = selective_state_update(**t, dt_softplus=True, inplace=kw["inplace"])
    ws, wy = O.selective_state_update(**d, dt_softplus=True, round_fn=O.round_fn_for("bf16"))
    check(new, ws, 1e-5, "state")
    check(y, wy, 1e-4, "out")
    if kw["inplace"]:
        assert new.data_ptr() == t["state"].data_ptr()
    else:
        assert torch.equal(t["state"], before)

"""A seeded sweep of the whole SSD forward over the supported envelope.

Forty shapes drawn once from a fixed seed (so every run checks the same ones):
batch 1-3, ragged lengths from 1 to 700 tokens (shorter than a chunk included),
2-16 heads in 1-8 groups, head dim 32 / 64 / 128, dstate 64 / 128 / 256, chunk
64 / 128 / 256, bf16 and fp32 inputs, with or without an initial state, a
per-head-dim D, a z gate, the softplus / dt_limit variants, and packed
sequences (seq_idx + cu_seqlens, the varlen final states).  Each is compared
with the CPU oracle at the parity bar (max|err|/rms <= 2e-2 bf16, 1e-3 fp32),
outputs and final states alike; the varlen states as _check_varlen says.  The
hand-picked tests cover the benchmark shapes; this one covers the combinations
between them (which path a shape takes: fused or staged kernels, the
state-pass split, chunk 256 run as 128).
"""

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, host, tdtype
from mamba2_jax import configs
from mamba2_jax.kernels import (chunk_cumsum_fwd, chunk_state_fwd, chunk_state_varlen_mosaic,
                                mamba_chunk_scan_combined_fwd, state_passing_fwd)
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dtype = "bf16" if rng.random() < 0.6 else "f32"
        P = int(rng.choice([32, 64, 64, 64, 128]))
        N = int(rng.choice([64, 128, 256]))
        Q = int(rng.choice([64, 128, 128, 256]))
        H = int(rng.choice([2, 4, 6, 8, 16]))
        G = int(rng.choice([g for g in (1, 2, 4, 8) if H % g == 0]))
        packed = rng.random() < 0.25
        b = 1 if packed else int(rng.integers(1, 4))
        L = int(rng.integers(1, 701))
        nseq = int(rng.integers(2, 6)) if packed and L >= 8 else 0
        opts = dict(
            init=bool(rng.random() < 0.4),
            z=bool(rng.random() < 0.3),
            Dhp=bool(rng.random() < 0.3),
            softplus=bool(rng.random() < 0.8),
            limit=bool(rng.random() < 0.3),
        )
        cfg = configs.SSDConfig(f"sweep{i}", b, L, H, G, P, N, Q, dtype, init_state=opts["init"],
                                nseq=nseq, min_seqlen=max(1, L // (2 * max(nseq, 1))),
                                seed=1000 + i)
        out.append((cfg, opts))
    return out


_CASES = _cases()


@pytest.mark.parametrize("idx", range(len(_CASES)))
def test_sweep(idx):
    cfg, opt = _CASES[idx]
    announce("sweep", cfg, opt)
    d = configs.make_ssd_inputs(cfg, with_z=opt["z"])
    if opt["Dhp"]:
        d["D"] = np.random.default_rng(idx).uniform(0.5, 1.5, (cfg.nheads, cfg.headdim)).astype(np.float32)
    varlen = cfg.nseq > 0
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=opt["softplus"], return_final_states=True,
              return_varlen_states=varlen)
    if opt["limit"]:
        kw["dt_limit"] = (0.001, 0.2)
    T = tdtype(cfg.dtype)
    t = dict(x=dev(d["x"], T), dt=dev(d["dt"], T), A=dev(d["A"]), B=dev(d["B"], T),
             C=dev(d["C"], T), D=dev(d["D"]), z=dev(d["z"], T), dt_bias=dev(d["dt_bias"]),
             initial_states=dev(d["initial_states"]), seq_idx=dev(d["seq_idx"]),
             cu_seqlens=dev(d["cu_seqlens"]))
    got = mamba_chunk_scan_combined_fwd(**t, **kw)
    torch.cuda.synchronize()
    want = O.ssd_combined(io_dtype=cfg.dtype, **d, **kw)
    tol = TOL[cfg.dtype]
    check(got[0], want[0], tol, "out")
    check(got[1], want[1], tol, "final_states")
    if varlen:
        _check_varlen(cfg, d, t, kw, got[2], want[2])


def _check_varlen(cfg, d, t, kw, vs, want_vs):
    """The packed final states.  They add exp(dA) * (the passed state of the
    sequence's last chunk, rounded to C.dtype) -- a rounding point of the
    reference (kernels/ssd_combined.py:140, kernels/chunk_state_fwd.py:587-595)
    -- so for bf16 two checks that do not depend on where fp32 summation order
    puts a rounding flip:
    * identical inputs: the passed states, dA and dt of the GPU stage operators
      fed to both chunk_state_varlen_mosaic and the oracle's
      chunk_state_varlen, at the plain bar;
    * the combined forward's varlen states against those of the stage
      operators: within one bf16 rounding of the carried term (2^-8 of the
      largest value).
    fp32 has no rounding point there: against the oracle at the plain bar."""
    tol = TOL[cfg.dtype]
    if cfg.dtype == "f32":
        check(vs, want_vs, tol, "varlen_states")
        return
    Q = cfg.chunk_size
    b, L, H, P = t["x"].shape
    N = t["B"].shape[-1]
    dA, dto = chunk_cumsum_fwd(t["dt"], t["A"], Q, t["dt_bias"], kw["dt_softplus"],
                               kw.get("dt_limit", (0.0, float("inf"))))
    st = chunk_state_fwd(t["x"], t["B"], dto, dA, seq_idx=t["seq_idx"])
    nc = st.shape[1]
    init = None if t["initial_states"] is None else t["initial_states"].reshape(b, H, P * N)
    passed, _ = state_passing_fwd(st.reshape(b, nc, H, P * N), dA[..., -1], init,
                                  seq_idx=t["seq_idx"], chunk_size=Q, out_dtype=t["x"].dtype)
    passed = passed.reshape(b, nc, H, P, N)
    got = chunk_state_varlen_mosaic(t["B"][0], t["x"][0], dto[0], dA[0], t["cu_seqlens"], passed[0])
    want = O.chunk_state_varlen(d["B"][0], d["x"][0], host(dto[0]), host(dA[0]), d["cu_seqlens"],
                                host(passed[0]))
    check(got, want, tol, "varlen_states (identical passed states)")
    g, w = host(vs), host(got)
    e = float(np.max(np.abs(g - w)) / np.max(np.abs(w)))
    print(f"  varlen_states combined vs stages: max|err|/max|ref| = {e:.3e} (tol 2^-8)", flush=True)
    assert e <= 2.0 ** -8, f"varlen_states combined vs stage operators: {e:.3e}"

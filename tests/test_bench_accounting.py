"""bench.py's algorithmic work per stage (the bytes and flops its roofline
fractions divide by), its chunk mapping, and its one-GPU guard -- host only.

The expected byte counts are written out from the tensor shapes of each stage
(inputs read once, outputs written once), independently of bench.stage_work's
formulas; profiles/hbm_traffic_<config>.json hold what rocprofv3 measured for
the same stages and must name exactly the stages the bench reports.
"""

import dataclasses
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mamba2-jax-pallas_amd")]

import bench  # noqa: E402
from mamba2_jax import _lib as L  # noqa: E402
from mamba2_jax import configs  # noqa: E402


def test_internal_chunk_matches_the_library():
    # m2_ssd_combined runs bf16 chunks of 256 as 128 when both fused kernels
    # apply and fp32 chunks of 256 always as 128 (csrc/capi.hip internal_args)
    assert bench.internal_chunk(configs.CONFIGS["c0"]) == 128          # fp32, chunk 256
    assert bench.internal_chunk(configs.CONFIGS["c1"]) == 128          # bf16, chunk 256, fused
    assert bench.internal_chunk(configs.CONFIGS["c2"]) == 128
    wide = dataclasses.replace(configs.CONFIGS["c1"], headdim=128)     # no fused kernels
    assert bench.internal_chunk(wide) == 256


@pytest.mark.parametrize("Q,dtype,P", [(32, "bf16", 64), (100, "bf16", 64), (512, "bf16", 64),
                                       (48, "f32", 64), (32, "bf16", 32), (256, "bf16", 32),
                                       (64, "f32", 64), (96, "bf16", 32)])
def test_other_chunk_sizes_match_the_library(Q, dtype, P):
    """Chunk sizes other than 64 / 128 / 256 run as 128 (and bf16 ones the fused
    kernels do not take, where 128 puts the layer on them): bench's mirror of
    that choice agrees with the workspace the library asks for."""
    cfg = dataclasses.replace(configs.CONFIGS["c2"], seqlen=1000, nheads=16, ngroups=2,
                              chunk_size=Q, dtype=dtype, headdim=P)
    c = dataclasses.replace(cfg, chunk_size=bench.internal_chunk(cfg))
    assert _workspace_bytes(cfg) == _expected_workspace(cfg, bench.states_is_fused(c))


def test_c2_fused_stage_bytes():
    b, L, H, G, P, N, Q = 1, 4096, 128, 8, 64, 128, 128
    nc = L // Q
    x, BC, dt = b * L * H * P * 2, b * L * G * N * 2, b * L * H * 2
    rows = b * H * nc * Q * 4                        # one fp32 [b, H, nc, Q] array
    chunks = b * H * nc * 4                          # one fp32 [b, H, nc] array
    states = b * nc * H * P * N * 2                  # bf16 states entering each chunk
    final = b * H * P * N * 4
    y = b * L * H * P * 4
    w = bench.stage_work(configs.CONFIGS["c2"])
    assert set(w) == {"chunk_cumsum", "chunk_state+state_passing", "bmm_chunk+chunk_scan"}
    # cumsum: dt in; dA_cumsum, dt', weights out; the chunk decay out; A / bias
    assert w["chunk_cumsum"][0] == dt + 3 * rows + chunks + 8 * H
    # state pass: x, B, weights, decay in; states, final states out
    assert w["chunk_state+state_passing"][0] == x + BC + rows + chunks + states + final
    # scan: x, B, C, dA_cumsum, dt', states, D in; y out
    assert w["bmm_chunk+chunk_scan"][0] == x + 2 * BC + 2 * rows + states + 4 * H + y
    assert w["bmm_chunk+chunk_scan"][0] == 289_407_488


def test_c0_fp32_stage_bytes_at_chunk_128():
    b, L, H, G, P, N, Q = 1, 2048, 24, 1, 64, 128, 128
    nc = L // Q
    x, BC, dt = b * L * H * P * 4, b * L * G * N * 4, b * L * H * 4
    rows = b * H * nc * Q * 4
    S = b * nc * H * P * N * 4                       # fp32 chunk states / passed states
    cb = b * nc * G * Q * Q * 4
    y = b * L * H * P * 4
    final = b * H * P * N * 4
    w = bench.stage_work(configs.CONFIGS["c0"])
    assert set(w) == {"chunk_cumsum+chunk_state", "state_passing+bmm_chunk", "chunk_scan"}
    # chunk_cumsum inside chunk_state: dt, x, B in; dA_cumsum, dt', states out
    assert w["chunk_cumsum+chunk_state"][0] == dt + x + BC + 2 * rows + S
    # state_passing (chunk states and chunk-end dA in; passed and final states
    # out) and bmm_chunk (C, B in; CB out) in one launch
    assert w["state_passing+bmm_chunk"][0] == 2 * S + b * H * nc * 4 + final + 2 * BC + cb
    assert w["chunk_scan"][0] == cb + x + 2 * rows + BC + S + 4 * H + y
    # flops of the chunk-128 algorithm: intra-chunk (k <= m) and carried-state terms
    assert w["chunk_scan"][1] == b * nc * H * P * Q * (Q + 1) + 2 * b * L * H * N * P


@pytest.mark.parametrize("name", ["c0", "c1", "c2", "c3", "c2_f32"])
def test_traffic_files_name_the_reported_stages(name):
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{name}.json")
    with open(path) as f:
        t = json.load(f)
    cfg = configs.CONFIGS[name.split("_")[0]]
    if name.endswith("_f32"):
        cfg = dataclasses.replace(cfg, dtype="f32")
    stages = set(bench.stage_work(cfg, with_init=cfg.init_state))
    # chunk_state_varlen (c3) runs after the five stage intervals
    measured = {k for k in t if k not in ("config", "unit", "source", "chunk_state_varlen",
                                          "above_algorithmic")}
    assert measured <= stages, measured - stages
    # the dominant stage of every configuration carries a measurement
    w = bench.stage_work(cfg, with_init=cfg.init_state)
    assert max(w, key=lambda s: w[s][0]) in measured
    # within 5 % of the algorithmic bytes, or up to 20 % above them for a stage
    # whose excess the file explains
    excess = t.get("above_algorithmic", {})
    assert set(excess) <= measured and all(isinstance(v, str) and v for v in excess.values())
    for k in measured:
        if k in excess:
            assert w[k][0] <= t[k] <= 1.2 * w[k][0], (k, t[k], w[k][0])
        else:
            assert abs(t[k] - w[k][0]) <= 0.05 * w[k][0], (k, t[k], w[k][0])


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def _workspace_bytes(cfg):
    """m2_ssd_combined_workspace_size for cfg (host arithmetic only)."""
    import ctypes
    from mamba2_jax import _lib as L
    a = L.SsdCombinedArgs(batch=cfg.batch, seqlen=cfg.seqlen, nheads=cfg.nheads,
                          headdim=cfg.headdim, ngroups=cfg.ngroups, dstate=cfg.dstate,
                          chunk_size=cfg.chunk_size, dtype=0 if cfg.dtype == "f32" else 1,
                          dt_dtype=0 if cfg.dtype == "f32" else 1)
    return L.load_library().m2_ssd_combined_workspace_size(ctypes.byref(a))


def _expected_workspace(cfg, fused):
    """The combined forward's workspace written out per slot: dA_cumsum and dt'
    always; the weights and the chunk decay (fused state pass) or the fp32 chunk
    states (staged); the states entering each chunk in the input dtype; CB
    unless bmm_chunk runs inside the scan."""
    al = lambda v: (v + 255) // 256 * 256
    Q = bench.internal_chunk(cfg)
    c = dataclasses.replace(cfg, chunk_size=Q)
    es = 4 if cfg.dtype == "f32" else 2
    nc = -(-cfg.seqlen // Q)
    cq = cfg.batch * cfg.nheads * nc * Q
    S = cfg.batch * nc * cfg.nheads * cfg.headdim * cfg.dstate
    tot = 2 * al(4 * cq) + al(S * es)
    tot += al(4 * cq) + al(4 * cfg.batch * cfg.nheads * nc) if fused else al(4 * S)
    if not bench.scan_is_fused(c, states_fused=fused):
        tot += al(es * cfg.batch * nc * cfg.ngroups * Q * Q)
    return tot


@pytest.mark.parametrize("name,dtype,force,fused", [
    ("c2", "bf16", None, True),
    ("c2", "f32", None, True),           # 256 workgroups: the fp32 fused state pass
    ("c2", "f32", "staged", False),
    ("c0", "f32", None, False),          # 48 workgroups: the staged kernels
    ("c0", "f32", "fused", True),
    ("c1", "bf16", None, True),
])
def test_state_pass_choice_matches_the_library(name, dtype, force, fused):
    """bench.states_is_fused (which names the stages the bench reports) agrees
    with the library's own choice, read from the workspace it asks for."""
    cfg = dataclasses.replace(configs.CONFIGS[name], dtype=dtype)
    c = dataclasses.replace(cfg, chunk_size=bench.internal_chunk(cfg))
    assert bench.states_is_fused(c, force=force) == fused
    if force:
        with L.dispatch_override("f32_states", force):
            assert _workspace_bytes(cfg) == _expected_workspace(cfg, fused)
    else:
        assert _workspace_bytes(cfg) == _expected_workspace(cfg, fused)

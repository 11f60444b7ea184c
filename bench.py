"""Benchmark: one Mamba2 SSD layer forward at the nemotron-h-8b shape on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--dtype f32|bf16]
                    [--no-cpu-baseline]
    python bench.py --ops [--lm 130m,2.7b]     (the ops around the SSD, LM decode)

A step is one call of mamba2_jax.kernels.mamba_chunk_scan_combined_fwd on
synthetic inputs already resident in HBM, returning the output and the final
states.  For bf16 at the benchmark shapes the five stages run as three kernels:
chunk_cumsum (+ chunk-state weights), chunk_state + state_passing (one
chunk-sequential kernel) and bmm_chunk + chunk_scan (one kernel).  Prints ONE
JSON line (rank 0): tokens/s and ms per layer (W warm-up steps, then K
back-to-back steps with events only around them), the roofline fraction of the
dominant kernel and the per-stage table (a pass of max(K, 300) steps just
before, with HIP events recorded on the launch stream at every kernel
boundary; it also brings the GPU to the steady clocks an idle GPU lacks).

Measured in the same run, before the headline (which they also bring to steady
GPU clocks): the other BASELINE configurations c0, c1 and c3 (`configs`: ms per
layer, tokens/s, per-kernel table, dominant kernel's roofline, a sampled CPU
baseline), the headline shape with fp32 inputs, each stage operator of the
reference's API called on its own (`stage_operators`) and the decode step
(c4: 256 in-place selective_state_update steps).  Then the CPU baseline: the
oracle's NumPy restatement of the reference's naive path on the full c2
workload, on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mamba2-jax-pallas_amd"))

METRIC = "SSD layer fwd ms + tokens/sec and % MFMA/HBM roofline, nemotron-h-8b shape"
PEAK_HBM_GBS = 8000.0            # MI355X HBM3E, GB/s
PEAK_MFMA_TFLOPS = {"bf16": 2500.0, "f32": 157.3}   # dense
STAGES = ["chunk_cumsum", "chunk_state", "state_passing", "bmm_chunk", "chunk_scan"]


def internal_chunk(cfg):
    """The chunk size the combined path runs (m2_ssd_combined's internal_args):
    bf16 chunk sizes the fused kernels do not take run as chunks of 128 when
    both fused kernels then apply, fp32 chunks of 256 always, and chunk sizes
    other than 64 / 128 / 256 always."""
    import dataclasses
    Q = cfg.chunk_size
    fused = lambda c: states_is_fused(c) and scan_is_fused(c)
    if cfg.dtype == "bf16" and Q != 128 and not fused(cfg):
        if fused(dataclasses.replace(cfg, chunk_size=128)):
            Q = 128
    if cfg.dtype == "f32" and Q == 256:
        Q = 128
    return Q if Q in (64, 128, 256) else 128


def stage_work(cfg, with_init=False, with_z=False, cu_seqlens=None):
    """Algorithmic (compulsory) HBM bytes and flops per launch of each stage, as
    the combined path runs them (CB and the carried states in the input dtype);
    with cu_seqlens (packed sequences, batch 1) also the varlen final states."""
    import dataclasses
    cfg = dataclasses.replace(cfg, chunk_size=internal_chunk(cfg))
    s = 2 if cfg.dtype == "bf16" else 4
    b, L, H, G, P, N, Q = (cfg.batch, cfg.seqlen, cfg.nheads, cfg.ngroups, cfg.headdim,
                           cfg.dstate, cfg.chunk_size)
    nc = math.ceil(L / Q)
    S = b * nc * H * P * N
    cq = b * H * nc * Q
    w = {}
    w["chunk_cumsum"] = (b * L * H * s + 8 * cq + 8 * H, 5 * b * L * H)
    w["chunk_state"] = (b * L * H * P * s + b * L * G * N * s + 8 * cq + 4 * S,
                        2 * b * L * H * P * N)
    w["state_passing"] = (4 * S + 4 * b * H * nc + (4 * b * H * P * N if with_init else 0)
                          + s * S + 4 * b * H * P * N, 2 * S)
    w["bmm_chunk"] = (2 * b * L * G * N * s + s * b * nc * G * Q * Q, 2 * b * nc * G * Q * Q * N)
    w["chunk_scan"] = (s * b * nc * G * Q * Q + b * L * H * P * s + 8 * cq + b * L * G * N * s
                       + s * S + 4 * H + (b * L * H * P * s if with_z else 0) + 4 * b * L * H * P,
                       b * nc * H * P * Q * (Q + 1) + 2 * b * L * H * N * P)
    if scan_is_fused(cfg):
        # bmm_chunk runs inside the scan kernel: B is read instead of a CB buffer
        sb, sf = w.pop("bmm_chunk")
        cb_bytes = s * b * nc * G * Q * Q
        by, fl = w.pop("chunk_scan")
        w["bmm_chunk+chunk_scan"] = (by - cb_bytes + b * L * G * N * s, fl + sf)
    if pass_bmm_fused(cfg):
        # fp32 with the tiled bmm_chunk kernel: state_passing and bmm_chunk in one launch
        pb, pf = w.pop("state_passing")
        mb, mf = w.pop("bmm_chunk")
        w[FUSED_PASS_BMM] = (pb + mb, pf + mf)
    if cumsum_in_state(cfg):
        # fp32: chunk_cumsum inside the chunk_state kernel, which reads the raw
        # dt and writes dA_cumsum / dt' for the later stages (no weights read)
        cb_, cf_ = w.pop("chunk_cumsum")
        sb_, sf_ = w.pop("chunk_state")
        w[FUSED_CUMSUM] = (sb_ - 8 * cq + b * L * H * s + 8 * cq, sf_ + cf_)
    if states_is_fused(cfg):
        # chunk_cumsum also writes the chunk-state weights and the chunk decay;
        # one chunk-sequential kernel then reads x, B and the weights and writes
        # the states entering each chunk and the final states (no fp32 chunk states)
        cb_, cf_ = w.pop("chunk_cumsum")
        w.pop("chunk_state"), w.pop("state_passing")
        w["chunk_cumsum"] = (cb_ + 4 * cq + 4 * b * H * nc, cf_ + 3 * cq)
        w[FUSED_STATES] = (b * L * H * P * s + b * L * G * N * s + 4 * cq + 4 * b * H * nc
                           + s * S + 4 * b * H * P * N + (4 * b * H * P * N if with_init else 0),
                           2 * b * L * H * P * N + 2 * S)
    if cu_seqlens is not None:
        # per sequence: the x and B rows of its part of its last chunk, their
        # dA_cumsum / dt', the state entering that chunk (when the sequence
        # started earlier) and the fp32 final state out
        cu = [int(v) for v in cu_seqlens]
        by = fl = 0
        for s0, s1 in zip(cu[:-1], cu[1:]):
            c0 = (s1 - 1) // Q * Q
            rows = s1 - max(s0, c0)
            by += (rows * H * P + rows * G * N) * s + 8 * H * rows + 4 * H * P * N
            by += s * H * P * N if s0 < c0 else 0
            fl += 2 * 2 * rows * H * P * N
        w[VARLEN] = (by, fl)
    return w


FUSED_STATES = "chunk_state+state_passing"
FUSED_CUMSUM = "chunk_cumsum+chunk_state"
FUSED_PASS_BMM = "state_passing+bmm_chunk"
VARLEN = "chunk_state_varlen"


def pass_bmm_fused(cfg):
    """fp32 inputs whose bmm_chunk takes the tiled kernel (fewer than 128
    (chunk, group) blocks, or chunk / dstate outside 64 / 128): state_passing
    and bmm_chunk run in one launch (m2::state_passing_bmm_supported)."""
    if cfg.dtype != "f32" or states_is_fused(cfg) or scan_is_fused(cfg):
        return False
    Q, K = cfg.chunk_size, cfg.dstate
    nblocks = cfg.batch * math.ceil(cfg.seqlen / Q) * cfg.ngroups
    return not (nblocks >= 128 and Q in (64, 128) and K in (64, 128))


def cumsum_in_state(cfg):
    """The combined path runs chunk_cumsum inside the fp32 chunk_state kernel
    for fp32, headdim 64, dstate a multiple of 128 and chunk_size 64 / 128
    when the fused state pass does not apply (m2::chunk_state_cumsum_supported)."""
    return (cfg.dtype == "f32" and cfg.headdim == 64 and cfg.dstate % 128 == 0
            and cfg.chunk_size in (64, 128) and cfg.nheads % cfg.ngroups == 0
            and not states_is_fused(cfg))


def states_is_fused(cfg, force=None):
    """The combined path runs chunk_state and state_passing as one kernel for
    headdim 64, dstate a multiple of 64 and chunk_size a multiple of 64 up to
    256: always for bf16, for fp32 where the pass has at least 256 workgroups
    (batch x heads x dstate / 64) or the f32_states testing override ("fused" /
    "staged", given as `force`) forces it (m2::states_fused_supported)."""
    shape = (cfg.headdim == 64 and cfg.dstate % 64 == 0 and cfg.chunk_size % 64 == 0
             and cfg.chunk_size <= 256 and cfg.nheads % cfg.ngroups == 0)
    if cfg.dtype == "bf16":
        return shape
    if not shape or force == "staged":
        return False
    return force == "fused" or cfg.batch * cfg.nheads * (cfg.dstate // 64) >= 256


def scan_is_fused(cfg, states_fused=None):
    """The combined path fuses bmm_chunk into chunk_scan for bf16, headdim 64,
    dstate 64/128/256 and chunk_size 64/128 (m2::scan_fused_supported), and for
    fp32, headdim 64, dstate 64/128 at chunk 128, where the group scan builds
    CB itself (layer_scan_builds_cb in csrc/capi.hip); `states_fused` gives the
    state pass choice where a testing override forces it."""
    if cfg.dtype == "f32":
        if states_fused is None:
            states_fused = states_is_fused(cfg)
        # except where state_passing carries bmm_chunk in its launch (fewer
        # than 128 (chunk, group) blocks on the staged path)
        nblocks = cfg.batch * math.ceil(cfg.seqlen / cfg.chunk_size) * cfg.ngroups
        return (cfg.headdim == 64 and cfg.dstate in (64, 128) and cfg.chunk_size == 128
                and cfg.nheads % cfg.ngroups == 0 and (states_fused or nblocks >= 128))
    return (cfg.dtype == "bf16" and cfg.headdim == 64 and cfg.dstate in (64, 128, 256)
            and cfg.chunk_size in (64, 128))


def measured_traffic(config):
    """HBM bytes per launch of each stage as measured by rocprofv3 FETCH_SIZE /
    WRITE_SIZE (scaled by a plain copy's readings) for this config, from
    profiles/hbm_traffic_<config>.json; empty when there is none."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{config}.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def attach_traffic(roof, traffic, dom):
    """roofline.traffic for the dominant stage `dom`, with the file it comes
    from and, where the file explains measured bytes above the algorithmic
    ones for that stage, the explanation."""
    roof["traffic"] = traffic.get(dom)
    if traffic:
        roof["traffic_source"] = traffic.get("source")
        note = traffic.get("above_algorithmic", {}).get(dom)
        if note:
            roof["traffic_note"] = note


class HipEvents:
    """Raw HIP events for the per-stage timing, created with
    hipEventDisableSystemFence: recording one does not write back and
    invalidate the caches between the kernels it separates (a default event
    does, which adds ~4 us per record).  Uses the HIP runtime torch loaded."""

    FLAGS = 0x20000000          # hipEventDisableSystemFence

    class Event:
        def __init__(self, handle):
            self.cuda_event = handle

    def __init__(self):
        import ctypes
        self._ct = ctypes
        self._hip = ctypes.CDLL("libamdhip64.so.7")
        self._hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self._hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                  ctypes.c_void_p]
        self._hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self._made = []

    def new(self):
        e = self._ct.c_void_p()
        rc = self._hip.hipEventCreateWithFlags(self._ct.byref(e), self.FLAGS)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        self._made.append(e.value)
        return self.Event(e.value)

    def elapsed_ms(self, a, b):
        f = self._ct.c_float()
        rc = self._hip.hipEventElapsedTime(self._ct.byref(f), a.cuda_event, b.cuda_event)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return f.value

    def __del__(self):
        for e in getattr(self, "_made", []):
            self._hip.hipEventDestroy(e)


def cpu_baseline(cfg, heads, min_seconds=10.0, max_reps=20):
    """The oracle's NumPy restatement of the reference naive path (float32), on
    the first `heads` heads (whole groups) of the workload, scaled to all heads."""
    import numpy as np
    from threadpoolctl import threadpool_info
    from mamba2_jax import configs
    from oracle import ssd_oracle as O
    import dataclasses
    hpg = cfg.nheads // cfg.ngroups
    heads = max(hpg, (heads // hpg) * hpg)
    sub = dataclasses.replace(cfg, nheads=heads, ngroups=heads // hpg)
    d = configs.make_ssd_inputs(sub)
    kw = dict(chunk_size=sub.chunk_size, dt_softplus=True, return_final_states=True,
              io_dtype=sub.dtype, acc=np.float32)
    O.ssd_combined(**d, **kw)                     # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < min_seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        O.ssd_combined(**d, **kw)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times)) * cfg.nheads / heads
    threads = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    what = ("the full workload" if heads == cfg.nheads else
            f"{heads} of {cfg.nheads} heads (whole groups) x {cfg.nheads / heads:g} (linear in heads)")
    return {
        "value": cfg.tokens / t, "unit": "tokens/s", "cores": threads, "kind": "port",
        "cpu": cpu_model(), "ms_per_layer": t * 1e3, "sampled": heads != cfg.nheads,
        "sample": (f"oracle NumPy float32 restatement of ssd_naive, {what}, full L={cfg.seqlen}; "
                   f"median of {len(times)} runs; host affinity "
                   f"{len(os.sched_getaffinity(0))} cpus, BLAS threads {threads}"),
    }


def bench_decode(steps=256, warmup=128):
    """c4: `steps` consecutive in-place decode steps (batch 64, H 128, G 8, P 64, N 128)."""
    import torch
    from mamba2_jax import configs
    from mamba2_jax.ops import selective_state_update
    cfg = configs.DECODE
    d = configs.make_decode_inputs(cfg, steps=steps)
    dev = torch.device("cuda")
    bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)
    f = lambda a: torch.from_numpy(a).to(dev)
    state = f(d["state"])
    xs, zs, Bs, Cs, dts = bf(d["x"]), bf(d["z"]), bf(d["B"]), bf(d["C"]), f(d["dt"])
    A, D, bias = f(d["A"]), f(d["D"]), f(d["dt_bias"])
    for t in range(warmup):
        selective_state_update(state, xs[t], dts[t], A, Bs[t], Cs[t], D=D, z=zs[t],
                               dt_bias=bias, dt_softplus=True, inplace=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for t in range(steps):
        selective_state_update(state, xs[t], dts[t], A, Bs[t], Cs[t], D=D, z=zs[t],
                               dt_bias=bias, dt_softplus=True, inplace=True)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    b, H, G, P, N = cfg.batch, cfg.nheads, cfg.ngroups, cfg.headdim, cfg.dstate
    by = 8 * b * H * P * N + b * H * P * (2 + 2 + 4) + b * H * 4 + 2 * b * G * N * 2 + 12 * H
    return {"workload": "selective_state_update, batch 64, H 128, G 8, P 64, N 128, "
                        "fp32 state in place, bf16 x/z/B/C, 256 consecutive steps",
            "ms_per_step": ms, "tokens_per_s": b / (ms * 1e-3),
            "hbm_gbs": by / (ms * 1e-3) / 1e9, "hbm_frac": by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "bytes_per_step": by}


def _graph_time_ms(fn, calls=20, replays=10):
    """Mean GPU time of fn() from a HIP graph of `calls` back-to-back calls
    replayed `replays` times (no per-call host overhead in the figure)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (calls * replays)


def bench_ops(lm_configs=("130m",)):
    """The ops on either side of the SSD at the nemotron-h-8b layer shape
    (causal_conv1d split into x / B / C, gated RMSNorm), the conv decode update
    at the c4 batch, and the LM decode step (HIP graph) for the given model
    shapes (random bf16 weights)."""
    import torch
    from mamba2_jax.ops import causal_conv1d, causal_conv1d_update, rms_norm_gated
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *shape, dt=torch.bfloat16: torch.randn(shape, generator=g, device=dev).to(dt)
    out = {}
    L, H, P, G, N, W = 4096, 128, 64, 8, 128, 4
    dssm, gn = H * P, G * N
    D = dssm + 2 * gn
    dproj = 2 * dssm + 2 * gn + H
    xbc = rnd(1, L, D)
    w, b = rnd(D, W), rnd(D)
    ms = _graph_time_ms(lambda: causal_conv1d(xbc.transpose(1, 2), w, b, "silu",
                                              split_sizes=(dssm, gn, gn)))
    by = 2 * 2 * L * D + D * (W + 1) * 2
    out["causal_conv1d"] = {"workload": f"xBC (1, {L}, {D}) bf16 channels-last, width {W}, silu, "
                                        "split into x / B / C", "ms": ms, "bytes": by,
                            "hbm_gbs": by / (ms * 1e-3) / 1e9,
                            "hbm_frac": by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}
    y = rnd(1, L, dssm, dt=torch.float32)
    zx = rnd(1, L, dproj)
    z = zx[:, :, dssm:2 * dssm]
    nw = torch.rand(dssm, generator=g, device=dev)
    ms = _graph_time_ms(lambda: rms_norm_gated(y, nw, z=z, group_size=dssm // G,
                                               norm_before_gate=False))
    by = L * dssm * (4 + 2 + 4) + dssm * 4
    out["rms_norm_gated"] = {"workload": f"y (1, {L}, {dssm}) f32, z bf16 slice of the "
                                         f"in-projection, groups of {dssm // G}, gate first",
                             "ms": ms, "bytes": by, "hbm_gbs": by / (ms * 1e-3) / 1e9,
                             "hbm_frac": by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}
    bsz = 64
    st = torch.randn((bsz, D, W), generator=g, device=dev)
    xn = rnd(bsz, D)
    ms = _graph_time_ms(lambda: causal_conv1d_update(xn, st, w, b, "silu", inplace=True))
    by = bsz * D * (2 * W * 4 + 2 + 4)
    out["causal_conv1d_update"] = {"workload": f"batch {bsz}, {D} channels, f32 state in place",
                                   "ms": ms, "bytes": by, "hbm_gbs": by / (ms * 1e-3) / 1e9}
    from mamba2_jax.models import Mamba2Config, Mamba2LMHeadModel, init_params
    from mamba2_jax.models.mamba2_lm import DecodeState
    shapes = {"130m": Mamba2Config(d_model=768, n_layer=24, vocab_size=50277),
              "2.7b": Mamba2Config(d_model=2560, n_layer=64, vocab_size=50277)}
    for name in lm_configs:
        cfg = shapes[name]
        params = init_params(cfg, dtype=torch.bfloat16, device=dev)
        m = Mamba2LMHeadModel(cfg)
        for bsz in (1, 16, 64):
            state = DecodeState(cfg, bsz, dev)
            ids = torch.randint(0, cfg.vocab_size, (bsz, 32), device=dev)
            m.prefill(params, ids, state)
            gr, tok, _ = m.capture_decode(params, state)
            tok.copy_(ids[:, -1])
            for _ in range(3):
                gr.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(50):
                gr.replay()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 50
            out[f"lm_decode_{name}_b{bsz}"] = {
                "workload": f"Mamba2 LM {name} shape (d_model {cfg.d_model}, {cfg.n_layer} "
                            f"layers), bf16 weights, batch {bsz}, one token per step, HIP graph",
                "ms_per_token_step": ms, "tokens_per_s": bsz / (ms * 1e-3)}
            del gr, state
        del params
    return out


def bench_fp32_same_shape(cfg, name="c2", steps=100, warmup=50):
    """The configuration's shape with fp32 inputs (the reference's published
    numbers are fp32 runs at the nemotron-h-8b shape, README.md:35): ms per
    layer, tokens/s, the per-kernel table with its dominant kernel's roofline.
    The event pass (300 layers) brings the GPU to its steady clocks first."""
    import dataclasses
    c32 = dataclasses.replace(cfg, dtype="f32")
    kw = _layer_inputs(c32)
    nev = 300
    finish = stage_table_enqueue(c32, kw, nev, stage_events(c32, nev))
    ms, _ = time_layer(kw, steps, warmup)
    stages, dom, roof, _, tot_by = finish()
    attach_traffic(roof, measured_traffic(f"{name}_f32"), dom)
    del kw
    return {"workload": f"{cfg.name} shape, fp32 inputs", "ms_per_layer": ms,
            "tokens_per_s": c32.tokens / (ms * 1e-3),
            "layer_hbm_frac": tot_by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "roofline": roof, "stages": stages}


def bench_stage_operators(cfg, calls=10, replays=5):
    """Each stage operator of the reference's API called on its own at the
    configuration's shape, as the reference's staged pipeline chains them
    (kernels/ssd_combined.py:112-170): chunk_cumsum, chunk_state (float32
    states), state_passing (float32 in, C's dtype out), bmm_chunk (float32 CB),
    chunk_scan.  Per operator: GPU time from HIP-graph replays and its
    compulsory HBM bytes (inputs read once, outputs written once)."""
    import torch
    from mamba2_jax import configs
    from mamba2_jax.kernels.bmm_chunk_fwd import bmm_chunk_fwd
    from mamba2_jax.kernels.chunk_cumsum_fwd import chunk_cumsum_fwd
    from mamba2_jax.kernels.chunk_scan_fwd import chunk_scan_fwd
    from mamba2_jax.kernels.chunk_state_fwd import chunk_state_fwd
    from mamba2_jax.kernels.state_passing_fwd import state_passing_fwd
    d = configs.make_ssd_inputs(cfg)
    dev = torch.device("cuda")
    T = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    t = lambda a, dt=None: torch.from_numpy(a).to(dev).to(dt or torch.float32)
    x, dt, B, C = t(d["x"], T), t(d["dt"], T), t(d["B"], T), t(d["C"], T)
    A, D, bias = t(d["A"]), t(d["D"]), t(d["dt_bias"])
    Q, (b, L, H, P), (G, N) = cfg.chunk_size, x.shape, B.shape[2:]
    nc = -(-L // Q)
    dA, dto = chunk_cumsum_fwd(dt, A, Q, dt_bias=bias, dt_softplus=True)
    st = chunk_state_fwd(x, B, dto, dA)
    passed = state_passing_fwd(st.view(b, nc, H, P * N), dA[:, :, :, -1], chunk_size=Q,
                               out_dtype=C.dtype)[0].view(b, nc, H, P, N)
    cb = bmm_chunk_fwd(C, B, Q, output_dtype=torch.float32)
    s = x.element_size()
    ops = {
        "chunk_cumsum": (lambda: chunk_cumsum_fwd(dt, A, Q, dt_bias=bias, dt_softplus=True),
                         b * L * H * s + 2 * 4 * b * H * nc * Q),
        "chunk_state": (lambda: chunk_state_fwd(x, B, dto, dA),
                        b * L * H * P * s + b * L * G * N * s + 2 * 4 * b * H * nc * Q
                        + 4 * b * nc * H * P * N),
        "state_passing": (lambda: state_passing_fwd(st.view(b, nc, H, P * N), dA[:, :, :, -1],
                                                    chunk_size=Q, out_dtype=C.dtype),
                          4 * b * nc * H * P * N + 4 * b * H * nc + s * b * nc * H * P * N
                          + 4 * b * H * P * N),
        "bmm_chunk": (lambda: bmm_chunk_fwd(C, B, Q, output_dtype=torch.float32),
                      2 * b * L * G * N * s + 4 * b * nc * G * Q * Q),
        "chunk_scan": (lambda: chunk_scan_fwd(cb, x, dto, dA, C, passed, D=D),
                       4 * b * nc * G * Q * Q + b * L * H * P * s + 2 * 4 * b * H * nc * Q
                       + b * L * G * N * s + s * b * nc * H * P * N + 4 * b * L * H * P),
    }
    out = {}
    for name, (fn, by) in ops.items():
        ms = _graph_time_ms(fn, calls, replays)
        out[name] = {"ms": ms, "bytes": by, "hbm_gbs": by / ms / 1e6,
                     "hbm_frac": by / ms / 1e6 / PEAK_HBM_GBS}
    return out


def _layer_inputs(cfg):
    """Synthetic inputs of a configuration, resident on the GPU, as keyword
    arguments of mamba_chunk_scan_combined_fwd."""
    import torch
    from mamba2_jax import configs
    d = configs.make_ssd_inputs(cfg)
    dev = torch.device("cuda")
    T = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    t = lambda a, dt=None: None if a is None else torch.from_numpy(a).to(dev).to(dt or torch.float32)
    return dict(x=t(d["x"], T), dt=t(d["dt"], T), A=t(d["A"]), B=t(d["B"], T), C=t(d["C"], T),
                D=t(d["D"]), dt_bias=t(d["dt_bias"]), initial_states=t(d["initial_states"]),
                seq_idx=None if d["seq_idx"] is None else torch.from_numpy(d["seq_idx"]).to(dev),
                cu_seqlens=None if d["cu_seqlens"] is None else torch.from_numpy(d["cu_seqlens"]).to(dev),
                chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
                return_varlen_states=d["cu_seqlens"] is not None)


def time_layer(kw, steps, warmup):
    """(ms per layer, wall ms per step): `warmup` untimed calls, then `steps`
    back-to-back calls with events only around them, synchronised on both sides."""
    import torch
    from mamba2_jax.kernels import mamba_chunk_scan_combined_fwd
    for _ in range(warmup):
        mamba_chunk_scan_combined_fwd(**kw)
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    g0.record()
    for _ in range(steps):
        mamba_chunk_scan_combined_fwd(**kw)
    g1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    return g0.elapsed_time(g1) / steps, wall / steps * 1e3


def stage_table(cfg, kw, steps):
    """Per-kernel times of the combined path: `steps` calls with HIP events
    recorded on the launch stream at every kernel boundary (a fused kernel's
    time lands in the first slot of its group; the other slots of the group are
    not recorded).  -> (stages dict, dominant stage, its roofline dict, total
    ms with events, algorithmic bytes of the layer)."""
    return stage_table_enqueue(cfg, kw, steps)()


def stage_table_enqueue(cfg, kw, steps, events=None):
    """stage_table in two halves: this enqueues the calls and returns a
    function that waits for them and computes the table, so that other GPU
    work can be enqueued in between without the GPU going idle.  `events`:
    the result of stage_events(cfg, steps), made beforehand (creating them
    takes host time during which the GPU would idle)."""
    from mamba2_jax.kernels import mamba_chunk_scan_combined_fwd
    hev, evs, keep, fs, fc = events or stage_events(cfg, steps)
    for _ in range(3):
        mamba_chunk_scan_combined_fwd(**kw, _stage_events=evs[0])
    for i in range(steps):
        mamba_chunk_scan_combined_fwd(**kw, _stage_events=evs[i])
    return lambda: _stage_table_finish(cfg, kw, steps, hev, evs, keep, fs, fc)


def stage_events(cfg, steps):
    """The HIP events of a stage_table pass of `steps` calls (host side only)."""
    import dataclasses
    hev = HipEvents()
    icfg = dataclasses.replace(cfg, chunk_size=internal_chunk(cfg))
    fs, fc = states_is_fused(icfg), scan_is_fused(icfg)
    fcs, fpb = cumsum_in_state(icfg), pass_bmm_fused(icfg)
    keep = [True, not fcs, True, not (fs or fpb), not fc, True, cfg.nseq > 0]
    evs = [[hev.new() if k else None for k in keep] for _ in range(steps)]
    return hev, evs, keep, fs, fc


def _stage_table_finish(cfg, kw, steps, hev, evs, keep, fs, fc):
    import numpy as np
    import torch
    torch.cuda.synchronize()

    # the library records the events in stream order `order` (with bf16 and
    # the fused scan the varlen states run right after state_passing: event 6
    # comes before events 4 and 5)
    order = [0, 1, 2, 3, 6, 4, 5] if keep[6] and fc and cfg.dtype == "bf16" else [0, 1, 2, 3, 4, 5, 6]
    rec = [e for e in order if keep[e]]

    def slot(e):
        # the interval ending at event e: from the last recorded event before it
        if not keep[e]:
            return 0.0
        a = rec[rec.index(e) - 1]
        return float(np.mean([hev.elapsed_ms(evs[i][a], evs[i][e]) for i in range(steps)]))
    slot_ms = [slot(e) for e in range(1, 7 if keep[6] else 6)]
    last = rec[-1]
    total = float(np.mean([hev.elapsed_ms(evs[i][0], evs[i][last]) for i in range(steps)]))
    cu = kw.get("cu_seqlens")
    work = stage_work(cfg, with_init=kw["initial_states"] is not None,
                      cu_seqlens=None if cu is None or not keep[6] else cu.cpu().tolist())
    slots = dict(zip(STAGES, slot_ms))
    if fs:
        first = {"chunk_cumsum": slots["chunk_cumsum"], FUSED_STATES: slots["chunk_state"]}
    elif not keep[1]:
        first = {FUSED_CUMSUM: slots["chunk_state"], "state_passing": slots["state_passing"]}
    else:
        first = {k: slots[k] for k in STAGES[:3]}
    if fc:
        second = {"bmm_chunk+chunk_scan": slots["chunk_scan"]}
    else:
        second = {k: slots[k] for k in STAGES[3:]}
    if not fs and not keep[3]:
        # state_passing and bmm_chunk in one launch (its time: the bmm interval)
        first.pop("state_passing")
        first[FUSED_PASS_BMM] = second.pop("bmm_chunk")
    stage_ms = {**first, **second}
    if keep[6]:
        stage_ms[VARLEN] = slot_ms[5]
    peak_mfma = PEAK_MFMA_TFLOPS[cfg.dtype]
    stages = {}
    for s in stage_ms:
        by, fl = work[s]
        sec = stage_ms[s] * 1e-3
        stages[s] = {"ms": stage_ms[s], "bytes": by, "gflop": fl / 1e9,
                     "hbm_gbs": by / sec / 1e9, "hbm_frac": by / sec / 1e9 / PEAK_HBM_GBS,
                     "mfma_tflops": fl / sec / 1e12, "mfma_frac": fl / sec / 1e12 / peak_mfma}
    dom = max(stage_ms, key=lambda s: stage_ms[s])
    by, fl = work[dom]
    ridge = peak_mfma * 1e12 / (PEAK_HBM_GBS * 1e9)
    if fl / by > ridge:
        roof = {"bound": "mfma", "achieved": stages[dom]["mfma_tflops"], "peak": peak_mfma,
                "unit": "TFLOP/s", "frac": stages[dom]["mfma_frac"]}
    else:
        roof = {"bound": "hbm", "achieved": stages[dom]["hbm_gbs"], "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": stages[dom]["hbm_frac"]}
    roof.update({"kernel": dom, "algorithmic_bytes": by, "algorithmic_flop": fl,
                 "avg_launch_ms": stage_ms[dom]})
    del hev
    return stages, dom, roof, total, sum(w[0] for w in work.values())


def bench_other_config(name, steps=200, warmup=20, cpu=True):
    """One more BASELINE configuration measured in the same run: ms per layer,
    tokens/s, the per-kernel table with its dominant kernel's roofline, and a
    sampled CPU baseline."""
    from mamba2_jax import configs
    cfg = configs.CONFIGS[name]
    kw = _layer_inputs(cfg)
    # the event pass first: it brings the GPU back to its steady clocks after
    # the host-side input generation, which takes ~30 ms of continuous work;
    # >= 300 steps and >= 40 ms by a short timing first (a small layer such as
    # c0's, ~35 us, needs ~1100 steps)
    est, _ = time_layer(kw, 20, 5)
    nev = max(steps, 300, int(40.0 / max(est, 1e-3)))
    finish = stage_table_enqueue(cfg, kw, nev, stage_events(cfg, nev))
    ms, _ = time_layer(kw, steps, warmup)
    stages, dom, roof, _, tot_by = finish()
    attach_traffic(roof, measured_traffic(name), dom)
    out = {"workload": f"{cfg.name} SSD layer forward ({name})", "dtype": cfg.dtype,
           "batch": cfg.batch, "seq_len": cfg.seqlen, "nheads": cfg.nheads,
           "ngroups": cfg.ngroups, "headdim": cfg.headdim, "dstate": cfg.dstate,
           "chunk_size": cfg.chunk_size, "steps": steps, "warmup": warmup,
           "ms_per_layer": ms, "tokens_per_s": cfg.tokens / (ms * 1e-3),
           "layer_hbm_frac": tot_by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
           "roofline": roof, "stages": stages}
    del kw
    return out


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--dtype", choices=("f32", "bf16"), default=None,
                    help="run --config with these input dtypes (default: the config's own)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations (c0, c1, c3) and the c2 extras")
    ap.add_argument("--event-steps", type=int, default=300,
                    help="steps of the per-kernel event pass (at least --steps)")
    ap.add_argument("--stage-ops", action="store_true",
                    help="instead of the layer: time each stage operator at --config (one JSON line)")
    ap.add_argument("--cpu-heads", type=int, default=0,
                    help="heads of the CPU baseline sample (0: all heads for c2)")
    ap.add_argument("--ops", action="store_true",
                    help="instead of the SSD layer: time the ops around it and the LM decode "
                         "step (one JSON line)")
    ap.add_argument("--lm", default="130m", help="LM shapes for --ops (comma list: 130m,2.7b)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="run one device copy of this many MiB first (HBM counter calibration)")
    args = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): "
              "this build has no multi-GPU path; the SSD forward shards by head groups with no "
              "communication, so per-GPU throughput is the one-GPU figure.", file=sys.stderr)
        return 2

    if args.ops:
        print(json.dumps({"ops": bench_ops(tuple(x for x in args.lm.split(",") if x))}))
        return 0

    import torch
    from mamba2_jax import configs

    cfg = configs.CONFIGS[args.config]
    own_dtype = args.dtype is None or args.dtype == cfg.dtype
    if not own_dtype:
        import dataclasses
        cfg = dataclasses.replace(cfg, dtype=args.dtype)
    if args.stage_ops:
        print(json.dumps({"stage_operators": bench_stage_operators(cfg), "config": args.config}))
        return 0
    dev = torch.device("cuda")
    kw = _layer_inputs(cfg)
    K = args.steps
    nev = max(K, args.event_steps)
    events = stage_events(cfg, nev)
    res_extra = {}
    # The other measurements run first and the headline follows them with no
    # idle gap: besides their own figures they keep the GPU at its steady
    # clocks, which an idle GPU drops (measured at the headline shape: 0.126 ms
    # per layer after 5 warm-up steps on an idle GPU, 0.107 ms when busy).
    if args.config == "c2" and own_dtype and not args.no_configs:
        res_extra["configs"] = {c: bench_other_config(c) for c in ("c0", "c1", "c3")}
        res_extra["fp32_same_shape"] = bench_fp32_same_shape(cfg, args.config)
        res_extra["stage_operators"] = bench_stage_operators(cfg)
    if not args.no_decode:
        res_extra["decode"] = bench_decode()
    if args.copy_mb:
        # a plain copy of known size: reads and writes copy_mb MiB once each
        src = torch.ones(args.copy_mb << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # the per-kernel table: max(K, 300) steps (--event-steps) with HIP events at kernel
    # boundaries (~35 ms of the workload, which brings the GPU to its steady
    # clocks); its events are read after the timed region, so the GPU does not
    # idle between the two
    finish = stage_table_enqueue(cfg, kw, nev, events)
    # timed region (value): W warm-up steps, then K back-to-back steps
    ms, wall_ms = time_layer(kw, K, args.warmup)
    stages, dom, roof, stages_ms_total, tot_by = finish()
    # measured traffic is kept for each config at its own dtype
    attach_traffic(roof, measured_traffic(args.config) if own_dtype else {}, dom)
    res = {
        "metric": METRIC, "value": cfg.tokens / (ms * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg.dtype, "data": "synthetic",
        "config": {"workload": f"{cfg.name} SSD layer forward ({args.config}"
                               f"{'' if own_dtype else ', ' + cfg.dtype + ' inputs'})",
                   "batch": cfg.batch, "seq_len": cfg.seqlen, "nheads": cfg.nheads,
                   "ngroups": cfg.ngroups, "headdim": cfg.headdim, "dstate": cfg.dstate,
                   "chunk_size": cfg.chunk_size, "parallelism": "single-gpu"},
        "ms_per_layer": ms, "wall_ms_per_step": wall_ms,
        "ms_per_layer_with_stage_events": stages_ms_total,
        "layer_hbm_frac": tot_by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "roofline": roof, "stages": stages,
        "reference_published": {"hardware": "H100", "dtype": "fp32", "pallas_ms": 0.94,
                                "triton_ms": 0.69, "source": "reference README.md:35"},
    }
    res.update(res_extra)
    del kw
    torch.cuda.synchronize()
    # CPU baselines last (host only): the full c2 workload, bounded samples of the others
    if not args.no_cpu_baseline:
        full = args.config == "c2" and own_dtype and args.cpu_heads == 0
        res["cpu_baseline"] = cpu_baseline(cfg, cfg.nheads if full else (args.cpu_heads or 32))
        for c, sample_heads in (("c0", 24), ("c1", 16), ("c3", 32)):
            if c in res.get("configs", {}):
                res["configs"][c]["cpu_baseline"] = cpu_baseline(configs.CONFIGS[c], sample_heads,
                                                                 min_seconds=3.0)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())

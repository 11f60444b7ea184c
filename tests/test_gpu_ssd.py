"""Parity of the whole SSD forward (mamba_chunk_scan_combined_fwd) on the GPU.

* against the CPU oracle (float64) at the benchmark shapes: c0, c1 and c2 in
  full, c3 in full one head group at a time (heads are independent) and with
  fewer heads or tokens;
* at the full c1 / c3 sizes through size-independent properties: agreement
  with the naive formulation run on the GPU (c1) and packed == per-sequence
  runs (c3);
* chunk-size invariance, L % Q != 0, D per head-dim, z gate, dispatch.
Tolerance: max|err|/rms <= 1e-3 (fp32 inputs), 2e-2 (bf16), outputs and
final states alike.
"""

import dataclasses

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, host, tdtype
from mamba2_jax import _lib as L
from mamba2_jax import configs
from mamba2_jax.kernels import mamba_chunk_scan_combined_fwd
from mamba2_jax.modules.mamba2 import _ssd_combined_fwd
from mamba2_jax.ops import mamba_chunk_scan_combined_naive
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu


def _dev_inputs(d, dtype):
    T = tdtype(dtype)
    return dict(x=dev(d["x"], T), dt=dev(d["dt"], T), A=dev(d["A"]), B=dev(d["B"], T),
                C=dev(d["C"], T), D=dev(d["D"]), z=dev(d["z"], T), dt_bias=dev(d["dt_bias"]),
                initial_states=dev(d["initial_states"]), seq_idx=dev(d["seq_idx"]),
                cu_seqlens=dev(d["cu_seqlens"]))


def _run_and_check(cfg, with_z=False, varlen=False, Dhp=False):
    d = configs.make_ssd_inputs(cfg, with_z=with_z)
    if Dhp:
        d["D"] = np.random.default_rng(1).uniform(0.5, 1.5, (cfg.nheads, cfg.headdim)).astype(np.float32)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
              return_varlen_states=varlen)
    got = mamba_chunk_scan_combined_fwd(**_dev_inputs(d, cfg.dtype), **kw)
    want = O.ssd_combined(io_dtype=cfg.dtype, **d, **kw)
    tol = TOL[cfg.dtype]
    check(got[0], want[0], tol, "out")
    check(got[1], want[1], tol, "final_states")
    if varlen:
        check(got[2], want[2], tol, "varlen_states")
    assert got[0].dtype == torch.float32 and got[1].dtype == torch.float32


@pytest.mark.parametrize("Q", [64, 128])
def test_increasing_decay(Q):
    """dt' of both signs (no softplus, dt_limit below 0), so dA_cumsum rises and
    falls within chunks: the fused scan takes its direct-weight path.  The
    chunk-state decay is clamped at 0 as in the reference's chunk_state kernel
    (kernels/chunk_state_fwd.py:251); the scan decay is not
    (kernels/chunk_scan_fwd.py:329, ops/ssd_naive.py:260-268)."""
    announce("increasing decay, Q", Q)
    cfg = dataclasses.replace(configs.CONFIGS["c2"], seqlen=512, nheads=16, ngroups=2)
    d = configs.make_ssd_inputs(cfg)
    # mostly positive steps with some negative ones: dA still rises within
    # chunks, while exp(dA) stays near 1 (a rising dA would amplify the bf16
    # rounding of C h_c, a rounding point of the reference, beyond the
    # tolerance)
    rng = np.random.default_rng(21)
    sign = np.where(rng.random(d["dt"].shape) < 0.15, -1.0, 1.0)
    d["dt"] = O.bf16_round(0.05 * np.abs(rng.standard_normal(d["dt"].shape)) * sign).astype(np.float32)
    d["dt_bias"] = None
    kw = dict(chunk_size=Q, dt_softplus=False, dt_limit=(-1.0, float("inf")),
              return_final_states=True)
    got = mamba_chunk_scan_combined_fwd(**_dev_inputs(d, cfg.dtype), **kw)
    want = O.ssd_combined(io_dtype=cfg.dtype, decay_clamp=True, **d, **kw)
    dA, _ = O.chunk_cumsum(d["dt"], d["A"], Q, None, False, (-1.0, float("inf")))
    assert np.any(np.diff(dA, axis=-1) > 0) and np.any(np.diff(dA, axis=-1) < 0)
    check(got[0], want[0], TOL[cfg.dtype], "out")
    check(got[1], want[1], TOL[cfg.dtype], "final_states")


@pytest.mark.parametrize("H,G,Q,dt_f32", [(5, 1, 128, False), (6, 2, 64, True), (3, 3, 128, True)])
def test_odd_heads_fp32_dt(H, G, Q, dt_f32):
    """Head counts with odd (t H + h) parity (the bf16 dt word read in halves)
    and fp32 dt beside bf16 x / B / C; L % Q != 0."""
    announce("odd heads / fp32 dt", H, G, Q, dt_f32)
    cfg = dataclasses.replace(configs.CONFIGS["c2"], seqlen=333, nheads=H, ngroups=G, chunk_size=Q)
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, cfg.dtype)
    if dt_f32:
        t["dt"] = dev(d["dt"])
    kw = dict(chunk_size=Q, dt_softplus=True, return_final_states=True)
    got = mamba_chunk_scan_combined_fwd(**t, **kw)
    want = O.ssd_combined(io_dtype=cfg.dtype, **d, **kw)
    check(got[0], want[0], TOL[cfg.dtype], "out")
    check(got[1], want[1], TOL[cfg.dtype], "final_states")


def test_c0_full_fp32():
    announce("c0 full")
    _run_and_check(configs.CONFIGS["c0"])


def test_c0_shape_fp32_batch2():
    """The c0 shape at batch 2: chunk and passed states of 24 MiB, above the
    16 MiB up to which they are stored non-temporally (c0 itself: 12 MiB), so
    the ordinary-store forms of the fp32 chunk_state and state walk run."""
    announce("c0 shape fp32 batch 2")
    _run_and_check(dataclasses.replace(configs.CONFIGS["c0"], batch=2))


def test_c2_shape_fp32_full():
    """The nemotron-h-8b shape in fp32 (the reference's published conditions):
    x and the passed states (256 MiB) exceed what the group scan stores its
    output non-temporally for, so its ordinary-store form runs, after the
    fused fp32 state pass."""
    announce("c2 shape fp32 full")
    _run_and_check(dataclasses.replace(configs.CONFIGS["c2"], dtype="f32"))


def test_c2_full_headline():
    announce("c2 full (nemotron-h-8b, headline)")
    _run_and_check(configs.CONFIGS["c2"])


def test_c1_fewer_tokens():
    announce("c1 b=2 L=512")
    _run_and_check(dataclasses.replace(configs.CONFIGS["c1"], batch=2, seqlen=512))


def test_c3_fewer_heads_and_tokens_varlen():
    announce("c3 L=2048 H=32 varlen")
    cfg = dataclasses.replace(configs.CONFIGS["c3"], seqlen=2048, nheads=32, min_seqlen=64)
    _run_and_check(cfg, varlen=True)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gate_D_per_headdim_and_ragged_length(dtype):
    announce("z + D[H,P] + L%Q", dtype)
    cfg = configs.SSDConfig("ragged", 2, 333, 16, 4, 64, 64, 128, dtype, init_state=True, seed=21)
    _run_and_check(cfg, with_z=True, Dhp=True)


@pytest.mark.parametrize("case", ["b2_init_ragged", "packed"])
def test_dstate256_chunk128_gate(case):
    """bf16, dstate 256, chunk 128, head dim 64: the scan kernel whose compute
    wavefronts stage and store their own output tiles, here with the z gate
    applied before the staging, D per head dim, a ragged last chunk (rows past
    it staged but not stored), an initial state / packed sequences."""
    announce("dstate 256 chunk 128 with z", case)
    if case == "b2_init_ragged":
        cfg = configs.SSDConfig("n256z", 2, 3 * 128 + 45, 8, 2, 64, 256, 128, "bf16",
                                init_state=True, seed=61)
    else:
        cfg = configs.SSDConfig("n256z", 1, 1000, 8, 4, 64, 256, 128, "bf16", nseq=4,
                                min_seqlen=100, seed=62)
    _run_and_check(cfg, with_z=True, Dhp=True, varlen=cfg.nseq > 0)


def test_headdim_128_dstate_256_chunk_64():
    announce("P=128 N=256 Q=64")
    cfg = configs.SSDConfig("wide", 1, 256, 8, 2, 128, 256, 64, "bf16", seed=22)
    _run_and_check(cfg)


def test_c1_full_vs_oracle():
    """Full c1 (batch 4, L 2048, 80 heads, chunk 256, initial state) against the
    CPU oracle."""
    announce("c1 full vs oracle")
    _run_and_check(configs.CONFIGS["c1"])


def test_c1_full_vs_naive_on_gpu():
    """Full c1 (with initial state) against the naive formulation in float32 on the GPU."""
    announce("c1 full vs naive")
    cfg = configs.CONFIGS["c1"]
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, cfg.dtype)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True)
    y, f = mamba_chunk_scan_combined_fwd(**t, **kw)
    t.pop("seq_idx"), t.pop("cu_seqlens")
    yn, fn = mamba_chunk_scan_combined_naive(**t, **kw)
    check(y, host(yn), TOL["bf16"], "out")
    check(f, host(fn), TOL["bf16"], "final_states")


def test_c3_full_packed_equals_per_sequence():
    """Full c3: the packed run equals independent runs of each sequence."""
    announce("c3 full packed vs per-sequence")
    cfg = configs.CONFIGS["c3"]
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, cfg.dtype)
    y, fin, vs = mamba_chunk_scan_combined_fwd(
        chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
        return_varlen_states=True, **t)
    cu = d["cu_seqlens"]
    errs = []
    for s in range(cfg.nseq):
        sl = slice(int(cu[s]), int(cu[s + 1]))
        part = {k: (v[:, sl].contiguous() if k in ("x", "dt", "B", "C") else v)
                for k, v in t.items() if k not in ("seq_idx", "cu_seqlens", "z", "initial_states")}
        ys, fs = mamba_chunk_scan_combined_fwd(chunk_size=cfg.chunk_size, dt_softplus=True,
                                               return_final_states=True, **part)
        errs.append(check(y[:, sl], host(ys), TOL["bf16"], f"seq {s} out"))
        # The packed varlen state adds exp(dA) * (state entering its last chunk)
        # taken from the bf16 states_passed, as the reference does
        # (kernels/ssd_combined.py:176-183): one bf16 rounding of that term.
        _within_bf16_ulp(vs[s], fs[0], f"seq {s} varlen state")
    _within_bf16_ulp(fin[0], vs[-1], "final == last varlen state")


@pytest.fixture(scope="module")
def c3_full_run():
    """The full c3 forward (L 8192, 256 heads in 8 groups, dstate 256, six
    packed sequences) on the GPU once, through the C ABI with a workspace of
    the test's own, so that the states entering each chunk (bf16, the slot after
    dA_cumsum, dt', the weights and the chunk decay of the fused state pass)
    can be read back; host copies of everything."""
    import ctypes
    cfg = configs.CONFIGS["c3"]
    d = configs.make_ssd_inputs(cfg)
    t = {k: (v.contiguous() if v is not None else None) for k, v in _dev_inputs(d, cfg.dtype).items()}
    b, Lq, H, P = t["x"].shape
    N, Q, nseq = cfg.dstate, cfg.chunk_size, cfg.nseq
    nc = -(-Lq // Q)
    y = torch.empty((b, Lq, H, P), dtype=torch.float32, device="cuda")
    fin = torch.empty((b, H, P, N), dtype=torch.float32, device="cuda")
    vs = torch.empty((nseq, H, P, N), dtype=torch.float32, device="cuda")
    a = L.SsdCombinedArgs(
        x=L.ptr(t["x"]), dt=L.ptr(t["dt"]), A=L.ptr(t["A"]), B=L.ptr(t["B"]), C=L.ptr(t["C"]),
        D=L.ptr(t["D"]), dt_bias=L.ptr(t["dt_bias"]), seq_idx=L.ptr(t["seq_idx"]),
        cu_seqlens=L.ptr(t["cu_seqlens"]), out=L.ptr(y), final_states=L.ptr(fin),
        varlen_states=L.ptr(vs), batch=b, seqlen=Lq, nheads=H, headdim=P, ngroups=cfg.ngroups,
        dstate=N, chunk_size=Q, nseq=nseq, dtype=L.M2_BF16, dt_dtype=L.M2_BF16, dt_softplus=1,
        dt_min=0.0, dt_max=float("inf"))
    lib = L.load_library()
    need = lib.m2_ssd_combined_workspace_size(ctypes.byref(a))
    al = lambda v: (v + 255) // 256 * 256
    cq = b * H * nc * Q
    off = 3 * al(4 * cq) + al(4 * b * H * nc)            # dA_cumsum, dt', weights, decay
    S = b * nc * H * P * N
    assert need == off + al(2 * S), "workspace layout of the fused bf16 path"
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    a.workspace, a.workspace_bytes = ws.data_ptr(), need
    L.call("m2_ssd_combined", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    passed = ws[off:off + 2 * S].view(torch.bfloat16).view(b, nc, H, P, N)
    host32 = lambda v: v.detach().float().cpu().numpy()
    return cfg, d, host32(y), host32(fin), host32(vs), host32(passed)


@pytest.mark.parametrize("g", range(configs.CONFIGS["c3"].ngroups))
def test_c3_full_vs_oracle_by_group(c3_full_run, g):
    """Full c3 against the oracle, one head group at a time: the heads of a
    group (with its B / C) are independent of every other head, so the oracle
    evaluated on group g's 32 heads is exactly the full problem's result for
    them.  At the plain bf16 bar: outputs, final states and the varlen states;
    the states entering each chunk (bf16) within one bf16 step of the oracle's
    (plus fp32 summation order), element by element.  The varlen states add exp(dA) * (the
    state entering the sequence's last chunk, rounded to bf16) -- a rounding
    point of the reference (kernels/ssd_combined.py:140,
    kernels/chunk_state_fwd.py:587-595) where one rounding flip, decided by
    fp32 summation order, can move a large state by more than the bar -- so
    they are compared with the oracle's chunk_state_varlen fed the states the
    GPU rounded (the same rounding decisions on both sides)."""
    cfg, d, y, fin, vs, passed = c3_full_run
    announce("c3 full vs oracle, group", g)
    hpg = cfg.nheads // cfg.ngroups
    hs = slice(g * hpg, (g + 1) * hpg)
    dg = dict(d, x=d["x"][:, :, hs], dt=d["dt"][:, :, hs], A=d["A"][hs], D=d["D"][hs],
              dt_bias=d["dt_bias"][hs], B=d["B"][:, :, g:g + 1], C=d["C"][:, :, g:g + 1])
    want = O.ssd_combined(io_dtype=cfg.dtype, chunk_size=cfg.chunk_size, dt_softplus=True,
                          return_final_states=True, return_varlen_states=True, **dg)
    tol = TOL[cfg.dtype]
    check(y[:, :, hs], want[0], tol, f"group {g} out")
    check(fin[:, hs], want[1], tol, f"group {g} final_states")
    dA, dto = O.chunk_cumsum(dg["dt"], dg["A"], cfg.chunk_size, dg["dt_bias"], True)
    st = O.chunk_state(dg["B"], dg["x"], dto, dA, seq_idx=d["seq_idx"])
    b, nc, Hg, P, N = st.shape
    sp, _ = O.state_passing(st.reshape(b, nc, Hg, P * N), dA[:, :, :, -1],
                            seq_idx=d["seq_idx"], chunk_size=cfg.chunk_size)
    # bf16 values rounded from fp32 sums of different order: element by
    # element equal or one bf16 step apart (2^-7 of the larger magnitude), on
    # top of the fp32 summation-order difference before the rounding (1e-5 of
    # the largest state)
    wp = O.bf16_round(sp).reshape(b, nc, Hg, P, N).astype(np.float64)
    gp = passed[:, :, hs].astype(np.float64)
    allow = 2.0 ** -7 * np.maximum(np.abs(gp), np.abs(wp)) + 1e-5 * np.abs(wp).max()
    excess = np.abs(gp - wp) / allow
    print(f"  group {g} states entering each chunk: {np.mean(gp != wp):.2e} of them differ, "
          f"max |diff| / (one bf16 step + 1e-5 max) = {excess.max():.3f} (tol 1)", flush=True)
    assert excess.max() <= 1.0
    wv = O.chunk_state_varlen(dg["B"][0], dg["x"][0], dto[0], dA[0], d["cu_seqlens"],
                              passed[0][:, hs])
    check(vs[:, hs], wv, tol, f"group {g} varlen_states")
    e = O.rel_err(vs[:, hs], want[2])
    print(f"  group {g} varlen_states vs the oracle's own rounding: {e:.3e}", flush=True)


def _within_bf16_ulp(got, want, what):
    g, w = host(got), host(want)
    e = float(np.max(np.abs(g - w)) / np.max(np.abs(w)))
    print(f"  {what}: max|err|/max|ref| = {e:.3e} (tol 2^-8)", flush=True)
    assert e <= 2.0 ** -8, f"{what}: {e:.3e}"


def test_chunk_size_invariance():
    announce("chunk-size invariance")
    cfg = dataclasses.replace(configs.CONFIGS["c2"], seqlen=1024)
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, cfg.dtype)
    outs = [mamba_chunk_scan_combined_fwd(chunk_size=q, dt_softplus=True,
                                          return_final_states=True, **t) for q in (64, 128, 256)]
    for y, f in outs[1:]:
        check(y, host(outs[0][0]), TOL["bf16"], "out")
        check(f, host(outs[0][1]), TOL["bf16"], "final")


def test_return_arity_and_dispatch():
    announce("arity + dispatch")
    cfg = configs.SSDConfig("small", 1, 256, 8, 2, 64, 64, 64, "f32", nseq=2, min_seqlen=64, seed=3)
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, "f32")
    y = mamba_chunk_scan_combined_fwd(chunk_size=64, **t)
    assert isinstance(y, torch.Tensor)
    r = mamba_chunk_scan_combined_fwd(chunk_size=64, return_varlen_states=True, **t)
    assert len(r) == 2 and r[1].shape == (2, 8, 64, 64)
    r = mamba_chunk_scan_combined_fwd(chunk_size=64, return_final_states=True,
                                      return_varlen_states=True, **t)
    assert len(r) == 3
    yd = _ssd_combined_fwd(use_pallas=True, chunk_size=64, **t)
    torch.testing.assert_close(yd, y, rtol=0, atol=0)
    t.pop("seq_idx"), t.pop("cu_seqlens")
    yn = _ssd_combined_fwd(use_pallas=False, chunk_size=64, **t)
    yh = _ssd_combined_fwd(use_pallas=True, chunk_size=64, **t)
    check(yh, host(yn), TOL["f32"], "hip vs naive")


# The fused state pass splits its work one of three ways, chosen from the
# shape (the states_split override forces one where the shape allows it): a head in
# 64-column halves, a pair of heads x 64 columns, a pair of heads x 128
# columns.  Each must match the oracle with an initial state, ragged lengths,
# batch > 1, sequence resets, dstate 64 / 128 / 256.
_SPLIT_CASES = {
    "init_b2": configs.SSDConfig("split", 2, 1024, 8, 2, 64, 128, 128, "bf16", init_state=True, seed=31),
    "ragged": configs.SSDConfig("split", 1, 5 * 128 - 37, 16, 4, 64, 128, 128, "bf16", seed=32),
    "n64_init": configs.SSDConfig("split", 1, 256, 8, 1, 64, 64, 128, "bf16", init_state=True, seed=33),
    "seq_resets": configs.SSDConfig("split", 1, 1536, 8, 2, 64, 128, 128, "bf16", nseq=5, min_seqlen=100, seed=34),
    "n256_init": configs.SSDConfig("split", 1, 768, 8, 2, 64, 256, 128, "bf16", init_state=True, seed=35),
}


@pytest.mark.parametrize("split", ["halves", "pair64", "pair128"])
@pytest.mark.parametrize("case", sorted(_SPLIT_CASES))
def test_state_pass_splits(case, split):
    announce("state-pass split", case, split)
    cfg = _SPLIT_CASES[case]
    d = configs.make_ssd_inputs(cfg)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True)
    t = _dev_inputs(d, cfg.dtype)
    t.pop("cu_seqlens")
    with L.dispatch_override("states_split", split):
        got = mamba_chunk_scan_combined_fwd(**t, **kw)
    d = dict(d, cu_seqlens=None)
    want = O.ssd_combined(io_dtype=cfg.dtype, **d, **kw)
    check(got[0], want[0], TOL[cfg.dtype], "out")
    check(got[1], want[1], TOL[cfg.dtype], "final_states")


@pytest.mark.parametrize("split", ["pair64", "pair128"])
def test_state_pass_pair_splits_varlen(split):
    """Packed sequences through the pair splits: outputs, final and varlen states."""
    announce("state-pass pair split, varlen", split)
    cfg = dataclasses.replace(configs.CONFIGS["c3"], seqlen=2048, nheads=32, min_seqlen=64)
    with L.dispatch_override("states_split", split):
        _run_and_check(cfg, varlen=True)


def test_state_pass_pair_splits_full_c3_nontemporal():
    """At the full c3 size the states entering each chunk (537 MB) exceed the
    256 MB Infinity Cache, so both head-pair kernels store them non-temporally
    through their LDS staging rows.  The two splits sum the same products in
    the same order, so their outputs, final and varlen states are bit-identical,
    and the launcher's own choice here (pair x 128 columns) gives the same."""
    announce("state-pass pair splits, full c3, non-temporal state stores")
    cfg = configs.CONFIGS["c3"]
    assert cfg.seqlen * cfg.nheads * cfg.headdim * cfg.dstate * 2 > 256 * 2**20
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, cfg.dtype)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
              return_varlen_states=True)
    auto = mamba_chunk_scan_combined_fwd(**t, **kw)
    for split in ("pair64", "pair128"):
        with L.dispatch_override("states_split", split):
            got = mamba_chunk_scan_combined_fwd(**t, **kw)
        for name, a, b in zip(("out", "final_states", "varlen_states"), got, auto):
            assert torch.equal(a, b), f"{split} {name}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_graph_replays_match_eager(dtype):
    """The combined forward captured in a HIP graph (fp32: the staged kernels,
    bf16: the fused ones).  Every replay (eager calls and synchronisations in
    between, outputs cleared first) equals the eager result bit for bit."""
    announce("combined forward graph replays", dtype)
    cfg = dataclasses.replace(configs.CONFIGS["c0"], seqlen=1000, dtype=dtype)
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, dtype)
    for k in ("cu_seqlens", "seq_idx", "z"):
        t.pop(k)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True)
    want = mamba_chunk_scan_combined_fwd(**t, **kw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mamba_chunk_scan_combined_fwd(**t, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y, fin = mamba_chunk_scan_combined_fwd(**t, **kw)
    for r in range(3):
        ye, fe = mamba_chunk_scan_combined_fwd(**t, **kw)
        torch.cuda.synchronize()
        assert torch.equal(ye, want[0]) and torch.equal(fe, want[1]), f"eager call {r}"
        y.fill_(float("nan"))
        fin.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want[0]), f"replay {r}: out"
        assert torch.equal(fin, want[1]), f"replay {r}: final_states"
    check(want[0], O.ssd_combined(io_dtype=dtype, **dict(d, cu_seqlens=None, seq_idx=None, z=None),
                                  **kw)[0], TOL[dtype], "out vs oracle")


_F32_WIDE_CASES = {
    # fp32 with >= 128 (chunk, group) blocks at chunk 128: the LDS-staged fp32
    # bmm_chunk and chunk_cumsum folded into the fp32 chunk_state kernel
    "c2_heads32": (dataclasses.replace(configs.CONFIGS["c2"], dtype="f32", nheads=32), {}),
    "n64_ragged_z_Dhdim": (dataclasses.replace(configs.CONFIGS["c2"], dtype="f32", seqlen=4000,
                                               nheads=16, ngroups=4, dstate=64),
                           dict(with_z=True, Dhp=True)),
    "packed_varlen": (dataclasses.replace(configs.CONFIGS["c3"], dtype="f32", seqlen=4096,
                                          nheads=32, dstate=128, min_seqlen=64),
                      dict(varlen=True)),
}


@pytest.mark.parametrize("case", sorted(_F32_WIDE_CASES))
def test_fp32_wide_shapes(case):
    announce("fp32 wide shape", case)
    cfg, kw = _F32_WIDE_CASES[case]
    _run_and_check(cfg, **kw)


@pytest.mark.parametrize("H,G,N,Q,L,packed", [
    (6, 2, 256, 64, 1000, True),     # 3 heads a group: one head per workgroup; 2 column blocks
    (8, 2, 128, 128, 777, False),    # head pairs, ragged length
    (4, 4, 256, 128, 640, True),     # one head a group
])
def test_fp32_cumsum_in_chunk_state(H, G, N, Q, L, packed):
    """fp32 with chunk_cumsum folded into the chunk_state kernel (dstate a
    multiple of 128, chunk 64 / 128): its dA_cumsum / dt' feed state passing
    and the scan; against the oracle, with D per head-dim and z."""
    announce("fp32 cumsum in chunk_state", H, G, N, Q, L, packed)
    cfg = configs.SSDConfig("f32cs", 1, L, H, G, 64, N, Q, "f32", nseq=3 if packed else 0,
                            min_seqlen=64, seed=H + N + L)
    _run_and_check(cfg, with_z=True, Dhp=True, varlen=packed)


# fp32 through the fused state pass (chosen from 256 workgroups up, forced by
# the f32_states override on these smaller shapes): initial states, batch > 1,
# ragged lengths, sequence resets with varlen states, dstate 64 / 256, chunk
# 64 and 256 (run as 128), z and D per head-dim
_F32_FUSED_CASES = {
    "init_b2": configs.SSDConfig("f32fs", 2, 1024, 8, 2, 64, 128, 128, "f32", init_state=True, seed=41),
    "ragged_q64": configs.SSDConfig("f32fs", 1, 5 * 64 - 19, 16, 4, 64, 128, 64, "f32", seed=42),
    "n64_init": configs.SSDConfig("f32fs", 1, 256, 8, 1, 64, 64, 128, "f32", init_state=True, seed=43),
    "seq_resets": configs.SSDConfig("f32fs", 1, 1536, 8, 2, 64, 128, 128, "f32", nseq=5, min_seqlen=100, seed=44),
    "n256_q256": configs.SSDConfig("f32fs", 1, 777, 8, 2, 64, 256, 256, "f32", init_state=True, seed=45),
}


@pytest.mark.parametrize("case", sorted(_F32_FUSED_CASES))
def test_fp32_fused_state_pass(case):
    announce("fp32 fused state pass", case)
    cfg = _F32_FUSED_CASES[case]
    with L.dispatch_override("f32_states", "fused"):
        _run_and_check(cfg, with_z=True, Dhp=True, varlen=cfg.nseq > 0)


# fp32 at chunk 128, head dim 64, dstate 64 / 128: the group scan builds CB
# itself (no bmm_chunk launch) after the fused state pass (forced by the
# f32_states override on these smaller shapes), and after the staged pass where
# bmm_chunk would be a launch of its own (>= 128 (chunk, group) blocks).  Each
# case against the oracle, and against the same layer with bmm_chunk and the
# per-(chunk, head) scan kernel (the f32_scan override), which computes CB and
# the products from the same bf16 triples
_F32_GROUP_CASES = {
    "packed_z_Dhp": (configs.SSDConfig("f32g", 1, 1200, 8, 2, 64, 128, 128, "f32", nseq=4,
                                       min_seqlen=100, seed=51),
                     dict(with_z=True, Dhp=True, varlen=True), "fused"),
    "b2_init_ragged": (configs.SSDConfig("f32g", 2, 777, 12, 3, 64, 128, 256, "f32", init_state=True,
                                         seed=52), dict(), "fused"),
    "n64_z": (configs.SSDConfig("f32g", 4, 640, 16, 2, 64, 64, 128, "f32", seed=53),
              dict(with_z=True), "fused"),
    "n64_packed": (configs.SSDConfig("f32g", 1, 900, 6, 1, 64, 64, 128, "f32", nseq=3,
                                     min_seqlen=64, seed=54), dict(varlen=True, Dhp=True), "fused"),
    "staged_256_blocks": (configs.SSDConfig("f32g", 2, 4096, 8, 4, 64, 128, 128, "f32", seed=55),
                          dict(with_z=True), None),
}


@pytest.mark.parametrize("case", sorted(_F32_GROUP_CASES))
def test_fp32_group_scan_builds_cb(case):
    announce("fp32 group scan with CB built in", case)
    cfg, kw, force = _F32_GROUP_CASES[case]
    states = L.dispatch_override("f32_states", force or "staged")
    with states:
        _run_and_check(cfg, **kw)
    d = configs.make_ssd_inputs(cfg, with_z=kw.get("with_z", False))
    if kw.get("Dhp"):
        d["D"] = np.random.default_rng(1).uniform(0.5, 1.5, (cfg.nheads, cfg.headdim)).astype(np.float32)
    ckw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
               return_varlen_states=kw.get("varlen", False))
    with L.dispatch_override("f32_states", force or "staged"):
        got = mamba_chunk_scan_combined_fwd(**_dev_inputs(d, "f32"), **ckw)
        with L.dispatch_override("f32_scan", "per_head"):
            ref = mamba_chunk_scan_combined_fwd(**_dev_inputs(d, "f32"), **ckw)
    check(got[0], host(ref[0]), 2e-5, "out, group scan vs bmm_chunk + per-head scan")
    assert torch.equal(got[1], ref[1])          # the state pass is the same kernel


def test_c2_full_fp32():
    """The headline shape with fp32 inputs (the reference's published
    conditions), where the fp32 fused state pass runs, against the oracle."""
    announce("c2 full, fp32")
    _run_and_check(dataclasses.replace(configs.CONFIGS["c2"], dtype="f32"))


def test_fp32_fused_state_pass_graph_replays():
    """The fp32 fused state pass inside a captured combined forward: replays
    equal the eager result bit for bit."""
    announce("fp32 fused state pass, graph replays")
    with L.dispatch_override("f32_states", "fused"):
        _fp32_fused_graph_replays()


def _fp32_fused_graph_replays():
    cfg = dataclasses.replace(configs.CONFIGS["c0"], seqlen=1000, init_state=True)
    d = configs.make_ssd_inputs(cfg)
    t = _dev_inputs(d, "f32")
    for k in ("cu_seqlens", "seq_idx", "z"):
        t.pop(k)
    kw = dict(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True)
    want = mamba_chunk_scan_combined_fwd(**t, **kw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mamba_chunk_scan_combined_fwd(**t, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y, fin = mamba_chunk_scan_combined_fwd(**t, **kw)
    for r in range(3):
        y.fill_(float("nan"))
        fin.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want[0]), f"replay {r}: out"
        assert torch.equal(fin, want[1]), f"replay {r}: final_states"
    ref = O.ssd_combined(io_dtype="f32", **dict(d, cu_seqlens=None, seq_idx=None, z=None), **kw)
    check(want[0], ref[0], TOL["f32"], "out vs oracle")
    check(want[1], ref[1], TOL["f32"], "final_states vs oracle")

"""Per-stage parity of the HIP kernels against the CPU oracle (float64).

Shapes replay the reference's own stage tests (tests/test_chunk_cumsum_and_state.py
:594-635, tests/test_state_passing_and_bmm.py:620-762,
tests/test_chunk_scan_and_varlen.py:797-853) with our seeded inputs, plus edge
cases (L % Q != 0, odd dims, bf16 and fp32).  Tolerances are the benchmark
contract's: max|err|/rms <= 1e-3 (fp32 inputs), 2e-2 (bf16 inputs); pure fp32
stages (cumsum, state passing) are held to 1e-5, bmm to 1e-5 for bf16 inputs and
1e-4 for fp32 inputs (fp32 operands run through the matrix cores as bf16 hi / lo
triples: ~2^-16 relative error per product).
"""

import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, dev, host, seq_idx_from_lengths, tdtype
from mamba2_jax import configs
from mamba2_jax.kernels import (bmm_chunk_fwd, chunk_cumsum_fwd, chunk_scan_fwd,
                                chunk_state_fwd, chunk_state_varlen_mosaic, state_passing_fwd)
from oracle import ssd_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(b, L, H, G, P, N, Q, dtype, seed, z=False, init=False):
    cfg = configs.SSDConfig("t", b, L, H, G, P, N, Q, dtype, init_state=init, seed=seed)
    return configs.make_ssd_inputs(cfg, with_z=z)


# ---------------------------------------------------------------------------
# chunk_cumsum
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("b,L,H,Q,dtype,limit", [
    (1, 128, 24, 64, "f32", (0.0, float("inf"))),
    (1, 256, 64, 256, "bf16", (0.0, float("inf"))),
    (2, 300, 40, 128, "bf16", (0.001, 0.1)),        # L % Q != 0, clamp
    (1, 4096, 128, 128, "bf16", (0.0, float("inf"))),
    # more than 512 workgroups of one chunk: two chunks per workgroup, an even
    # chunk count (c3's) and an odd one whose last workgroup has no second chunk
    (1, 8192, 256, 128, "bf16", (0.0, float("inf"))),
    (2, 3900, 160, 128, "f32", (0.001, 0.1)),
])
def test_chunk_cumsum(b, L, H, Q, dtype, limit):
    announce("chunk_cumsum", b, L, H, Q, dtype, limit)
    d = _inputs(b, L, H, 1, 16, 16, Q, dtype, seed=L + H)
    dA, dto = chunk_cumsum_fwd(dev(d["dt"], tdtype(dtype)), dev(d["A"]), Q,
                               dt_bias=dev(d["dt_bias"]), dt_softplus=True, dt_limit=limit)
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True, limit)
    check(dto, wdt, 1e-5, "dt_out")
    check(dA, wA, 1e-5, "dA_cumsum")


# ---------------------------------------------------------------------------
# chunk_state
# ---------------------------------------------------------------------------

STATE_CFGS = [
    # (b, L, H, P, N, G, Q)   reference state_configs + ours
    (1, 128, 8, 64, 64, 1, 64),
    (1, 128, 16, 64, 64, 2, 128),
    (1, 256, 64, 64, 64, 8, 256),
    (1, 128, 4, 128, 64, 1, 64),
    (1, 256, 256, 64, 256, 8, 256),
    (2, 200, 8, 32, 128, 2, 64),     # L % Q != 0, headdim 32
    (2, 200, 8, 64, 128, 2, 64),     # L % Q != 0, batch 2, one-shot bf16 kernel
    (1, 100, 8, 64, 128, 2, 32),     # chunk 32, L % Q != 0
    (1, 4096, 128, 64, 128, 8, 128), # nemotron-h-8b layer shape
    (1, 256, 6, 64, 128, 2, 128),    # 3 heads per group: one head per workgroup
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg", STATE_CFGS)
def test_chunk_state(cfg, dtype):
    b, L, H, P, N, G, Q = cfg
    announce("chunk_state", cfg, dtype)
    d = _inputs(b, L, H, G, P, N, Q, dtype, seed=sum(cfg))
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    got = chunk_state_fwd(dev(d["x"], tdtype(dtype)), dev(d["B"], tdtype(dtype)),
                          dev(wdt.astype(np.float32)), dev(wA.astype(np.float32)))
    want = O.chunk_state(d["B"], d["x"], wdt.astype(np.float32), wA.astype(np.float32))
    check(got, want, TOL[dtype], "states")


@pytest.mark.parametrize("cfg,lens", [
    ((1, 128, 8, 64, 64, 1, 64), [[64, 64]]),
    ((1, 256, 16, 64, 64, 2, 128), [[128, 128]]),
    ((2, 512, 8, 64, 128, 4, 64), [[200, 312], [100, 412]]),
])
def test_chunk_state_seq_idx(cfg, lens):
    b, L, H, P, N, G, Q = cfg
    announce("chunk_state seq_idx", cfg, lens)
    d = _inputs(b, L, H, G, P, N, Q, "bf16", seed=7 + L)
    seq = seq_idx_from_lengths(lens)
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wdt, wA = wdt.astype(np.float32), wA.astype(np.float32)
    got = chunk_state_fwd(dev(d["x"], torch.bfloat16), dev(d["B"], torch.bfloat16), dev(wdt),
                          dev(wA), seq_idx=dev(seq))
    want = O.chunk_state(d["B"], d["x"], wdt, wA, seq_idx=seq)
    check(got, want, TOL["bf16"], "states")


# ---------------------------------------------------------------------------
# state_passing
# ---------------------------------------------------------------------------

SP_CFGS = [
    # (batch, nchunks, nheads, dim, init, seq_lengths, chunk_size)  reference sp configs
    (1, 4, 1, 128, False, None, None),
    (1, 4, 1, 128, True, None, None),
    (2, 8, 4, 128, True, None, None),
    (1, 8, 8, 4096, True, None, None),
    (2, 8, 16, 4096, True, None, None),
    (1, 8, 4, 16384, True, None, None),
    (2, 32, 4, 4096, True, None, None),
    (1, 4, 2, 200, True, None, None),
    (2, 8, 4, 300, True, None, None),
    (1, 5, 3, 202, True, None, None),              # dim % 4 != 0: scalar path
    (1, 4, 4, 128, True, [[256]], 64),
    (1, 4, 4, 128, False, [[128, 128]], 64),
    (2, 8, 8, 128, True, [[200, 312], [100, 412]], 64),
    (2, 8, 4, 4096, True, [[64, 192, 256], [128, 128, 256]], 64),
    (1, 4, 4, 128, True, [[64, 64, 64, 64]], 64),
    (1, 3, 2, 64, True, [[100, 90]], 64),          # seqlen not a multiple of Q
]


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("cfg", SP_CFGS)
def test_state_passing(cfg, out_dtype):
    b, nc, H, D, init, lens, Q = cfg
    announce("state_passing", cfg, out_dtype)
    rng = np.random.default_rng(b * 1000 + nc * 10 + H + D)
    st = rng.standard_normal((b, nc, H, D)).astype(np.float32)
    dAfull = -rng.uniform(0.0, 3.0, (b, H, nc, 4)).astype(np.float32)
    s0 = rng.standard_normal((b, H, D)).astype(np.float32) if init else None
    seq = seq_idx_from_lengths(lens) if lens else None
    dAc_t = dev(dAfull)[..., -1]          # strided view, as ssd_combined passes it
    out, fin = state_passing_fwd(dev(st), dAc_t, dev(s0), seq_idx=dev(seq), chunk_size=Q,
                                 out_dtype=tdtype(out_dtype))
    assert out.dtype == tdtype(out_dtype) and fin.dtype == torch.float32
    wo, wf = O.state_passing(st, dAfull[..., -1], s0, seq_idx=seq, chunk_size=Q)
    check(out, wo, 1e-5 if out_dtype == "f32" else TOL["bf16"], "out")
    check(fin, wf, 1e-5, "final")


# ---------------------------------------------------------------------------
# bmm_chunk
# ---------------------------------------------------------------------------

BMM_CFGS = [
    # (batch, seqlen, ngroups, k, chunk_size, causal, seq_lengths)
    (1, 256, 1, 64, 64, False, None),
    (2, 512, 1, 64, 128, False, None),
    (2, 1024, 1, 64, 256, False, None),
    (2, 512, 8, 64, 128, False, None),
    (1, 256, 8, 256, 64, False, None),
    (1, 2048, 8, 256, 256, False, None),
    (2, 1024, 8, 64, 256, True, None),
    (1, 256, 8, 256, 64, True, None),
    (1, 300, 2, 128, 128, True, None),               # L % Q != 0
    (1, 256, 1, 64, 64, False, [[128, 128]]),
    (2, 512, 4, 64, 64, False, [[200, 312], [100, 412]]),
    (2, 512, 1, 64, 128, True, [[256, 256], [128, 384]]),
    (2, 512, 8, 64, 64, True, [[64, 192, 256], [128, 128, 256]]),
    (1, 256, 1, 64, 64, False, [[64, 64, 64, 64]]),
    # >= 128 (chunk, group) blocks: the LDS-staged kernels (fp32 and bf16)
    (1, 4096, 8, 128, 128, False, None),             # c2 shape
    (1, 4000, 8, 128, 128, True, [[1000, 3000]]),    # L % Q != 0, seq_idx
    (2, 2048, 4, 64, 64, True, [[700, 1348], [2048]]),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg", BMM_CFGS)
def test_bmm_chunk(cfg, dtype):
    b, L, G, K, Q, causal, lens = cfg
    announce("bmm_chunk", cfg, dtype)
    rng = np.random.default_rng(L + G + K + Q)
    a = configs.round_to(rng.standard_normal((b, L, G, K)).astype(np.float32), dtype)
    bb = configs.round_to(rng.standard_normal((b, L, G, K)).astype(np.float32), dtype)
    seq = seq_idx_from_lengths(lens) if lens else None
    got = bmm_chunk_fwd(dev(a, tdtype(dtype)), dev(bb, tdtype(dtype)), Q, seq_idx=dev(seq),
                        causal=causal)
    assert got.dtype == torch.float32
    want = O.bmm_chunk(a, bb, Q, seq_idx=seq, causal=causal)
    check(got, want, 1e-5 if dtype == "bf16" else 1e-4, "CB")


def test_bmm_chunk_bf16_output():
    rng = np.random.default_rng(3)
    a = configs.round_to(rng.standard_normal((1, 256, 2, 64)).astype(np.float32), "bf16")
    got = bmm_chunk_fwd(dev(a, torch.bfloat16), dev(a, torch.bfloat16), 128,
                        output_dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16
    # fp32 accumulation then one round-to-nearest-even: within half a bf16 ulp
    want = O.bmm_chunk(a, a, 128)
    err = np.abs(host(got) - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -8 + 1e-6), float(err.max())


# ---------------------------------------------------------------------------
# chunk_scan
# ---------------------------------------------------------------------------

SCAN_CFGS = [
    # (b, L, H, P, N, G, Q, D, z, seq_lengths)
    (1, 256, 4, 64, 64, 1, 64, True, True, None),
    (2, 512, 8, 64, 64, 8, 64, False, False, None),
    (1, 512, 16, 64, 128, 2, 128, True, False, None),
    (1, 512, 8, 64, 128, 1, 256, True, True, None),
    (1, 384, 8, 64, 256, 8, 128, True, False, None),
    (1, 300, 4, 32, 64, 2, 128, True, True, None),        # L % Q != 0, headdim 32
    (1, 256, 4, 128, 64, 1, 64, True, False, None),       # headdim 128
    (1, 300, 4, 128, 128, 2, 256, True, True, None),      # headdim 128, chunk 256 (fp32: state read from L2)
    (2, 512, 8, 64, 64, 1, 64, False, False, [[200, 312], [100, 412]]),
    (2, 512, 8, 64, 64, 4, 128, True, True, [[256, 256], [128, 384]]),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg", SCAN_CFGS)
def test_chunk_scan(cfg, dtype):
    b, L, H, P, N, G, Q, hasD, hasz, lens = cfg
    announce("chunk_scan", cfg, dtype)
    d = _inputs(b, L, H, G, P, N, Q, dtype, seed=L + H + N + Q, z=hasz)
    seq = seq_idx_from_lengths(lens) if lens else None
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    rf = O.round_fn_for(dtype)
    CB = O.bmm_chunk(d["C"], d["B"], Q, seq_idx=seq).astype(np.float32)
    nc = math.ceil(L / Q)
    rng = np.random.default_rng(11)
    states = (0.5 * rng.standard_normal((b, nc, H, P, N))).astype(np.float32)
    D = d["D"] if hasD else None
    T = tdtype(dtype)
    out, out_x = chunk_scan_fwd(dev(CB), dev(d["x"], T), dev(wdt), dev(wA), dev(d["C"], T),
                                dev(states), D=dev(D), z=dev(d["z"], T), seq_idx=dev(seq))
    wo, wox = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states, D=D, z=d["z"], seq_idx=seq,
                           round_fn=rf)
    check(out, wo, TOL[dtype], "out")
    if hasz:
        check(out_x, wox, TOL[dtype], "out_x")
    else:
        assert out_x is None


F32_GROUP = [
    # (b, L, H, G, N, D per head dim, z, seq_lengths, heads per workgroup: 0 = the
    # launcher's choice)
    (2, 300, 8, 2, 128, True, True, None, 3),            # slices of 3 + 1, last chunk 44 rows
    (1, 512, 24, 1, 128, False, False, None, 2),         # mamba2-130m heads, 12 slices
    (1, 384, 8, 4, 64, False, True, [[100, 284]], 2),    # dstate 64: three ring slots
    (2, 256, 16, 2, 128, True, False, [[60, 196], [256]], 8),
    (1, 130, 4, 1, 64, True, True, None, 4),             # last chunk of 2 positions
    (1, 512, 16, 2, 128, True, False, None, 0),
    (1, 4096, 128, 8, 128, False, False, None, 0),       # nemotron-h-8b shape
    (1, 50, 4, 4, 128, True, True, None, 1),             # one partial chunk, one head a group
    (2, 100, 6, 3, 64, False, False, [[30, 70], [100]], 0),
    (1, 256, 8, 2, 128, True, False, None, 9),           # slice larger than the group
]


@pytest.mark.parametrize("case", F32_GROUP)
def test_chunk_scan_f32_group(case):
    """fp32 chunk_scan at chunk 128, head dim 64 runs the group kernel (one
    workgroup per (chunk, group, slice of the group's heads)): against the
    oracle, and against the per-(chunk, head) kernel (the same bf16-triple
    products, summed in another order)."""
    from mamba2_jax._lib import dispatch_override
    b, L, H, G, N, Dhp, hasz, lens, hps = case
    P, Q = 64, 128
    announce("chunk_scan fp32 group kernel", case)
    d = _inputs(b, L, H, G, P, N, Q, "f32", seed=L + H + N, z=hasz)
    seq = seq_idx_from_lengths(lens) if lens else None
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    CB = O.bmm_chunk(d["C"], d["B"], Q, seq_idx=seq).astype(np.float32)
    nc = math.ceil(L / Q)
    rng = np.random.default_rng(H + N)
    states = (0.5 * rng.standard_normal((b, nc, H, P, N))).astype(np.float32)
    D = rng.uniform(0.5, 1.5, (H, P) if Dhp else H).astype(np.float32)
    args = (dev(CB), dev(d["x"]), dev(wdt), dev(wA), dev(d["C"]), dev(states))
    kw = dict(D=dev(D), z=dev(d["z"]), seq_idx=dev(seq))
    with dispatch_override("f32_scan", f"group{hps}" if hps else "per_head"):
        if hps:
            out, out_x = chunk_scan_fwd(*args, **kw)
        else:
            ref, ref_x = chunk_scan_fwd(*args, **kw)
    if hps:
        with dispatch_override("f32_scan", "per_head"):
            ref, ref_x = chunk_scan_fwd(*args, **kw)
    else:
        out, out_x = chunk_scan_fwd(*args, **kw)
    wo, wox = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states, D=D, z=d["z"], seq_idx=seq,
                           round_fn=O.round_fn_for("f32"))
    check(out, wo, TOL["f32"], "out")
    check(out, host(ref), 2e-5, "out, group vs per-head kernel")
    if hasz:
        check(out_x, wox, TOL["f32"], "out_x")
        check(out_x, host(ref_x), 2e-5, "out_x, group vs per-head kernel")


def test_chunk_scan_bf16_cb_and_states():
    """cb and states given in bf16 (the combined path's internal formats)."""
    b, L, H, P, N, G, Q = 1, 256, 8, 64, 128, 2, 128
    d = _inputs(b, L, H, G, P, N, Q, "bf16", seed=5)
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    CB = O.bf16_round(O.bmm_chunk(d["C"], d["B"], Q))
    rng = np.random.default_rng(2)
    states = O.bf16_round(0.5 * rng.standard_normal((b, 2, H, P, N)))
    out, _ = chunk_scan_fwd(dev(CB, torch.bfloat16), dev(d["x"], torch.bfloat16), dev(wdt),
                            dev(wA), dev(d["C"], torch.bfloat16), dev(states, torch.bfloat16),
                            D=dev(d["D"]))
    wo, _ = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states, D=d["D"])
    check(out, wo, TOL["bf16"], "out")


@pytest.mark.parametrize("b,L,H,N,G,Q,Dhp,lens", [
    (1, 512, 16, 128, 2, 128, False, None),
    (2, 300, 8, 64, 4, 64, True, None),                  # L % Q != 0, D per head dim
    (1, 384, 8, 256, 8, 128, False, None),
    (2, 512, 8, 128, 1, 64, False, [[200, 312], [100, 412]]),
    (1, 4096, 128, 128, 8, 128, False, None),            # nemotron-h-8b layer shape
])
def test_chunk_scan_fused_cb(b, L, H, N, G, Q, Dhp, lens):
    """bf16 x / C, CB from bmm_chunk (fp32) and bf16 states, no z: the stage
    operator runs on the fused scan kernel with CB read in (rounded to bf16,
    causal mask only: the seq_idx mask of CB is bmm_chunk's)."""
    P = 64
    announce("chunk_scan fused, CB given", b, L, H, N, G, Q, Dhp, lens)
    d = _inputs(b, L, H, G, P, N, Q, "bf16", seed=L + N + Q)
    seq = seq_idx_from_lengths(lens) if lens else None
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    CB = O.bmm_chunk(d["C"], d["B"], Q, seq_idx=seq).astype(np.float32)
    nc = math.ceil(L / Q)
    states = O.bf16_round(0.5 * np.random.default_rng(4).standard_normal((b, nc, H, P, N)))
    D = np.random.default_rng(5).uniform(0.5, 1.5, (H, P) if Dhp else H).astype(np.float32)
    out, out_x = chunk_scan_fwd(dev(CB), dev(d["x"], torch.bfloat16), dev(wdt), dev(wA),
                                dev(d["C"], torch.bfloat16), dev(states, torch.bfloat16),
                                D=dev(D), seq_idx=dev(seq))
    assert out_x is None
    wo, _ = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states, D=D, seq_idx=seq,
                         round_fn=O.round_fn_for("bf16"))
    check(out, wo, TOL["bf16"], "out")


def test_chunk_scan_large_decay_is_stable():
    """|dA| inside a chunk far beyond 80: the factored exp(dA_m) * exp(-dA_k) form
    overflows there; the kernel evaluates exp(dA_m - dA_k) directly."""
    b, L, H, P, N, G, Q = 1, 256, 4, 64, 64, 1, 256
    d = _inputs(b, L, H, G, P, N, Q, "f32", seed=9)
    dt = np.full((b, L, H), 8.0, np.float32)                 # dt' = softplus(8 + bias) ~ 2-6
    A = np.full(H, -16.0, np.float32)
    wA, wdt = O.chunk_cumsum(dt, A, Q, d["dt_bias"], True)
    assert wA.min() < -2000
    wA, wdt = wA.astype(np.float32), wdt.astype(np.float32)
    CB = O.bmm_chunk(d["C"], d["B"], Q).astype(np.float32)
    states = np.zeros((b, 1, H, P, N), np.float32)
    out, _ = chunk_scan_fwd(dev(CB), dev(d["x"]), dev(wdt), dev(wA), dev(d["C"]), dev(states))
    wo, _ = O.chunk_scan(CB, d["x"], wdt, wA, d["C"], states)
    assert torch.isfinite(out).all()
    check(out, wo, TOL["f32"], "out")


# ---------------------------------------------------------------------------
# chunk_state_varlen
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nseq,H,P,N,G,Q,states_dtype,empty", [
    (10, 8, 64, 64, 1, 64, "f32", False),        # reference varlen configs
    (5, 8, 64, 64, 8, 64, "bf16", False),
    (6, 16, 64, 256, 8, 128, "bf16", False),     # c3-like
    (5, 8, 64, 128, 2, 256, "bf16", True),       # chunk 256, an empty sequence
    (6, 8, 64, 128, 2, 128, "bf16", True),       # two heads per workgroup, an empty sequence
    (7, 4, 32, 64, 1, 64, "bf16", True),         # head dim 32 (general kernel)
])
def test_chunk_state_varlen(nseq, H, P, N, G, Q, states_dtype, empty):
    announce("chunk_state_varlen", nseq, H, P, N, G, Q, states_dtype, empty)
    rng = np.random.default_rng(nseq * 7 + N)
    lens = rng.integers(1, 3 * Q, nseq)
    lens[0] = Q                                  # one ending exactly on a chunk edge
    if empty:
        lens[2] = 0                              # zero state
    total = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = _inputs(1, total, H, G, P, N, Q, "bf16", seed=nseq)
    wA, wdt = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    wA, wdt = wA[0].astype(np.float32), wdt[0].astype(np.float32)
    nc = wA.shape[1]
    cs = O.round_fn_for(states_dtype)(rng.standard_normal((nc, H, P, N))).astype(np.float32)
    got = chunk_state_varlen_mosaic(dev(d["B"][0], torch.bfloat16), dev(d["x"][0], torch.bfloat16),
                                    dev(wdt), dev(wA), dev(cu), dev(cs, tdtype(states_dtype)))
    want = O.chunk_state_varlen(d["B"][0], d["x"][0], wdt, wA, cu, cs)
    check(got, want, TOL["bf16"], "varlen states")

"""The size mapping of mamba2_jax/kernels/_shapes.py leaves every result
unchanged: zero padding of headdim / dstate, head splitting and dstate blocks.

Each operator's mapping is run on the CPU with the oracle (float64, without
the reference's rounding points: io_dtype=None) standing in for the kernels
behind it, and compared with the oracle on the original sizes; the mapped problem must agree to float64 summation
order.  The stand-in also asserts that it only ever sees sizes the kernels are
built for.  (The GPU tests run the same mapping in front of the kernels.)
"""

import importlib

import numpy as np
import pytest
import torch

from mamba2_jax.kernels import _shapes as S
from oracle import ssd_oracle as O

# the modules (the package re-exports functions of the same names)
CSC = importlib.import_module("mamba2_jax.kernels.chunk_scan_fwd")
CST = importlib.import_module("mamba2_jax.kernels.chunk_state_fwd")
SC = importlib.import_module("mamba2_jax.kernels.ssd_combined")

TIGHT = 1e-12


def _np(t):
    if t is None:
        return None
    a = t.numpy()
    return a if a.dtype.kind == "i" else a.astype(np.float64)


def _t(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a))


def _inputs(b, L, H, G, P, N, seed, init=True, z=True, Dhp=True, nseq=0):
    rng = np.random.default_rng(seed)
    d = dict(x=rng.standard_normal((b, L, H, P)), dt=rng.standard_normal((b, L, H)),
             A=-np.exp(rng.uniform(0, np.log(16), H)), B=rng.standard_normal((b, L, G, N)) / np.sqrt(N),
             C=rng.standard_normal((b, L, G, N)) / np.sqrt(N),
             D=rng.uniform(0.5, 1.5, (H, P) if Dhp else H), z=rng.standard_normal((b, L, H, P)) if z else None,
             dt_bias=rng.uniform(-4, -2, H), initial_states=0.1 * rng.standard_normal((b, H, P, N)) if init else None,
             seq_idx=None, cu_seqlens=None)
    if nseq:
        cuts = np.sort(rng.choice(np.arange(1, L), nseq - 1, replace=False))
        lens = np.diff(np.concatenate([[0], cuts, [L]]))
        d["cu_seqlens"] = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        d["seq_idx"] = np.repeat(np.arange(nseq), lens)[None].astype(np.int32)
    return d


def test_plans():
    assert S.p_plan_stage(48) == (64, 1) and S.p_plan_stage(16) == (32, 1)
    assert S.p_plan_stage(96) == (128, 1) and S.p_plan_stage(128) == (128, 1)
    assert S.p_plan_stage(200) == (256, 4) and S.p_plan_stage(192) == (192, 3)
    assert S.p_plan_layer(32) == (32, 1) and S.p_plan_layer(64) == (64, 1)
    assert S.p_plan_layer(128) == (128, 2) and S.p_plan_layer(80) == (128, 2)
    assert S.p_plan_layer(16) == (64, 1)
    assert [S.n_pad(n) for n in (1, 16, 64, 65, 96, 160, 256)] == [64, 64, 64, 128, 128, 256, 256]
    assert S.n_blocks(600) == [(0, 256), (256, 512), (512, 600)]
    assert S.n_blocks(256) == [(0, 256)]


def test_split_heads_is_a_view_and_groups_follow():
    x = torch.arange(2 * 3 * 4 * 128).reshape(2, 3, 4, 128)
    xs = S.split_heads(x, 2, 2)
    assert xs.shape == (2, 3, 8, 64) and xs.data_ptr() == x.data_ptr()
    assert torch.equal(S.merge_heads(xs, 2, 2, 128), x)
    # head h * k + j of the split problem sits in the group of head h
    H, G, k = 12, 3, 4
    for h in range(H):
        for j in range(k):
            assert (h * k + j) // (k * H // G) == h // (H // G)


COMBINED_CASES = [
    # (P, N, Q, init, z, Dhp, nseq)
    (48, 16, 32, True, True, True, 0),
    (80, 48, 32, False, True, False, 3),
    (96, 96, 64, True, False, True, 0),
    (128, 160, 32, True, True, True, 2),
    (200, 64, 32, True, True, True, 0),
    (64, 320, 32, True, True, True, 3),
    (16, 300, 64, False, True, True, 0),
]


@pytest.mark.parametrize("case", COMBINED_CASES)
def test_combined_mapping_exact(case):
    P, N, Q, init, z, Dhp, nseq = case
    b = 1 if nseq else 2
    d = _inputs(b, 96, 4, 2, P, N, seed=P + N, init=init, z=z, Dhp=Dhp, nseq=nseq)
    seen = []

    def oracle_native(x, dt, A, B, C, chunk_size, D, z, dt_bias, init, seq_idx, cu, nseq, softplus,
                      limit, want_final, events):
        seen.append((x.shape[-1], B.shape[-1]))
        assert x.shape[-1] in S.NATIVE_P_LAYER and B.shape[-1] in S.NATIVE_N
        res = O.ssd_combined(_np(x), _np(dt), _np(A), _np(B), _np(C), chunk_size, D=_np(D), z=_np(z),
                             dt_bias=_np(dt_bias), initial_states=_np(init), seq_idx=_np(seq_idx),
                             cu_seqlens=_np(cu), dt_softplus=softplus, dt_limit=limit,
                             return_final_states=True, return_varlen_states=cu is not None,
                             io_dtype=None)
        return _t(res[0]), _t(res[1]) if want_final else None, _t(res[2]) if cu is not None else None

    t = {k: _t(v) for k, v in d.items()}
    out, fin, vs = SC._combined(t["x"], t["dt"], t["A"], t["B"], t["C"], Q, t["D"], t["z"],
                                t["dt_bias"], t["initial_states"], t["seq_idx"],
                                t["cu_seqlens"] if nseq else None, nseq, True,
                                (0.0, float("inf")), True, None, native=oracle_native)
    assert seen and all(s != (P, N) for s in seen)
    want = O.ssd_combined(chunk_size=Q, dt_softplus=True, return_final_states=True,
                          return_varlen_states=bool(nseq), io_dtype=None, **d)
    assert out.shape == (b, 96, 4, P) and fin.shape == (b, 4, P, N)
    assert O.rel_err(out.numpy(), want[0]) < TIGHT
    assert O.rel_err(fin.numpy(), want[1]) < TIGHT
    if nseq:
        assert vs.shape == (nseq, 4, P, N)
        assert O.rel_err(vs.numpy(), want[2]) < TIGHT


STAGE_CASES = [(48, 16), (80, 48), (96, 96), (16, 160), (200, 64), (64, 320), (130, 300)]


def _stage_inputs(P, N, Q=32, b=2, L=80, H=4, G=2, seed=0):
    d = _inputs(b, L, H, G, P, N, seed=seed + P + N, nseq=0)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    return d, dA, dto


@pytest.mark.parametrize("P,N", STAGE_CASES)
def test_chunk_state_mapping_exact(P, N):
    d, dA, dto = _stage_inputs(P, N)
    seq = np.repeat([[0, 1]], [30, 50], axis=1).astype(np.int32).repeat(2, 0)

    def oracle_native(x, B, dt, dA_cumsum, seq_idx):
        assert x.shape[-1] in S.NATIVE_P_STAGE and B.shape[-1] in S.NATIVE_N
        return _t(O.chunk_state(_np(B), _np(x), _np(dt), _np(dA_cumsum), seq_idx=_np(seq_idx)))

    got = CST._chunk_state(_t(d["x"]), _t(d["B"]), _t(dto), _t(dA), _t(seq), native=oracle_native)
    want = O.chunk_state(d["B"], d["x"], dto, dA, seq_idx=seq)
    assert got.shape == want.shape
    assert O.rel_err(got.numpy(), want) < TIGHT


@pytest.mark.parametrize("P,N", STAGE_CASES)
def test_chunk_scan_mapping_exact(P, N):
    d, dA, dto = _stage_inputs(P, N)
    rng = np.random.default_rng(P * N)
    CB = O.bmm_chunk(d["C"], d["B"], 32)
    states = 0.5 * rng.standard_normal((2, 3, 4, P, N))

    def oracle_native(cb, x, dt, dA_cumsum, C, st, D, z, seq_idx):
        assert x.shape[-1] in S.NATIVE_P_STAGE and C.shape[-1] in (32,) + S.NATIVE_N
        o, ox = O.chunk_scan(_np(cb), _np(x), _np(dt), _np(dA_cumsum), _np(C), _np(st), D=_np(D),
                             z=_np(z), seq_idx=_np(seq_idx))
        return _t(o), _t(ox) if z is not None else None

    got, got_x = CSC._chunk_scan(_t(CB), _t(d["x"]), _t(dto), _t(dA), _t(d["C"]), _t(states),
                                 _t(d["D"]), _t(d["z"]), None, native=oracle_native)
    want, want_x = O.chunk_scan(CB, d["x"], dto, dA, d["C"], states, D=d["D"], z=d["z"])
    assert O.rel_err(got.numpy(), want) < TIGHT
    assert O.rel_err(got_x.numpy(), want_x) < TIGHT


@pytest.mark.parametrize("P,N", STAGE_CASES)
def test_varlen_mapping_exact(P, N):
    d = _inputs(1, 80, 4, 2, P, N, seed=P + N, nseq=3)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], 32, d["dt_bias"], True)
    rng = np.random.default_rng(N)
    cs = 0.5 * rng.standard_normal((3, 4, P, N))

    def oracle_native(B, x, dt, dA_cumsum, cu, chunk_states):
        assert x.shape[-1] in S.NATIVE_P_STAGE and B.shape[-1] in S.NATIVE_N
        return _t(O.chunk_state_varlen(_np(B), _np(x), _np(dt), _np(dA_cumsum), _np(cu),
                                       _np(chunk_states)))

    got = CST._varlen(_t(d["B"][0]), _t(d["x"][0]), _t(dto[0]), _t(dA[0]), _t(d["cu_seqlens"]),
                      _t(cs), native=oracle_native)
    want = O.chunk_state_varlen(d["B"][0], d["x"][0], dto[0], dA[0], d["cu_seqlens"], cs)
    assert O.rel_err(got.numpy(), want) < TIGHT


def test_gate_matches_oracle_silu():
    rng = np.random.default_rng(3)
    ox, z = rng.standard_normal((5, 7)), rng.standard_normal((5, 7)).astype(np.float32)
    got = S.gate(torch.from_numpy(ox).float(), torch.from_numpy(z))
    assert O.rel_err(got.numpy(), ox * O.silu(z.astype(np.float64))) < 1e-6

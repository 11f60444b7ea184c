"""Pins for the CPU oracle (oracle/ssd_oracle.py), CPU only.

Each oracle function is checked against something that does not share its
formulation: brute-force loops, closed forms, the token-by-token recurrence,
chunk-size invariance, or per-sequence decomposition.  A dropped term, a wrong
sign or index, or a transposed operand in the oracle fails at least one check.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ssd_oracle as O
from mamba2_jax import configs


def _rand_inputs(rng, b, L, H, G, P, N, with_D=True, with_z=False, init=False):
    x = rng.standard_normal((b, L, H, P))
    dt = rng.standard_normal((b, L, H))
    A = -np.exp(rng.uniform(0.0, math.log(16.0), H))
    B = rng.standard_normal((b, L, G, N)) / math.sqrt(N)
    C = rng.standard_normal((b, L, G, N)) / math.sqrt(N)
    dt_bias = rng.uniform(-4.0, -1.0, H)
    D = rng.uniform(0.5, 1.5, H) if with_D else None
    z = rng.standard_normal((b, L, H, P)) if with_z else None
    s0 = 0.3 * rng.standard_normal((b, H, P, N)) if init else None
    return dict(x=x, dt=dt, A=A, B=B, C=C, dt_bias=dt_bias, D=D, z=z,
                initial_states=s0)


# ---------------------------------------------------------------------------
# bf16 emulation == torch's RNE cast (the cast the device tensors go through)
# ---------------------------------------------------------------------------

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        # exact ties: mantissa low half == 0x8000, with even and odd kept bit
        (np.arange(1, 2001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.4e38, -3.4e38, 1e-45], np.float32),
    ]).astype(np.float32)
    want = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    got = O.bf16_round(v)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------
# chunk_cumsum
# ---------------------------------------------------------------------------

def test_chunk_cumsum_closed_form_loop():
    rng = np.random.default_rng(1)
    b, L, H, Q = 2, 37, 3, 8
    dt = rng.standard_normal((b, L, H))
    A = -rng.uniform(1, 5, H)
    bias = rng.uniform(-3, 0, H)
    dA, dto = O.chunk_cumsum(dt, A, Q, dt_bias=bias, dt_softplus=True,
                             dt_limit=(0.01, 0.5))
    nc = -(-L // Q)
    assert dA.shape == (b, H, nc, Q)
    for bi in range(b):
        for h in range(H):
            for c in range(nc):
                run = 0.0
                for q in range(Q):
                    t = c * Q + q
                    if t < L:
                        v = math.log1p(math.exp(dt[bi, t, h] + bias[h]))
                        v = min(max(v, 0.01), 0.5)
                    else:
                        v = 0.0
                    run += v * A[h]
                    assert dto[bi, h, c, q] == pytest.approx(v, abs=1e-14)
                    assert dA[bi, h, c, q] == pytest.approx(run, abs=1e-12)


def test_chunk_cumsum_special_cases():
    rng = np.random.default_rng(2)
    dt = rng.standard_normal((1, 16, 2))
    # dt -> -inf through softplus gives dt' = 0 and dA = 0
    dA, dto = O.chunk_cumsum(np.full_like(dt, -1e4), np.array([-2.0, -3.0]), 8,
                             dt_softplus=True)
    assert np.all(dto == 0.0) and np.all(dA == 0.0)
    # A = 0 gives dA = 0 whatever dt is
    dA, _ = O.chunk_cumsum(dt, np.zeros(2), 8, dt_softplus=True)
    assert np.all(dA == 0.0)
    # large arguments: softplus(v) == v
    _, dto = O.chunk_cumsum(np.full_like(dt, 50.0), np.array([-1.0, -1.0]), 8,
                            dt_softplus=True)
    assert np.allclose(dto, 50.0, rtol=0, atol=1e-12)


def test_chunk_cumsum_pad_modes_differ_only_in_padding():
    rng = np.random.default_rng(3)
    dt = rng.standard_normal((1, 20, 2))
    kw = dict(dt_bias=np.array([-2.0, -1.0]), dt_softplus=True)
    a1, d1 = O.chunk_cumsum(dt, np.array([-1.0, -2.0]), 8, pad="kernel", **kw)
    a2, d2 = O.chunk_cumsum(dt, np.array([-1.0, -2.0]), 8, pad="naive", **kw)
    flat1 = d1.transpose(0, 2, 3, 1).reshape(1, 24, 2)
    flat2 = d2.transpose(0, 2, 3, 1).reshape(1, 24, 2)
    np.testing.assert_array_equal(flat1[:, :20], flat2[:, :20])
    assert np.all(flat1[:, 20:] == 0.0) and np.all(flat2[:, 20:] > 0.0)


# ---------------------------------------------------------------------------
# chunk_state
# ---------------------------------------------------------------------------

def _brute_chunk_state(B, x, dt, dA, seq_idx=None):
    b, L, H, P = x.shape
    G, N = B.shape[2:]
    _, _, nc, Q = dt.shape
    out = np.zeros((b, nc, H, P, N))
    for bi in range(b):
        for c in range(nc):
            end = min((c + 1) * Q, L) - 1
            for h in range(H):
                g = h // (H // G)
                for q in range(Q):
                    t = c * Q + q
                    if t >= L:
                        continue
                    if seq_idx is not None:
                        se = seq_idx[bi, end]
                        if se < 0 or seq_idx[bi, t] != se:
                            continue
                    w = math.exp(dA[bi, h, c, Q - 1] - dA[bi, h, c, q]) * dt[bi, h, c, q]
                    out[bi, c, h] += w * np.outer(x[bi, t, h], B[bi, t, g])
    return out


@pytest.mark.parametrize("seq", [False, True])
def test_chunk_state_brute_force(seq):
    rng = np.random.default_rng(4)
    b, L, H, G, P, N, Q = 2, 21, 4, 2, 3, 5, 8
    d = _rand_inputs(rng, b, L, H, G, P, N)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], Q, d["dt_bias"], True)
    seq_idx = None
    if seq:
        seq_idx = np.array([[0] * 5 + [1] * 10 + [2] * 6, [0] * 12 + [3] * 9])
    got = O.chunk_state(d["B"], d["x"], dto, dA, seq_idx=seq_idx)
    want = _brute_chunk_state(d["B"], d["x"], dto, dA, seq_idx)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_chunk_state_decay_clamp():
    """decay_clamp (the reference kernel's min(., 0)) only matters where dA
    increases: identical for a non-increasing dA; for Q = 2 with dt' A > 0 at
    the second position the first weight is dt'_0 (clamped) instead of
    exp(A dt'_1) dt'_0."""
    rng = np.random.default_rng(14)
    d = _rand_inputs(rng, 1, 16, 2, 1, 3, 4)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], 8, d["dt_bias"], True)
    assert np.all(np.diff(dA, axis=-1) <= 0)
    np.testing.assert_array_equal(O.chunk_state(d["B"], d["x"], dto, dA, decay_clamp=True),
                                  O.chunk_state(d["B"], d["x"], dto, dA))
    x = rng.standard_normal((1, 2, 1, 3))
    B = rng.standard_normal((1, 2, 1, 4))
    A, d0, d1 = 0.7, 0.3, 0.5
    dA2, dt2 = O.chunk_cumsum(np.array([[[d0], [d1]]]), np.array([A]), 2)
    term0 = d0 * np.outer(x[0, 0, 0], B[0, 0, 0])
    term1 = d1 * np.outer(x[0, 1, 0], B[0, 1, 0])
    np.testing.assert_allclose(O.chunk_state(B, x, dt2, dA2, decay_clamp=True)[0, 0, 0],
                               term0 + term1, rtol=1e-13)
    np.testing.assert_allclose(O.chunk_state(B, x, dt2, dA2)[0, 0, 0],
                               math.exp(A * d1) * term0 + term1, rtol=1e-13)


def test_chunk_state_q1_closed_form():
    rng = np.random.default_rng(5)
    d = _rand_inputs(rng, 1, 6, 2, 1, 3, 4)
    dA, dto = O.chunk_cumsum(d["dt"], d["A"], 1, d["dt_bias"], True)
    st = O.chunk_state(d["B"], d["x"], dto, dA)
    want = (dto[0, :, :, 0].T[:, :, None, None] * d["x"][0][:, :, :, None]
            * d["B"][0][:, :, None, :])
    np.testing.assert_allclose(st[0], want, rtol=1e-13, atol=1e-14)


# ---------------------------------------------------------------------------
# state_passing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("init", [False, True])
def test_state_passing_pairwise_equals_sequential(init):
    rng = np.random.default_rng(6)
    b, nc, H, D = 2, 7, 3, 10
    st = rng.standard_normal((b, nc, H, D))
    dAc = -rng.uniform(0, 3, (b, H, nc))
    s0 = rng.standard_normal((b, H, D)) if init else None
    o1, f1 = O.state_passing(st, dAc, s0, method="pairwise")
    o2, f2 = O.state_passing(st, dAc, s0, method="sequential")
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(f1, f2, rtol=1e-12, atol=1e-12)
    # out[0] is the initial state, out[c+1] = exp(dA[c]) out[c] + states[c]
    np.testing.assert_allclose(o1[:, 0], 0.0 if s0 is None else s0)
    np.testing.assert_allclose(o1[:, 1], np.exp(dAc[:, :, 0])[..., None] * o1[:, 0] + st[:, 0])


def test_state_passing_no_decay_is_prefix_sum():
    rng = np.random.default_rng(7)
    st = rng.standard_normal((1, 5, 2, 4))
    out, fin = O.state_passing(st, np.zeros((1, 2, 5)))
    np.testing.assert_allclose(out[:, 1:], np.cumsum(st, axis=1)[:, :-1], atol=1e-12)
    np.testing.assert_allclose(fin, st.sum(axis=1), atol=1e-12)


def test_state_passing_seq_idx_resets():
    rng = np.random.default_rng(8)
    Q, nc, H, D = 4, 5, 2, 3
    st = rng.standard_normal((1, nc, H, D))
    dAc = -rng.uniform(0, 1, (1, H, nc))
    # chunk ends: pos 3 (seq 0), 7 (1), 11 (1), 15 (2), 19 (2)
    seq = np.array([[0] * 6 + [1] * 6 + [2] * 8])
    out, fin = O.state_passing(st, dAc, None, seq_idx=seq, chunk_size=Q)
    s = np.zeros((H, D))
    want = []
    keep = [1, 0, 1, 0, 1]        # end seq equals the previous chunk-end seq (prev of chunk 0 is 0)
    for c in range(nc):
        want.append(s.copy())
        s = keep[c] * np.exp(dAc[0, :, c])[:, None] * s + st[0, c]
    np.testing.assert_allclose(out[0], np.stack(want), atol=1e-12)
    np.testing.assert_allclose(fin[0], s, atol=1e-12)


# ---------------------------------------------------------------------------
# bmm_chunk
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("causal,seq", [(False, False), (True, False), (True, True)])
def test_bmm_chunk_loops(causal, seq):
    rng = np.random.default_rng(9)
    b, L, G, K, Q = 2, 19, 2, 6, 8
    Cm = rng.standard_normal((b, L, G, K))
    Bm = rng.standard_normal((b, L, G, K))
    seq_idx = np.array([[0] * 9 + [1] * 10, [0] * 3 + [1] * 16]) if seq else None
    got = O.bmm_chunk(Cm, Bm, Q, seq_idx=seq_idx, causal=causal)
    nc = 3
    for bi in range(b):
        for c in range(nc):
            for g in range(G):
                for i in range(Q):
                    for j in range(Q):
                        ti, tj = c * Q + i, c * Q + j
                        v = 0.0
                        if ti < L and tj < L:
                            v = float(np.dot(Cm[bi, ti, g], Bm[bi, tj, g]))
                        if causal and j > i:
                            v = 0.0
                        if seq and ti < L and tj < L and seq_idx[bi, ti] != seq_idx[bi, tj]:
                            v = 0.0
                        assert got[bi, c, g, i, j] == pytest.approx(v, abs=1e-12)


# ---------------------------------------------------------------------------
# The whole SSD == the token-by-token recurrence
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("L,Q,init,z,Dhp", [
    (32, 8, False, False, False),
    (37, 8, True, True, False),      # L % Q != 0, initial state, gate
    (40, 16, True, False, True),     # D per (head, headdim)
    (24, 1, False, True, False),     # chunk_size 1
])
def test_ssd_combined_equals_recurrence(L, Q, init, z, Dhp):
    rng = np.random.default_rng(10 + L + Q)
    b, H, G, P, N = 2, 4, 2, 3, 5
    d = _rand_inputs(rng, b, L, H, G, P, N, with_z=z, init=init)
    if Dhp:
        d["D"] = rng.uniform(0.5, 1.5, (H, P))
    y, fin = O.ssd_combined(chunk_size=Q, dt_softplus=True, return_final_states=True,
                            io_dtype=None, **d)
    ys, hs = O.ssd_sequential(dt_softplus=True, **d)
    np.testing.assert_allclose(y, ys, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(fin, hs, rtol=1e-10, atol=1e-10)


def test_ssd_combined_chunk_size_invariance():
    rng = np.random.default_rng(11)
    d = _rand_inputs(rng, 1, 64, 4, 1, 4, 6, init=True)
    outs = [O.ssd_combined(chunk_size=q, dt_softplus=True, return_final_states=True,
                           io_dtype=None, **d) for q in (4, 16, 64)]
    for y, f in outs[1:]:
        np.testing.assert_allclose(y, outs[0][0], rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(f, outs[0][1], rtol=1e-10, atol=1e-10)


def test_naive_padding_quirk_only_changes_final_state():
    rng = np.random.default_rng(12)
    d = _rand_inputs(rng, 1, 20, 2, 1, 3, 4)
    yk, fk = O.ssd_combined(chunk_size=8, dt_softplus=True, return_final_states=True,
                            io_dtype=None, pad="kernel", **d)
    yn, fn = O.ssd_combined(chunk_size=8, dt_softplus=True, return_final_states=True,
                            io_dtype=None, pad="naive", **d)
    np.testing.assert_allclose(yk, yn, rtol=1e-12, atol=1e-12)
    assert np.max(np.abs(fk - fn)) > 1e-3


# ---------------------------------------------------------------------------
# seq_idx / varlen == independent per-sequence runs
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("lens,Q", [([5, 11, 8], 8), ([8, 8, 8], 8), ([3, 20], 16), ([24], 8)])
def test_packed_sequences_equal_independent_runs(lens, Q):
    rng = np.random.default_rng(13 + Q + len(lens))
    L = sum(lens)
    H, G, P, N = 4, 2, 3, 5
    d = _rand_inputs(rng, 1, L, H, G, P, N, with_z=True)
    seq_idx = np.repeat(np.arange(len(lens)), lens)[None]
    cu = np.concatenate([[0], np.cumsum(lens)])
    y, fin, vs = O.ssd_combined(chunk_size=Q, dt_softplus=True, seq_idx=seq_idx,
                                cu_seqlens=cu, return_final_states=True,
                                return_varlen_states=True, io_dtype=None, **d)
    # packed recurrence with resets
    ys, hs = O.ssd_sequential(seq_idx=seq_idx, dt_softplus=True, **d)
    np.testing.assert_allclose(y, ys, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(fin, hs, rtol=1e-10, atol=1e-10)
    for s in range(len(lens)):
        sl = slice(cu[s], cu[s + 1])
        part = {k: (v[:, sl] if k in ("x", "dt", "B", "C", "z") else v)
                for k, v in d.items() if k != "initial_states"}
        yi, hi = O.ssd_sequential(dt_softplus=True, **part)
        np.testing.assert_allclose(y[:, sl], yi, rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(vs[s], hi[0], rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------------------
# decode step
# ---------------------------------------------------------------------------

def test_ssu_closed_form():
    rng = np.random.default_rng(14)
    b, H, G, P, N = 2, 4, 2, 8, 16
    state = rng.standard_normal((b, H, P, N))
    x = rng.standard_normal((b, H, P))
    dt = rng.standard_normal((b, H))
    A = -np.abs(rng.standard_normal(H))
    Bm = rng.standard_normal((b, G, N))
    Cm = rng.standard_normal((b, G, N))
    D = rng.standard_normal(H)
    z = rng.standard_normal((b, H, P))
    bias = rng.standard_normal(H)
    new, out = O.selective_state_update(state, x, dt, A, Bm, Cm, D=D, z=z,
                                        dt_bias=bias, dt_softplus=True)
    for bi in range(b):
        for h in range(H):
            g = h // (H // G)
            d_ = math.log1p(math.exp(dt[bi, h] + bias[h]))
            for p in range(P):
                row = state[bi, h, p] * math.exp(d_ * A[h]) + d_ * x[bi, h, p] * Bm[bi, g]
                np.testing.assert_allclose(new[bi, h, p], row, rtol=1e-13, atol=1e-13)
                y = float(row @ Cm[bi, g]) + D[h] * x[bi, h, p]
                zz = z[bi, h, p]
                y *= zz / (1 + math.exp(-zz))
                assert out[bi, h, p] == pytest.approx(y, rel=1e-12, abs=1e-12)


def test_ssu_steps_equal_prefill():
    rng = np.random.default_rng(15)
    b, L, H, G, P, N = 2, 12, 4, 2, 3, 5
    d = _rand_inputs(rng, b, L, H, G, P, N, with_z=True, init=True)
    y, fin = O.ssd_combined(chunk_size=4, dt_softplus=True, return_final_states=True,
                            io_dtype=None, **d)
    s = d["initial_states"]
    for t in range(L):
        s, yt = O.selective_state_update(
            s, d["x"][:, t], d["dt"][:, t], d["A"], d["B"][:, t], d["C"][:, t],
            D=d["D"], z=d["z"][:, t], dt_bias=d["dt_bias"], dt_softplus=True)
        np.testing.assert_allclose(yt, y[:, t], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(s, fin, rtol=1e-10, atol=1e-10)


def test_ssu_per_headdim_params():
    rng = np.random.default_rng(16)
    b, H, G, P, N = 1, 2, 1, 3, 4
    state = rng.standard_normal((b, H, P, N))
    x = rng.standard_normal((b, H, P))
    dt = rng.standard_normal((b, H, P))
    A = -np.abs(rng.standard_normal((H, P, N)))
    Bm = rng.standard_normal((b, G, N))
    Cm = rng.standard_normal((b, G, N))
    D = rng.standard_normal((H, P))
    bias = rng.standard_normal((H, P))
    new, out = O.selective_state_update(state, x, dt, A, Bm, Cm, D=D, dt_bias=bias,
                                        dt_softplus=True)
    for h in range(H):
        for p in range(P):
            d_ = math.log1p(math.exp(dt[0, h, p] + bias[h, p]))
            row = state[0, h, p] * np.exp(d_ * A[h, p]) + d_ * x[0, h, p] * Bm[0, 0]
            np.testing.assert_allclose(new[0, h, p], row, rtol=1e-13)
            assert out[0, h, p] == pytest.approx(row @ Cm[0, 0] + D[h, p] * x[0, h, p], rel=1e-12)


# ---------------------------------------------------------------------------
# the bf16 rounding points the oracle reproduces stay inside the tolerance
# ---------------------------------------------------------------------------

def test_bf16_rounding_points_are_small_but_present():
    cfg = configs.SSDConfig("t", 1, 256, 4, 1, 16, 32, 64, "bf16", seed=5)
    d = configs.make_ssd_inputs(cfg)
    kw = dict(chunk_size=64, dt_softplus=True, return_final_states=True)
    y0, f0 = O.ssd_combined(io_dtype=None, **kw, **d)
    y1, f1 = O.ssd_combined(io_dtype="bf16", **kw, **d)
    e = O.rel_err(y1, y0)
    assert 1e-5 < e < 2e-2
    assert O.rel_err(f1, f0) == 0.0   # final states stay fp32


def test_passed_jitter_is_a_measurement_knob_only():
    """passed_jitter (a test-only knob of the oracle) leaves results untouched
    at 0, and in fp32 (no rounding of the passed states) moves them by about
    the jitter itself: it perturbs the passed states and nothing else."""
    rng = np.random.default_rng(5)
    b, L, H, G, P, N, Q = 1, 96, 2, 1, 8, 16, 32
    x = rng.standard_normal((b, L, H, P)).astype(np.float32)
    dt = (0.1 * rng.random((b, L, H))).astype(np.float32)
    A = -rng.uniform(0.5, 2.0, H).astype(np.float32)
    B = rng.standard_normal((b, L, G, N)).astype(np.float32)
    C = rng.standard_normal((b, L, G, N)).astype(np.float32)
    seq = np.repeat([0, 1], [40, 56])[None].astype(np.int32)
    cu = np.array([0, 40, 96], np.int32)
    kw = dict(chunk_size=Q, seq_idx=seq, cu_seqlens=cu, return_final_states=True,
              return_varlen_states=True)
    base = O.ssd_combined(x, dt, A, B, C, **kw)
    same = O.ssd_combined(x, dt, A, B, C, **kw, passed_jitter=0.0, jitter_seed=7)
    for a, c in zip(base, same):
        assert np.array_equal(a, c)
    jit = O.ssd_combined(x, dt, A, B, C, **kw, passed_jitter=1e-6, jitter_seed=7)
    assert 0 < O.rel_err(jit[2], base[2]) < 1e-5        # varlen states use the passed states
    assert O.rel_err(jit[0], base[0]) < 1e-5            # so do the outputs
    assert np.array_equal(jit[1], base[1])              # the final states do not

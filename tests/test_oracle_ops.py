"""Pins of the CPU oracle for causal_conv1d, causal_conv1d_update and
rms_norm_gated (oracle/ops_oracle.py) against the reference tests' closed
forms (reference tests/test_mamba2_ops.py:115-296), hand-worked cases and
independent formulations.  CPU only."""

import numpy as np
import pytest

from oracle import ops_oracle as X
from oracle.ssd_oracle import bf16_round


def _rng(seed=0):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("shape", [(2, 8, 16, 4), (1, 4, 8, 3), (3, 5, 7, 8), (1, 2, 3, 4)])
def test_conv_matches_manual_conv(shape):
    """reference tests/test_mamba2_ops.py:115-143: pad and convolve by hand."""
    b, d, L, k = shape
    r = _rng(1)
    x, w, bias = r.standard_normal((b, d, L)), r.standard_normal((d, k)), r.standard_normal(d)
    got, dt = X.causal_conv1d(x, w, bias)
    assert dt == "float32"
    np.testing.assert_allclose(got, X.causal_conv1d_brute(x, w, bias), rtol=1e-12, atol=1e-12)
    # (d, 1, k) weights are the same conv
    got3, _ = X.causal_conv1d(x, w[:, None, :], bias)
    np.testing.assert_array_equal(got3, got)


def test_conv_silu_after_conv():
    """reference tests/test_mamba2_ops.py:146-166."""
    r = _rng(7)
    x, w = r.standard_normal((1, 4, 8)), r.standard_normal((4, 3))
    plain, _ = X.causal_conv1d(x, w)
    act, _ = X.causal_conv1d(x, w, activation="silu")
    np.testing.assert_allclose(act, plain / (1 + np.exp(-plain)), rtol=1e-14)


def test_conv_closed_forms():
    r = _rng(2)
    x = r.standard_normal((2, 3, 10))
    # width 1: y = w x + b
    w1, b = r.standard_normal((3, 1)), r.standard_normal(3)
    got, _ = X.causal_conv1d(x, w1, b)
    np.testing.assert_allclose(got, w1[None, :, 0, None] * x + b[None, :, None], rtol=1e-14)
    # a unit tap at the last position is the identity, at the first a shift by k - 1
    k = 4
    e_last = np.zeros((3, k)); e_last[:, -1] = 1
    np.testing.assert_array_equal(X.causal_conv1d(x, e_last)[0], x)
    e_first = np.zeros((3, k)); e_first[:, 0] = 1
    shifted = np.zeros_like(x); shifted[:, :, k - 1:] = x[:, :, :-(k - 1)]
    np.testing.assert_array_equal(X.causal_conv1d(x, e_first)[0], shifted)


def test_sequence_boundary_mask_hand_worked():
    """seq = 0 0 0 1 1 2 2 2, width 3: sequence starts at 3 and 5; lag 1 zeroes
    positions 2 and 4, lag 2 zeroes 1 and 3 (reference ops/causal_conv1d.py:186-191)."""
    seq = np.array([[0, 0, 0, 1, 1, 2, 2, 2]])
    np.testing.assert_array_equal(X.sequence_boundary_mask(seq, 3)[0], [1, 0, 0, 0, 0, 1, 1, 1])
    # width 1: nothing is masked; one sequence: nothing is masked
    np.testing.assert_array_equal(X.sequence_boundary_mask(seq, 1)[0], np.ones(8))
    np.testing.assert_array_equal(X.sequence_boundary_mask(np.zeros((1, 8)), 4)[0], np.ones(8))
    # a sequence of one token between two others: width 2 zeroes the token
    # before each start, i.e. positions 1 and 2
    np.testing.assert_array_equal(
        X.sequence_boundary_mask(np.array([[5, 5, 7, 5, 5]]), 2)[0], [1, 0, 0, 1, 1])
    # the masked conv equals the plain conv of the masked input
    r = _rng(3)
    x, w = r.standard_normal((1, 2, 8)), r.standard_normal((2, 3))
    got, _ = X.causal_conv1d(x, w, seq_idx=seq)
    want = X.causal_conv1d_brute(x * np.array([1, 0, 0, 0, 0, 1, 1, 1.0]), w)
    np.testing.assert_allclose(got, want, rtol=1e-14)


def test_conv_bf16_rounding_points():
    """bf16 x and weight: the conv result is rounded; an f32 bias promotes the rest."""
    r = _rng(4)
    x = bf16_round(r.standard_normal((1, 4, 12)))
    w = bf16_round(r.standard_normal((4, 4)))
    b32 = r.standard_normal(4).astype(np.float32)
    got, dt = X.causal_conv1d(x, w, b32, x_dtype="bfloat16", w_dtype="bfloat16")
    assert dt == "float32"
    conv = bf16_round(X.causal_conv1d_brute(x, w)).astype(np.float64)
    np.testing.assert_array_equal(got, conv + b32.astype(np.float64)[None, :, None])
    got, dt = X.causal_conv1d(x, w, bf16_round(b32), "silu", x_dtype="bfloat16",
                              w_dtype="bfloat16", bias_dtype="bfloat16")
    assert dt == "bfloat16"
    np.testing.assert_array_equal(got, bf16_round(got))


@pytest.mark.parametrize("width", [1, 3, 4])
def test_update_matches_full_conv(width):
    """reference tests/test_mamba2_ops.py:169-202: steps from a zero state
    reproduce the full conv at every position."""
    r = _rng(99)
    b, d, L = 2, 8, 10
    x, w, bias = r.standard_normal((b, d, L)), r.standard_normal((d, width)), r.standard_normal(d)
    full, _ = X.causal_conv1d(x, w, bias, "silu")
    state = np.zeros((b, d, width))
    for t in range(L):
        state, out, _, _ = X.causal_conv1d_update(x[:, :, t], state, w, bias, "silu")
        np.testing.assert_allclose(out, full[:, :, t], rtol=1e-12, atol=1e-14)
    # the state holds the last `width` inputs
    want = np.concatenate([np.zeros((b, d, max(0, width - L))), x[:, :, max(0, L - width):]], 2)
    np.testing.assert_array_equal(state, want)


def _rms_closed(x, w, eps=1e-5):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def test_rms_norm_closed_forms():
    """reference tests/test_mamba2_ops.py:205-261."""
    r = _rng(42)
    x, z, w = r.standard_normal((2, 16)), r.standard_normal((2, 16)), r.standard_normal(16)
    got, _ = X.rms_norm_gated(x, np.ones(16))
    np.testing.assert_allclose(got, _rms_closed(x, 1.0), rtol=1e-13)
    sz = z / (1 + np.exp(-z))
    got, _ = X.rms_norm_gated(x, w, z=z, norm_before_gate=True)
    np.testing.assert_allclose(got, _rms_closed(x, w) * sz, rtol=1e-13)
    got, _ = X.rms_norm_gated(x, w, z=z, norm_before_gate=False)
    np.testing.assert_allclose(got, _rms_closed(x * sz, w), rtol=1e-13)


@pytest.mark.parametrize("nbg", [True, False])
def test_rms_norm_grouped_is_per_group(nbg):
    """reference tests/test_mamba2_ops.py:264-290: a grouped norm equals the
    ungrouped norm applied to each group separately; with eps = 0 the norm is
    invariant to scaling a group."""
    r = _rng(5)
    x, z, w = r.standard_normal((3, 32)), r.standard_normal((3, 32)), r.standard_normal(32)
    got, _ = X.rms_norm_gated(x, w, z=z, group_size=8, norm_before_gate=nbg)
    for g in range(4):
        sl = slice(8 * g, 8 * g + 8)
        want, _ = X.rms_norm_gated(x[:, sl], w[sl], z=z[:, sl], norm_before_gate=nbg)
        np.testing.assert_allclose(got[:, sl], want, rtol=1e-13)
    scale = np.repeat(r.uniform(0.5, 3.0, (3, 4)), 8, axis=1)
    a, _ = X.rms_norm_gated(x, w, group_size=8, eps=0.0)
    b, _ = X.rms_norm_gated(x * scale, w, group_size=8, eps=0.0)
    np.testing.assert_allclose(a, b, rtol=1e-12)


def test_promote():
    assert X.promote("bfloat16", "bfloat16") == "bfloat16"
    assert X.promote("bfloat16", "float32") == "float32"
    assert X.promote("bfloat16", None) == "bfloat16"


def _layer_params(rng, d_model=16, d_state=8, d_conv=4, expand=2, headdim=8, ngroups=2,
                  d_ssm=None, D_has_hdim=False, bias=False):
    d_inner = expand * d_model
    dssm = d_inner if d_ssm is None else d_ssm
    H = dssm // headdim
    conv_dim = dssm + 2 * ngroups * d_state
    d_in_proj = 2 * d_inner + 2 * ngroups * d_state + H
    p = {"in_proj_kernel": rng.standard_normal((d_model, d_in_proj)) / np.sqrt(d_model),
         "out_proj_kernel": rng.standard_normal((d_inner, d_model)) / np.sqrt(d_inner),
         "conv1d_weight": rng.standard_normal((conv_dim, d_conv)) / 2,
         "conv1d_bias": rng.standard_normal(conv_dim) * 0.1,
         "dt_bias": np.log(np.expm1(rng.uniform(0.01, 0.1, H))),
         "A_log": np.log(rng.uniform(1, 16, H)),
         "D": rng.uniform(0.5, 1.5, dssm if D_has_hdim else H),
         "norm_weight": rng.uniform(0.5, 1.5, dssm)}
    if bias:
        p["in_proj_bias"] = rng.standard_normal(d_in_proj) * 0.1
        p["out_proj_bias"] = rng.standard_normal(d_model) * 0.1
    cfg = dict(d_ssm=dssm, d_mlp=d_inner - dssm, ngroups=ngroups, d_state=d_state, headdim=headdim,
               nheads=H, chunk_size=8, rmsnorm=True, norm_before_gate=False,
               D_has_hdim=D_has_hdim, dt_limit=(0.0, float("inf")))
    return p, cfg


@pytest.mark.parametrize("variant", ["plain", "mlp+bias+Dhdim", "no-rmsnorm"])
def test_layer_prefill_equals_decode_steps(variant):
    """reference tests/test_mamba2_vs_torch.py:312-408: the layer's chunked
    prefill over T tokens equals T decode steps (conv update + token
    recurrence) from zero states, output by output, and ends in the same states."""
    rng = _rng(11)
    kw = {"plain": {}, "mlp+bias+Dhdim": dict(d_ssm=16, D_has_hdim=True, bias=True),
          "no-rmsnorm": {}}[variant]
    p, cfg = _layer_params(rng, **kw)
    if variant == "no-rmsnorm":
        cfg["rmsnorm"] = False
    b, T = 2, 21
    u = rng.standard_normal((b, T, 16))
    full, fin, conv_state = X.mamba2_layer(p, u, cfg)
    cs = np.zeros_like(conv_state)
    ss = np.zeros((b, cfg["nheads"], cfg["headdim"], cfg["d_state"]))
    # the chunked path rounds the passed states, CB and C @ states to the
    # input dtype (float32 here) as the reference does, so agreement is to
    # ~1e-7 of the output scale
    scale = np.sqrt(np.mean(full ** 2))
    for t in range(T):
        out, cs, ss = X.mamba2_layer_step(p, u[:, t], cs, ss, cfg)
        assert np.max(np.abs(out - full[:, t])) <= 1e-6 * scale, t
    assert np.max(np.abs(ss - fin)) <= 1e-6 * np.sqrt(np.mean(fin ** 2))
    np.testing.assert_array_equal(cs, conv_state)

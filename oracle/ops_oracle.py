"""CPU oracle for the ops on either side of the SSD: causal_conv1d (prefill),
causal_conv1d_update (decode) and rms_norm_gated.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker -- never as a product path.  The product (``mamba2_jax``) runs the HIP
kernels in ``libm2ssd.so`` and has no CPU path.

NumPy restatement of
  * ``/root/reference/src/mamba2_jax/modules/mamba2.py:296-549`` (the mixer
    layer, composed from the pieces below);
  * ``/root/reference/src/mamba2_jax/ops/causal_conv1d.py`` (causal_conv1d
    :18-85, causal_conv1d_update :88-139, _mask_sequence_boundaries :142-193);
  * ``/root/reference/src/mamba2_jax/ops/rms_norm.py:15-92`` (rms_norm_gated).
Arithmetic runs in float64 (``acc``); bf16 rounding points follow the dtype
each JAX expression has (``bf16_round`` at every place where the reference's
intermediate array is bfloat16).

How each function is pinned (tests/test_oracle_ops.py):
  causal_conv1d         the reference's manual pad-and-convolve loop
                        (tests/test_mamba2_ops.py:131-138) restated as a
                        brute-force loop; silu applied after the conv
                        (:159-163); width 1 closed form; a delta kernel is a
                        shift; the seq_idx mask against a hand-worked example
  causal_conv1d_update  T updates from a zero state == the full conv at every
                        position (the reference's own test, :169-202); the
                        shifted state is the last ``width`` inputs
  rms_norm_gated        the reference tests' closed forms
                        (tests/test_mamba2_ops.py:205-296): plain, gated before
                        and after the norm, grouped; scale invariance
  mamba2_layer          a composition of the pinned pieces; prefill of T tokens
                        == T decode steps through the conv update and the
                        token recurrence (tests/test_oracle_ops.py)
"""

from __future__ import annotations

import numpy as np

from .ssd_oracle import bf16_round, identity


def _rf(is_bf16):
    return bf16_round if is_bf16 else identity


def promote(*names):
    """JAX's result type for a mix of 'float32' / 'bfloat16' arrays."""
    names = [n for n in names if n is not None]
    return "bfloat16" if names and all(n == "bfloat16" for n in names) else "float32"


def silu(v, is_bf16=False):
    """jax.nn.silu in the array's dtype: computed exactly, rounded once."""
    v = np.asarray(v, dtype=np.float64)
    return _rf(is_bf16)(v / (1.0 + np.exp(-v))).astype(np.float64)


# ---------------------------------------------------------------------------
# causal_conv1d  (reference ops/causal_conv1d.py)
# ---------------------------------------------------------------------------

def sequence_boundary_mask(seq_idx, width):
    """mask[b, s] = 0 where the reference zeroes x[:, :, s] (:142-193).

    boundary[t] = (t == 0) or seq[t] != seq[t-1] (:171-177); for every lag
    j = 1 .. width-1, position s is zeroed when boundary[s + j] holds with
    s + j < L (:186-191).  So the last width-1 positions before each sequence
    start are zeroed for every output (including outputs of their own
    sequence), as the reference does.
    """
    seq = np.asarray(seq_idx)
    b, L = seq.shape
    boundary = np.ones((b, L), dtype=bool)
    boundary[:, 1:] = seq[:, 1:] != seq[:, :-1]
    mask = np.ones((b, L), dtype=np.float64)
    for j in range(1, width):
        shifted = np.zeros((b, L), dtype=bool)
        if j < L:
            shifted[:, :L - j] = boundary[:, j:]
        mask = mask * (1.0 - shifted)
    return mask


def causal_conv1d(x, weight, bias=None, activation=None, seq_idx=None,
                  x_dtype="float32", w_dtype="float32", bias_dtype="float32"):
    """-> (out (batch, d, L) float64 holding values of the result dtype, dtype name).

    x (batch, d, L); weight (d, width) or (d, 1, width); bias (d,).
    out[t] = sum_i w[i] * xm[t - width + 1 + i] (xm: x with the seq_idx mask
    applied, zero before position 0) (:67-76); + bias (:78-79); silu (:81-82).
    The conv's result dtype is promote(x, weight) (rounded once: the conv
    accumulates in float32 and rounds its output); the bias add and silu each
    round to their dtype.
    """
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    if w.ndim == 3:
        w = w[:, 0, :]
    b, d, L = x.shape
    width = w.shape[1]
    if seq_idx is not None:
        x = x * sequence_boundary_mask(seq_idx, width)[:, None, :]
    xp = np.concatenate([np.zeros((b, d, width - 1)), x], axis=2)
    out = np.zeros((b, d, L))
    for i in range(width):
        out += w[None, :, i, None] * xp[:, :, i:i + L]
    dt = promote(x_dtype, w_dtype)
    out = _rf(dt == "bfloat16")(out).astype(np.float64)
    if bias is not None:
        dt = promote(dt, bias_dtype)
        out = _rf(dt == "bfloat16")(out + np.asarray(bias, np.float64)[None, :, None])
        out = np.asarray(out, np.float64)
    if activation == "silu":
        out = silu(out, dt == "bfloat16")
    return out, dt


def causal_conv1d_brute(x, weight, bias=None):
    """The reference test's manual conv (tests/test_mamba2_ops.py:131-138) as
    a per-position loop: an independent restatement used to pin causal_conv1d."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    b, d, L = x.shape
    k = w.shape[1]
    out = np.zeros((b, d, L))
    for t in range(L):
        for i in range(k):
            s = t - k + 1 + i
            if s >= 0:
                out[:, :, t] += w[None, :, i] * x[:, :, s]
        if bias is not None:
            out[:, :, t] += np.asarray(bias, np.float64)[None, :]
    return out


def causal_conv1d_update(x_new, conv_state, weight, bias=None, activation=None,
                         x_dtype="float32", state_dtype="float32", w_dtype="float32",
                         bias_dtype="float32"):
    """-> (new_state (b, d, width), out (b, d), state dtype name, out dtype name).

    new_state = concat(state[:, :, 1:], x_new) in promote(state, x) (:123-127);
    out = sum(new_state * w, -1) (:130) in promote(state dtype, w): with bf16
    products each product is rounded, the sum accumulated and rounded once;
    + bias (:132-133); silu (:135-136).
    """
    s = np.asarray(conv_state, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    if w.ndim == 3:
        w = w[:, 0, :]
    sdt = promote(state_dtype, x_dtype)
    new_state = np.concatenate([s[:, :, 1:], np.asarray(x_new, np.float64)[:, :, None]], axis=2)
    new_state = _rf(sdt == "bfloat16")(new_state).astype(np.float64)
    dt = promote(sdt, w_dtype)
    r = _rf(dt == "bfloat16")
    out = r(np.sum(np.asarray(r(new_state * w[None]), np.float64), axis=-1)).astype(np.float64)
    if bias is not None:
        dt = promote(dt, bias_dtype)
        out = np.asarray(_rf(dt == "bfloat16")(out + np.asarray(bias, np.float64)[None, :]),
                         np.float64)
    if activation == "silu":
        out = silu(out, dt == "bfloat16")
    return new_state, out, sdt, dt


# ---------------------------------------------------------------------------
# rms_norm_gated  (reference ops/rms_norm.py:15-92)
# ---------------------------------------------------------------------------

def rms_norm_gated(x, weight, z=None, eps=1e-5, group_size=None, norm_before_gate=True,
                   x_dtype="float32", w_dtype="float32", z_dtype="float32"):
    """-> (out, dtype name).

    Over each group of ``group_size`` trailing elements (the whole row when
    None): with z and not norm_before_gate, x = x * silu(z) first (:64-66,
    :80-83); rms = sqrt(mean(x^2) + eps); out = x / rms * weight (:70-71,
    :87-92); with z and norm_before_gate, out *= silu(z) (:73-74, :94-95).
    silu(z) has z's dtype; every product's dtype is the promotion of its
    operands (bf16 only when all of them are bf16).
    """
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    hidden = x.shape[-1]
    gs = hidden if group_size is None else group_size
    assert hidden % gs == 0
    xdt = x_dtype
    zb = z_dtype == "bfloat16"
    if z is not None and not norm_before_gate:
        xdt = promote(x_dtype, z_dtype)
        x = np.asarray(_rf(xdt == "bfloat16")(x * silu(z, zb)), np.float64)
    r = _rf(xdt == "bfloat16")
    xg = x.reshape(*x.shape[:-1], hidden // gs, gs)
    # mean(x*x) + eps, sqrt and the division each round to x's dtype
    ms = np.asarray(r(np.mean(np.asarray(r(xg * xg), np.float64), axis=-1, keepdims=True)),
                    np.float64)
    rms = np.asarray(r(np.sqrt(np.asarray(r(ms + eps), np.float64))), np.float64)
    xn = np.asarray(r(xg / rms), np.float64).reshape(x.shape)
    dt = promote(xdt, w_dtype)
    out = np.asarray(_rf(dt == "bfloat16")(xn * w), np.float64)
    if z is not None and norm_before_gate:
        dt = promote(dt, z_dtype)
        out = np.asarray(_rf(dt == "bfloat16")(out * silu(z, zb)), np.float64)
    return out, dt


# ---------------------------------------------------------------------------
# Mamba2 mixer layer (reference modules/mamba2.py:296-549), float32 weights
# ---------------------------------------------------------------------------

def mamba2_layer(p, u, cfg, seq_idx=None, dtype="float32"):
    """Prefill of one Mamba2 layer from the oracle pieces above and
    ssd_oracle.ssd_combined: in-projection, conv + SiLU, SSD, gated RMSNorm,
    MLP bypass, out-projection (reference modules/mamba2.py:296-414).

    p: parameter arrays by reference name; cfg: dict with d_ssm, d_mlp,
    ngroups, d_state, headdim, nheads, chunk_size, rmsnorm, norm_before_gate,
    D_has_hdim, dt_limit.  dtype: the parameters' (and so the activations')
    dtype; with "bfloat16" the projections' outputs, the conv and the SSD's
    internal casts are rounded to bf16 and the norm output is cast to bf16
    before the out-projection, as the reference's arrays are.
    Returns (out, final_states, conv_state).
    """
    from .ssd_oracle import ssd_combined
    bf = dtype == "bfloat16"
    r = _rf(bf)
    u = np.asarray(u, np.float64)
    b, L, _ = u.shape
    dssm, dmlp, G, N = cfg["d_ssm"], cfg["d_mlp"], cfg["ngroups"], cfg["d_state"]
    H, P = cfg["nheads"], cfg["headdim"]
    zx = np.asarray(r(u @ np.asarray(p["in_proj_kernel"], np.float64)), np.float64)
    if p.get("in_proj_bias") is not None:
        zx = np.asarray(r(zx + p["in_proj_bias"]), np.float64)
    o = np.cumsum([0, dmlp, dmlp, dssm, dssm + 2 * G * N, H])
    z0, x0, z, xBC, dt = (zx[..., o[i]:o[i + 1]] for i in range(5))
    d_conv = p["conv1d_weight"].shape[1]
    xT = xBC.transpose(0, 2, 1)
    conv_state = (xT[:, :, -d_conv:] if L >= d_conv
                  else np.concatenate([np.zeros((b, xT.shape[1], d_conv - L)), xT], 2))
    xc, _ = causal_conv1d(xT, p["conv1d_weight"], p.get("conv1d_bias"), "silu", seq_idx,
                          dtype, dtype, dtype)
    xc = xc.transpose(0, 2, 1)
    x = xc[..., :dssm].reshape(b, L, H, P)
    B = xc[..., dssm:dssm + G * N].reshape(b, L, G, N)
    C = xc[..., dssm + G * N:].reshape(b, L, G, N)
    A = -np.exp(np.asarray(p["A_log"], np.float64))
    D = np.asarray(p["D"], np.float64)
    if cfg["D_has_hdim"]:
        D = D.reshape(H, P)
    zs = None if cfg["rmsnorm"] else z.reshape(b, L, H, P)
    y, fin = ssd_combined(x, dt, A, B, C, cfg["chunk_size"], D=D, z=zs, dt_bias=p["dt_bias"],
                          seq_idx=seq_idx, dt_softplus=True, dt_limit=cfg["dt_limit"],
                          return_final_states=True, io_dtype="bf16" if bf else "f32")
    y = y.reshape(b, L, dssm)
    if cfg["rmsnorm"]:
        y, _ = rms_norm_gated(y, p["norm_weight"], z=z, group_size=dssm // G,
                              norm_before_gate=cfg["norm_before_gate"], w_dtype=dtype,
                              z_dtype=dtype)
    if dmlp > 0:
        y = np.concatenate([r(silu(z0, bf) * x0), y], -1)
    y = np.asarray(r(y), np.float64)                  # cast to the out-projection's dtype
    out = np.asarray(r(y @ np.asarray(p["out_proj_kernel"], np.float64)), np.float64)
    if p.get("out_proj_bias") is not None:
        out = np.asarray(r(out + p["out_proj_bias"]), np.float64)
    return out, fin, conv_state


def mamba2_layer_step(p, u_t, conv_state, ssm_state, cfg):
    """One decode token of the layer (reference modules/mamba2.py:427-549):
    the conv update, the selective state update (no dt_limit clamp, as the
    reference's decode), the gated norm and the projections.
    u_t (b, d_model) -> (out (b, d_model), new conv_state, new ssm_state)."""
    from .ssd_oracle import selective_state_update
    u_t = np.asarray(u_t, np.float64)
    b = u_t.shape[0]
    dssm, dmlp, G, N = cfg["d_ssm"], cfg["d_mlp"], cfg["ngroups"], cfg["d_state"]
    H, P = cfg["nheads"], cfg["headdim"]
    zx = u_t @ np.asarray(p["in_proj_kernel"], np.float64)
    if p.get("in_proj_bias") is not None:
        zx = zx + p["in_proj_bias"]
    o = np.cumsum([0, dmlp, dmlp, dssm, dssm + 2 * G * N, H])
    z0, x0, z, xBC, dt = (zx[..., o[i]:o[i + 1]] for i in range(5))
    conv_state, xc, _, _ = causal_conv1d_update(xBC, conv_state, p["conv1d_weight"],
                                                p.get("conv1d_bias"), "silu")
    A = -np.exp(np.asarray(p["A_log"], np.float64))
    D = np.asarray(p["D"], np.float64)
    if cfg["D_has_hdim"]:
        D = D.reshape(H, P)
    zs = None if cfg["rmsnorm"] else z.reshape(b, H, P)
    ssm_state, y = selective_state_update(
        ssm_state, xc[:, :dssm].reshape(b, H, P), dt, A, xc[:, dssm:dssm + G * N].reshape(b, G, N),
        xc[:, dssm + G * N:].reshape(b, G, N), D=D, z=zs, dt_bias=p["dt_bias"], dt_softplus=True)
    y = y.reshape(b, dssm)
    if cfg["rmsnorm"]:
        y, _ = rms_norm_gated(y, p["norm_weight"], z=z, group_size=dssm // G,
                              norm_before_gate=cfg["norm_before_gate"])
    if dmlp > 0:
        y = np.concatenate([z0 / (1 + np.exp(-z0)) * x0, y], -1)
    out = y @ np.asarray(p["out_proj_kernel"], np.float64)
    if p.get("out_proj_bias") is not None:
        out = out + p["out_proj_bias"]
    return out, conv_state, ssm_state


def mamba2_lm(params, input_ids, mcfg, eps=1e-5):
    """Logits of the Mamba2 LM (reference models/mamba2_lm.py:178-217) from
    float32 parameters: embedding, per layer residual + mixer(rmsnorm(x)),
    final rmsnorm, tied LM head.  params: the reference's nested dict of
    arrays; mcfg: the mixer cfg of mamba2_layer."""
    x = np.asarray(params["embedding"]["weight"], np.float64)[np.asarray(input_ids)]
    for lp in params["layers"]:
        xn, _ = rms_norm_gated(x, lp["norm_weight"], eps=eps)
        out, _, _ = mamba2_layer(lp["mixer"], xn, mcfg)
        x = x + out
    x, _ = rms_norm_gated(x, params["norm_f_weight"], eps=eps)
    return x @ np.asarray(params["lm_head_weight"], np.float64).T

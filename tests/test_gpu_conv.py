"""Parity of causal_conv1d / causal_conv1d_update (HIP) with the CPU oracle.

* the reference tests' cases (tests/test_mamba2_ops.py:115-202);
* every kernel path: channels-first (unit time stride), channels-last (unit
  channel stride, the Mamba2 layer's xBC.transpose(1, 2)), other strides;
  widths 1..8; fp32 / bf16 inputs; bias, silu and seq_idx on and off;
  ragged lengths (seqlen below the width, not a multiple of the vector or run
  size, channel counts that are not a multiple of the vector width);
* the split output (x, B, C of an SSD layer in their own tensors) at the
  nemotron-h-8b layer shape;
* decode: T in-place updates from a zero state == the prefill conv;
  dtype promotion and in-place / copy semantics.
Tolerance: fp32 results 1e-5 relative to the output RMS; bf16 results one
bf16 ulp of each value (the oracle rounds where the reference's arrays are
bf16; the conv's f32 sum order may move a rounding by one ulp).
"""

import zlib

import numpy as np
import pytest
import torch

from gpu_util import announce, dev, host
from mamba2_jax.ops.causal_conv1d import causal_conv1d, causal_conv1d_update
from oracle import ops_oracle as X
from oracle.ssd_oracle import bf16_round

pytestmark = pytest.mark.gpu

NAME = {torch.float32: "float32", torch.bfloat16: "bfloat16"}


def _close(got, want, is_bf16, what, mag=None):
    """bf16: |err| <= 2^-7 (|want| + mag), mag = sum_i |w_i x_i| + |bias| (the
    conv's terms): one ulp of the result plus one ulp of the rounded conv,
    which a bias that cancels it leaves as a large relative error."""
    g = host(got)
    assert g.shape == want.shape, (g.shape, want.shape)
    if is_bf16:
        m = np.abs(want) if mag is None else np.abs(want) + mag
        err = np.abs(g - want) / np.maximum(m, 1e-30)
        bad = np.abs(g - want) > 2.0 ** -7 * m + 1e-30
        print(f"  {what}: max err / (|want| + mag) {err.max():.2e}, beyond tolerance: "
              f"{int(bad.sum())}", flush=True)
        assert not bad.any(), f"{what}: {int(bad.sum())} values beyond one bf16 ulp"
    else:
        e = np.max(np.abs(g - want)) / max(np.sqrt(np.mean(want ** 2)), 1e-30)
        print(f"  {what}: max|err|/rms = {e:.2e}", flush=True)
        assert e <= 1e-5, f"{what}: {e:.2e}"


def _inputs(rng, b, d, L, k, xdt, wdt, bdt, with_bias=True):
    x = rng.standard_normal((b, d, L)).astype(np.float32)
    w = (rng.standard_normal((d, k)) / np.sqrt(k)).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32) if with_bias else None
    rnd = lambda a, t: None if a is None else (bf16_round(a) if t == torch.bfloat16 else a)
    return rnd(x, xdt), rnd(w, wdt), rnd(bias, bdt)


def _mag(x, w, bias):
    """sum_i |w_i| |x_{t-k+1+i}| + |bias| per output, (b, d, L)."""
    return X.causal_conv1d_brute(np.abs(x), np.abs(w), None if bias is None else np.abs(bias))


def _seq(rng, b, L, nseq):
    out = np.zeros((b, L), np.int32)
    for i in range(b):
        cuts = np.sort(rng.choice(np.arange(1, L), size=min(nseq - 1, L - 1), replace=False))
        out[i] = np.searchsorted(cuts, np.arange(L), side="right")
    return out


def _layout(x_t, layout):
    """x_t (b, d, L) contiguous -> the same values in the given memory layout."""
    if layout == "cf":
        return x_t
    if layout == "cl":
        return x_t.transpose(1, 2).contiguous().transpose(1, 2)
    # "strided": every other channel of a wider channels-last buffer
    b, d, L = x_t.shape
    big = torch.zeros((b, L, 2 * d), dtype=x_t.dtype, device=x_t.device)
    big[:, :, ::2] = x_t.transpose(1, 2)
    return big[:, :, ::2].transpose(1, 2)


def test_reference_cases():
    """reference tests/test_mamba2_ops.py:115-166, fp32."""
    rng = np.random.default_rng(42)
    announce("conv reference cases")
    x, w, bias = _inputs(rng, 2, 8, 16, 4, None, None, None)
    want, _ = X.causal_conv1d(x, w, bias)
    _close(causal_conv1d(dev(x), dev(w), dev(bias)), want, False, "basic (2, 8, 16, k 4)")
    x, w, _ = _inputs(rng, 1, 4, 8, 3, None, None, None, with_bias=False)
    plain = causal_conv1d(dev(x), dev(w))
    act = causal_conv1d(dev(x), dev(w), activation="silu")
    _close(act, X.silu(host(plain)), False, "silu after conv")
    _close(act, X.causal_conv1d(x, w, activation="silu")[0], False, "silu (1, 4, 8, k 3)")


CASES = [
    # b, d, L, k, layout, dtypes (x, w, bias), bias, act, nseq
    (2, 64, 300, 4, "cl", ("bf16", "bf16", "bf16"), True, "silu", 0),
    (2, 64, 300, 4, "cl", ("bf16", "f32", "f32"), True, "silu", 3),
    (1, 40, 129, 4, "cl", ("f32", "f32", "f32"), True, None, 0),
    (3, 24, 77, 3, "cf", ("f32", "f32", "f32"), True, "silu", 4),
    (2, 16, 64, 4, "cf", ("bf16", "bf16", "bf16"), False, "silu", 2),
    (1, 9, 37, 2, "cf", ("bf16", "bf16", "f32"), True, None, 0),
    (2, 12, 50, 4, "cl", ("bf16", "bf16", "bf16"), True, "silu", 3),   # 12 % 8: one channel per lane
    (2, 32, 45, 4, "strided", ("f32", "f32", "f32"), True, "silu", 3),
    (1, 16, 2, 4, "cl", ("bf16", "bf16", "bf16"), True, "silu", 0),    # L < width
    (1, 16, 3, 4, "cf", ("f32", "f32", "f32"), True, None, 2),
    (1, 8, 200, 1, "cl", ("bf16", "bf16", "bf16"), True, "silu", 5),
    (2, 24, 100, 5, "cf", ("f32", "f32", "f32"), True, "silu", 3),
    (1, 64, 150, 6, "cl", ("f32", "f32", "f32"), False, None, 4),
    (1, 16, 90, 7, "strided", ("bf16", "bf16", "bf16"), True, "silu", 2),
    (2, 32, 140, 8, "cl", ("bf16", "bf16", "bf16"), True, "silu", 6),
    (2, 8, 40, 8, "cf", ("bf16", "f32", "f32"), True, "silu", 3),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[4]}-k{c[3]}-{'/'.join(c[5])}-L{c[2]}-d{c[1]}"
                                              f"-seq{c[8]}" for c in CASES])
def test_conv_paths(case):
    b, d, L, k, layout, dts, with_bias, act, nseq = case
    announce("causal_conv1d", case)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    T = {"bf16": torch.bfloat16, "f32": torch.float32}
    xdt, wdt, bdt = (T[t] for t in dts)
    x, w, bias = _inputs(rng, b, d, L, k, xdt, wdt, bdt, with_bias)
    seq = _seq(rng, b, L, nseq) if nseq else None
    want, rdt = X.causal_conv1d(x, w, bias, act, seq, NAME[xdt], NAME[wdt], NAME[bdt])
    xt = _layout(dev(x, xdt), layout)
    got = causal_conv1d(xt, dev(w, wdt), dev(bias, bdt), act,
                        None if seq is None else dev(seq))
    assert NAME[got.dtype] == rdt
    if layout == "cl" and d > 1:   # (one channel: both layouts are the same memory order)
        assert got.stride(1) == 1, "the result keeps the channels-last layout"
    _close(got, want, rdt == "bfloat16", f"{layout} k={k}", _mag(x, w, bias))


def test_conv_weight_3d_and_unaligned():
    rng = np.random.default_rng(3)
    x, w, bias = _inputs(rng, 1, 16, 33, 4, None, None, None)
    want, _ = X.causal_conv1d(x, w, bias, "silu")
    _close(causal_conv1d(dev(x), dev(w)[:, None, :], dev(bias), "silu"), want, False, "(d,1,k) weight")
    # x starting at an odd element offset (not 16-byte aligned)
    big = torch.zeros(1 + 16 * 33, dtype=torch.float32, device="cuda")
    big[1:] = dev(x).flatten()
    xo = big[1:].view(1, 16, 33)
    _close(causal_conv1d(xo, dev(w), dev(bias), "silu"), want, False, "unaligned x")


def test_conv_split_layer_shape():
    """The nemotron-h-8b layer: xBC (1, 4096, 8192 + 2 * 1024) bf16, width 4,
    silu, written straight into x (1, 4096, 128, 64), B and C (1, 4096, 8, 128)."""
    announce("causal_conv1d split, nemotron-h-8b layer shape")
    rng = np.random.default_rng(8)
    Lq, dssm, gn = 4096, 8192, 1024
    D = dssm + 2 * gn
    xbc = bf16_round(rng.standard_normal((1, Lq, D)).astype(np.float32))
    w = bf16_round((rng.standard_normal((D, 4)) / 2).astype(np.float32))
    bias = bf16_round(rng.standard_normal(D).astype(np.float32))
    xt = dev(xbc, torch.bfloat16)
    parts = causal_conv1d(xt.transpose(1, 2), dev(w, torch.bfloat16), dev(bias, torch.bfloat16),
                          "silu", split_sizes=(dssm, gn, gn))
    xs, Bs, Cs = (p.transpose(1, 2) for p in parts)
    assert xs.is_contiguous() and Bs.is_contiguous() and Cs.is_contiguous()
    assert xs.view(1, Lq, 128, 64).shape == (1, Lq, 128, 64)
    want, rdt = X.causal_conv1d(xbc.transpose(0, 2, 1), w, bias, "silu", None,
                                "bfloat16", "bfloat16", "bfloat16")
    assert rdt == "bfloat16"
    want = want.transpose(0, 2, 1)
    mag = _mag(xbc.transpose(0, 2, 1), w, bias).transpose(0, 2, 1)
    _close(xs, want[:, :, :dssm], True, "x part", mag[:, :, :dssm])
    _close(Bs, want[:, :, dssm:dssm + gn], True, "B part", mag[:, :, dssm:dssm + gn])
    _close(Cs, want[:, :, dssm + gn:], True, "C part", mag[:, :, dssm + gn:])
    # the same result unsplit
    whole = causal_conv1d(xt.transpose(1, 2), dev(w, torch.bfloat16), dev(bias, torch.bfloat16), "silu")
    assert torch.equal(whole.transpose(1, 2)[:, :, :dssm], xs)


@pytest.mark.parametrize("dts,k", [(("f32", "f32", "f32", "f32"), 4), (("bf16", "bf16", "bf16", "bf16"), 4),
                                   (("bf16", "f32", "bf16", "f32"), 3), (("f32", "bf16", "f32", "bf16"), 2),
                                   (("bf16", "bf16", "f32", "f32"), 8)])
def test_update_matches_prefill(dts, k):
    """reference tests/test_mamba2_ops.py:169-202 (in place, with dtypes)."""
    T = {"bf16": torch.bfloat16, "f32": torch.float32}
    sdt, xdt, wdt, bdt = (T[t] for t in dts)
    announce("causal_conv1d_update", dts, k)
    rng = np.random.default_rng(99)
    b, d, L = 2, 24, 10
    x, w, bias = _inputs(rng, b, d, L, k, xdt, wdt, bdt)
    state = torch.zeros((b, d, k), dtype=sdt, device="cuda")
    st_np = np.zeros((b, d, k))
    names = (NAME[xdt], NAME[sdt], NAME[wdt], NAME[bdt])
    for t in range(L):
        new_state, out = causal_conv1d_update(dev(x[:, :, t], xdt), state, dev(w, wdt),
                                              dev(bias, bdt), "silu", inplace=True)
        st_np, want, nsdt, odt = X.causal_conv1d_update(x[:, :, t], st_np, w, bias, "silu", *names)
        assert NAME[new_state.dtype] == nsdt and NAME[out.dtype] == odt
        if new_state.dtype == state.dtype:
            assert new_state.data_ptr() == state.data_ptr(), "in-place update"
        assert np.array_equal(host(new_state), st_np)
        ob = host(out)
        mag = np.sum(np.abs(st_np * w[None]), axis=-1) + np.abs(bias)[None, :]
        tol = 2.0 ** -7 * (np.abs(want) + mag) if odt == "bfloat16" else 1e-5 * mag
        assert np.all(np.abs(ob - want) <= tol), f"step {t}"
        state = new_state
    if sdt == torch.float32 and xdt == torch.float32:
        full, _ = X.causal_conv1d(x, w, bias, "silu", None, "float32", NAME[wdt], NAME[bdt])
        _close(out, full[:, :, -1], False, "last step == prefill")


def test_update_copy_and_split():
    rng = np.random.default_rng(5)
    b, d, k = 4, 48, 4
    x, w, bias = _inputs(rng, b, d, 1, k, None, None, None)
    st = rng.standard_normal((b, d, k)).astype(np.float32)
    s0 = dev(st)
    keep = s0.clone()
    ns, parts = causal_conv1d_update(dev(x[:, :, 0]), s0, dev(w), dev(bias), "silu",
                                     inplace=False, split_sizes=(32, 8, 8))
    assert torch.equal(s0, keep), "inplace=False leaves the state alone"
    want_s, want, _, _ = X.causal_conv1d_update(x[:, :, 0], st, w, bias, "silu")
    assert np.array_equal(host(ns), want_s)
    got = torch.cat(parts, dim=1)
    _close(got, want, False, "split update")
    # x_new as a strided view (a slice of a wider row)
    wide = torch.zeros((b, 2 * d), device="cuda")
    wide[:, d:] = dev(x[:, :, 0])
    s1 = dev(st)
    ns2, out2 = causal_conv1d_update(wide[:, d:], s1, dev(w), dev(bias), "silu")
    _close(out2, want, False, "strided x_new")
    # the default is functional, as the reference (ops/causal_conv1d.py:88-139)
    assert ns2.data_ptr() != s1.data_ptr() and np.array_equal(host(s1), st)
    assert np.array_equal(host(ns2), want_s)


def test_capi_token_vectors_with_ragged_tail():
    """m2_causal_conv1d called directly: x and out are (b, d, L) views of
    (b, d, 48) buffers, so the token-vector path runs with a partial last
    vector (L = 45), and a NULL bias."""
    from mamba2_jax import _lib as L
    rng = np.random.default_rng(11)
    b, d, Lq, Lp, k = 2, 16, 45, 48, 4
    x, w, _ = _inputs(rng, b, d, Lq, k, torch.bfloat16, torch.bfloat16, None, with_bias=False)
    xb = torch.zeros((b, d, Lp), dtype=torch.bfloat16, device="cuda")
    xb[:, :, :Lq] = dev(x, torch.bfloat16)
    ob = torch.full((b, d, Lp), 7.0, dtype=torch.bfloat16, device="cuda")
    wt = dev(w, torch.bfloat16)
    outs = (L.ConvOut * 3)()
    outs[0] = L.ConvOut(L.ptr(ob), 0, d * Lp, Lp, 1)
    args = L.CausalConv1dArgs(x=L.ptr(xb), x_stride_batch=d * Lp, x_stride_dim=Lp, x_stride_time=1,
                              weight=L.ptr(wt), bias=0, seq_idx=0, out=outs, batch=b, dim=d,
                              seqlen=Lq, width=k, nout=1, x_dtype=L.M2_BF16, w_dtype=L.M2_BF16,
                              bias_dtype=L.M2_F32, out_dtype=L.M2_BF16, silu=1)
    L.call("m2_causal_conv1d", args, L.stream_of(torch.device("cuda")))
    torch.cuda.synchronize()
    want, _ = X.causal_conv1d(x, w, None, "silu", None, "bfloat16", "bfloat16")
    _close(ob[:, :, :Lq], want, True, "token vectors, ragged tail", _mag(x, w, None))
    assert bool((ob[:, :, Lq:] == 7.0).all()), "nothing written past seqlen"
    # a wrong out_dtype is rejected
    args.out_dtype = L.M2_F32
    with pytest.raises(L.M2Error):
        L.call("m2_causal_conv1d", args, L.stream_of(torch.device("cuda")))


def test_errors():
    x = torch.zeros((1, 4, 8), device="cuda")
    with pytest.raises(AssertionError):
        causal_conv1d(x, torch.zeros((4, 9), device="cuda"))      # width 9
    with pytest.raises(AssertionError):
        causal_conv1d(x, torch.zeros((5, 3), device="cuda"))      # d mismatch
    with pytest.raises(ValueError):
        causal_conv1d(x.cpu(), torch.zeros((4, 3)))               # no CPU path


def _sweep_cases(n=24, seed=91):
    """Cases of test_conv_paths' form drawn once from a fixed seed: 1-3 rows,
    1-96 channels, 1-400 tokens, widths 1-8, every layout, mixed dtypes, bias,
    silu and sequence resets on and off."""
    rng = np.random.default_rng(seed)
    tys = ("bf16", "f32")
    out = []
    for _ in range(n):
        L = int(rng.integers(1, 401))
        out.append((int(rng.integers(1, 4)), int(rng.integers(1, 97)), L, int(rng.integers(1, 9)),
                    str(rng.choice(["cl", "cf", "strided"])),
                    tuple(str(rng.choice(tys)) for _ in range(3)), bool(rng.random() < 0.7),
                    "silu" if rng.random() < 0.6 else None,
                    min(int(rng.integers(0, 6)), L)))
    return out


@pytest.mark.parametrize("case", _sweep_cases())
def test_conv_sweep(case):
    test_conv_paths(case)

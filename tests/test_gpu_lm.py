"""The Mamba2 LM (mamba2_jax.models) on the GPU: logits against the CPU
oracle's composition, prefill + decode against the full forward, HIP-graph
replays of the decode step against the eager step (every replay checked, with
eager work and synchronisations between replays), and generation with and
without the graph (reference models/mamba2_lm.py:178-302, 667-736)."""

import numpy as np
import pytest
import torch

from gpu_util import TOL, announce, check, host
from mamba2_jax.models import Mamba2Config, Mamba2LMHeadModel, init_params
from mamba2_jax.models.mamba2_lm import DecodeState
from oracle import ops_oracle as X

pytestmark = pytest.mark.gpu

CFG = Mamba2Config(d_model=128, n_layer=3, vocab_size=300, d_state=64, headdim=64, ngroups=1,
                   chunk_size=64)


def _np_params(p):
    f = lambda t: None if t is None else host(t)
    return {"embedding": {"weight": f(p["embedding"]["weight"])},
            "layers": [{"norm_weight": f(lp["norm_weight"]),
                        "mixer": {k: f(v) for k, v in lp["mixer"].items()}} for lp in p["layers"]],
            "norm_f_weight": f(p["norm_f_weight"]), "lm_head_weight": f(p["lm_head_weight"])}


def _mcfg(cfg):
    d = cfg.mixer_dims()
    return dict(d_ssm=d.d_ssm, d_mlp=0, ngroups=d.ngroups, d_state=d.d_state, headdim=d.headdim,
                nheads=d.nheads, chunk_size=d.chunk_size, rmsnorm=d.rmsnorm,
                norm_before_gate=d.norm_before_gate, D_has_hdim=d.D_has_hdim, dt_limit=d.dt_limit)


def _cast(p, dtype):
    f = lambda t: None if t is None else (t.to(dtype) if t.dtype == torch.bfloat16 else t)
    return {"embedding": {"weight": f(p["embedding"]["weight"])},
            "layers": [{"norm_weight": f(lp["norm_weight"]),
                        "mixer": {k: f(v) for k, v in lp["mixer"].items()}} for lp in p["layers"]],
            "norm_f_weight": f(p["norm_f_weight"]), "lm_head_weight": f(p["lm_head_weight"])}


def _ids(rng, b, L):
    return torch.from_numpy(rng.integers(0, CFG.vocab_size, (b, L))).cuda()


def test_lm_logits_fp32():
    announce("LM logits fp32")
    params = init_params(CFG, dtype=torch.float32, seed=1)
    ids = _ids(np.random.default_rng(2), 2, 90)
    got = Mamba2LMHeadModel(CFG)(params, ids)
    want = X.mamba2_lm(_np_params(params), host(ids).astype(np.int64), _mcfg(CFG))
    check(got, want, TOL["f32"], "logits")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_lm_prefill_then_decode(dtype):
    announce("LM prefill + decode", dtype)
    pd = torch.bfloat16 if dtype == "bf16" else torch.float32
    params = init_params(CFG, dtype=pd, seed=3)
    m = Mamba2LMHeadModel(CFG)
    ids = _ids(np.random.default_rng(4), 2, 80)
    full = m(params, ids)
    T0 = 70
    st = DecodeState(CFG, 2)
    last = m.prefill(params, ids[:, :T0], st)
    check(last, host(full[:, T0 - 1]), 1e-5 if dtype == "f32" else 2e-2, "prefill logits")
    outs = [m.decode_step(params, ids[:, t], st) for t in range(T0, 80)]
    dec = torch.stack(outs[:-1], 1)
    if dtype == "f32":
        check(dec, host(full[:, T0:79]), TOL["f32"], "decode logits")
        return
    # bf16: prefill and decode round at different points (the chunked SSD's
    # bf16 passed states and conv outputs vs the decode's f32 conv / SSM
    # state), and the differences compound over the layers; both are held to
    # the same float32 run of these (bf16-valued) parameters (the prefill
    # measured ~5e-2 from it: bf16 projections, conv and SSD over 3 layers),
    # the decode no further from it than twice the prefill
    p32 = _cast(params, torch.float32)
    truth = host(m(p32, ids)[:, T0:79])
    e_pre = check(full[:, T0:79], truth, 1e-1, "bf16 prefill vs f32")
    check(dec, truth, max(2 * e_pre, TOL["bf16"]), "bf16 decode vs f32")


@pytest.mark.parametrize("batch", [1, 2, 3])
def test_decode_graph_replays_match_eager(batch):
    """Every replay of the captured step equals the eager step from the same
    state, bit for bit (logits and both states); eager work and syncs run
    between the replays.  Batches 1 and 2 with bf16 parameters run the fused
    decode layer (norms inside the projections, the conv update in the
    in-projection's epilogue), the path of the LM decode figures; batch 3 the
    separate kernels."""
    announce("LM decode graph replays", batch)
    params = init_params(CFG, dtype=torch.bfloat16, seed=5)
    m = Mamba2LMHeadModel(CFG)
    assert m._fusable(params, batch) == (batch <= 2)
    ids = _ids(np.random.default_rng(6), batch, 40)
    st_e, st_g = DecodeState(CFG, batch), DecodeState(CFG, batch)
    m.prefill(params, ids[:, :30], st_e)
    m.prefill(params, ids[:, :30], st_g)
    g, tok, out = m.capture_decode(params, st_g)
    assert torch.equal(st_e.ssm, st_g.ssm) and torch.equal(st_e.conv, st_g.conv)
    for t in range(30, 40):
        want = m.decode_step(params, ids[:, t], st_e)
        torch.cuda.synchronize()
        tok.copy_(ids[:, t])
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay at token {t}"
        assert torch.equal(st_g.ssm, st_e.ssm) and torch.equal(st_g.conv, st_e.conv)
        _ = (torch.randn(1000, device="cuda") * 2).sum().item()   # eager work in between


def test_generate_graph_equals_eager():
    announce("LM generate, graph vs eager")
    params = init_params(CFG, dtype=torch.float32, seed=7)
    m = Mamba2LMHeadModel(CFG)
    ids = _ids(np.random.default_rng(8), 2, 24)
    a = m.generate(params, ids, max_new_tokens=12, temperature=0, use_graph=True)
    b = m.generate(params, ids, max_new_tokens=12, temperature=0, use_graph=False)
    assert a.shape == (2, 36) and torch.equal(a[:, :24], ids)
    assert torch.equal(a, b)
    c = m.generate(params, ids, max_new_tokens=8, temperature=1.0, top_k=20, rng_key=3)
    d = m.generate(params, ids, max_new_tokens=8, temperature=1.0, top_k=20, rng_key=3, use_graph=False)
    assert torch.equal(c, d)


@pytest.mark.parametrize("batch", [1, 2])
def test_fused_decode_matches_unfused(batch):
    """The decode step with the norms inside the projections
    (mamba2_block_step_fused, batch <= 4) against the separate norm kernels:
    the two differ only where a norm's sum of squares rounds differently
    (another summation order), so logits and states stay within the bf16
    bar over ten steps."""
    announce("LM fused decode vs unfused", batch)
    params = init_params(CFG, dtype=torch.bfloat16, seed=9)
    fused, plain = Mamba2LMHeadModel(CFG), Mamba2LMHeadModel(CFG)
    plain.fuse_decode = False
    assert fused._fusable(params, batch) and not plain._fusable(params, batch)
    ids = _ids(np.random.default_rng(10), batch, 40)
    st_f, st_p = DecodeState(CFG, batch), DecodeState(CFG, batch)
    fused.prefill(params, ids[:, :30], st_f)
    plain.prefill(params, ids[:, :30], st_p)
    for t in range(30, 40):
        lf = fused.decode_step(params, ids[:, t], st_f)
        lp = plain.decode_step(params, ids[:, t], st_p)
        check(lf, host(lp), TOL["bf16"], f"logits, token {t}")
    check(st_f.ssm, host(st_p.ssm), TOL["bf16"], "ssm states")
    check(st_f.conv, host(st_p.conv), TOL["bf16"], "conv states")


@pytest.mark.parametrize("batch", [1, 3])
def test_logits_are_float32_with_bf16_params(batch):
    """The reference's head multiplies float32 activations by the head weight,
    which promotes to float32 logits (models/mamba2_lm.py:213-216, 732-736):
    prefill and decode (fused and unfused batches) return float32."""
    announce("LM logits dtype", batch)
    params = init_params(CFG, dtype=torch.bfloat16, seed=11)
    m = Mamba2LMHeadModel(CFG)
    ids = _ids(np.random.default_rng(12), batch, 20)
    st = DecodeState(CFG, batch)
    assert m(params, ids).dtype == torch.float32
    assert m.prefill(params, ids[:, :19], st).dtype == torch.float32
    assert m.decode_step(params, ids[:, 19], st).dtype == torch.float32


def test_decode_residual_is_float32_without_residual_in_fp32():
    """residual_in_fp32=False: the reference's decode step still keeps its
    residual in float32 (_scan_decode_step, models/mamba2_lm.py:680), so the
    decode equals the float32-residual decode of the same parameters exactly,
    and stays within the bf16 bar of the bf16-residual prefill."""
    announce("LM decode residual f32")
    import dataclasses
    cfg16 = dataclasses.replace(CFG, residual_in_fp32=False)
    params = init_params(CFG, dtype=torch.bfloat16, seed=13)
    m16, m32 = Mamba2LMHeadModel(cfg16), Mamba2LMHeadModel(CFG)
    m16.fuse_decode = m32.fuse_decode = False
    ids = _ids(np.random.default_rng(14), 3, 24)
    s16, s32 = DecodeState(cfg16, 3), DecodeState(CFG, 3)
    m32.prefill(params, ids[:, :20], s32)
    s16.conv.copy_(s32.conv)
    s16.ssm.copy_(s32.ssm)
    for t in range(20, 24):
        a = m16.decode_step(params, ids[:, t], s16)
        b = m32.decode_step(params, ids[:, t], s32)
        assert torch.equal(a, b), f"token {t}"


def test_prepared_copies_follow_in_place_weight_updates():
    """The decode step's derived copies (A, [out, in] projections, the float32
    head) are rebuilt when a source weight is updated in place."""
    announce("LM prepared-cache invalidation")
    params = init_params(CFG, dtype=torch.bfloat16, seed=15)
    m = Mamba2LMHeadModel(CFG)
    ids = _ids(np.random.default_rng(16), 1, 12)
    st = DecodeState(CFG, 1)
    m.prefill(params, ids[:, :11], st)
    saved = (st.conv.clone(), st.ssm.clone())
    before = m.decode_step(params, ids[:, 11], st)
    with torch.no_grad():
        params["layers"][0]["mixer"]["out_proj_kernel"].mul_(2.0)
    fresh = Mamba2LMHeadModel(CFG)
    st.conv.copy_(saved[0])
    st.ssm.copy_(saved[1])
    after = m.decode_step(params, ids[:, 11], st)
    st.conv.copy_(saved[0])
    st.ssm.copy_(saved[1])
    want = fresh.decode_step(params, ids[:, 11], st)
    assert not torch.equal(before, after)
    assert torch.equal(after, want)

"""Checkpoint formats of the Mamba2 LM (reference models/mamba2_lm.py:84-113,
530-635): config.json of the HF state-spaces format and its weights as
pytorch_model.bin, one safetensors file or a directory of safetensors shards.

No real checkpoint is available offline, so the checkpoints here are written
by the tests in the HF key layout (torch Linear weights (out, in), conv1d
weights (channels, 1, width)) from known tensors; the loaded parameters must
have the shapes of ``init_params`` (the layout the model runs on) and the
source values in that layout.  The GPU test runs a model on a saved-and-loaded
copy of random parameters and requires bit-identical logits.
"""

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from mamba2_jax.models import (MAMBA2_CONFIGS, Mamba2Config, Mamba2LMHeadModel, init_params,
                               load_from_pretrained, load_from_torch_checkpoint)

CFG = Mamba2Config(d_model=64, n_layer=2, vocab_size=100, d_state=32, headdim=16, ngroups=2,
                   chunk_size=32)

# config.json of state-spaces/mamba2-130m (public HF model card data)
CFG_130M = {"d_model": 768, "d_intermediate": 0, "n_layer": 24, "vocab_size": 50277,
            "ssm_cfg": {"layer": "Mamba2"}, "attn_layer_idx": [], "attn_cfg": {},
            "rms_norm": True, "residual_in_fp32": True, "fused_add_norm": True,
            "pad_vocab_size_multiple": 16, "tie_embeddings": True}


def hf_state_dict(params, cfg, lm_head=None):
    """Parameters (reference dict layout) -> HF state-spaces keys and layouts."""
    sd = {"backbone.embedding.weight": params["embedding"]["weight"],
          "backbone.norm_f.weight": params["norm_f_weight"]}
    for i, lp in enumerate(params["layers"]):
        m, pre = lp["mixer"], f"backbone.layers.{i}."
        sd[pre + "norm.weight"] = lp["norm_weight"]
        sd[pre + "mixer.in_proj.weight"] = m["in_proj_kernel"].t()
        sd[pre + "mixer.conv1d.weight"] = m["conv1d_weight"][:, None, :]
        sd[pre + "mixer.conv1d.bias"] = m["conv1d_bias"]
        for k in ("dt_bias", "A_log", "D"):
            sd[pre + "mixer." + k] = m[k]
        sd[pre + "mixer.norm.weight"] = m["norm_weight"]
        sd[pre + "mixer.out_proj.weight"] = m["out_proj_kernel"].t()
    if lm_head is not None:
        sd["lm_head.weight"] = lm_head
    return {k: v.detach().cpu().contiguous() for k, v in sd.items()}


def _flat(params):
    out = {"embedding": params["embedding"]["weight"], "norm_f": params["norm_f_weight"],
           "lm_head": params["lm_head_weight"]}
    for i, lp in enumerate(params["layers"]):
        out[f"{i}.norm"] = lp["norm_weight"]
        for k, v in lp["mixer"].items():
            out[f"{i}.{k}"] = v
    return out


def _assert_same_layout_and_values(got, want, dtype):
    g, w = _flat(got), _flat(want)
    assert g.keys() == w.keys()
    for k in w:
        assert tuple(g[k].shape) == tuple(w[k].shape), k
        want_dt = torch.float32 if k.endswith("dt_bias") else dtype
        assert g[k].dtype == want_dt, (k, g[k].dtype)
        assert torch.equal(g[k].cpu(), w[k].cpu().to(want_dt)), k


def test_config_from_hf_json(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps(CFG_130M))
    c = Mamba2Config.from_pretrained(str(tmp_path))
    assert c == MAMBA2_CONFIGS["mamba2-130m"]
    assert (c.d_inner, c.nheads, c.d_in_proj, c.vocab_size_padded) == (1536, 24, 3352, 50288)
    ssm = {"d_state": 64, "d_conv": 3, "expand": 1, "headdim": 32, "ngroups": 4, "chunk_size": 128}
    (tmp_path / "config.json").write_text(json.dumps(dict(CFG_130M, ssm_cfg=ssm, rms_norm=False,
                                                          tie_embeddings=False)))
    c = Mamba2Config.from_pretrained(str(tmp_path / "config.json"))
    assert (c.d_state, c.d_conv, c.expand, c.headdim, c.ngroups, c.chunk_size) == \
        (64, 3, 1, 32, 4, 128)
    assert not c.rmsnorm and not c.tie_embeddings


@pytest.mark.parametrize("fmt", ["bin", "safetensors", "shards"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_load_formats(tmp_path, fmt, dtype):
    src = init_params(CFG, dtype=torch.float32, device="cpu", seed=3)
    sd = hf_state_dict(src, CFG)
    if fmt == "bin":
        path = tmp_path / "pytorch_model.bin"
        torch.save(sd, path)
    elif fmt == "safetensors":
        path = tmp_path / "model.safetensors"
        # the tied embedding appears once in the file
        save_file(sd, str(path))
    else:
        path = tmp_path
        keys = sorted(sd)
        save_file({k: sd[k] for k in keys[::2]}, str(tmp_path / "model-00001-of-00002.safetensors"))
        save_file({k: sd[k] for k in keys[1::2]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    got = load_from_torch_checkpoint(CFG, str(path), dtype=dtype, device="cpu")
    _assert_same_layout_and_values(got, src, dtype)
    assert got["lm_head_weight"] is got["embedding"]["weight"]     # tied


def test_untied_head_and_errors(tmp_path):
    cfg = Mamba2Config(**{**CFG.__dict__, "tie_embeddings": False})
    src = init_params(cfg, dtype=torch.float32, device="cpu", seed=4)
    head = torch.randn_like(src["embedding"]["weight"])
    got = load_from_torch_checkpoint(cfg, hf_state_dict(src, cfg, lm_head=head), device="cpu")
    assert torch.equal(got["lm_head_weight"], head)
    assert not torch.equal(got["lm_head_weight"], got["embedding"]["weight"])
    with pytest.raises(FileNotFoundError):
        load_from_torch_checkpoint(cfg, str(tmp_path), device="cpu")      # empty directory
    with pytest.raises(FileNotFoundError):
        load_from_pretrained("state-spaces/mamba2-130m")                    # no downloads
    with pytest.raises(KeyError):
        sd = hf_state_dict(src, cfg, lm_head=head)
        del sd["backbone.layers.1.mixer.out_proj.weight"]
        load_from_torch_checkpoint(cfg, sd, device="cpu")


@pytest.mark.gpu
def test_saved_and_loaded_model_same_logits(tmp_path):
    """A model directory written from random parameters (config.json +
    safetensors) loads into parameters whose logits equal the originals'."""
    cfg = Mamba2Config(d_model=128, n_layer=2, vocab_size=300, d_state=64, headdim=64,
                       chunk_size=64)
    src = init_params(cfg, dtype=torch.float32, seed=5)
    (tmp_path / "config.json").write_text(json.dumps(
        {"d_model": 128, "n_layer": 2, "vocab_size": 300, "pad_vocab_size_multiple": 16,
         "ssm_cfg": {"d_state": 64, "headdim": 64, "chunk_size": 64}, "rms_norm": True,
         "residual_in_fp32": True, "tie_embeddings": True}))
    save_file(hf_state_dict(src, cfg), str(tmp_path / "model.safetensors"))
    model, params, cfg2 = load_from_pretrained(str(tmp_path))
    assert cfg2 == cfg
    ids = torch.from_numpy(np.random.default_rng(6).integers(0, 300, (2, 70))).cuda()
    want = Mamba2LMHeadModel(cfg)(src, ids)
    got = model(params, ids)
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_bf16_checkpoint_generates(tmp_path):
    """Loaded with dtype=bfloat16 (A_log and D in bf16 too, as the reference
    loads them): generation through the decode graph equals eager decoding."""
    cfg = Mamba2Config(d_model=128, n_layer=3, vocab_size=300, d_state=64, headdim=64,
                       chunk_size=64)
    src = init_params(cfg, dtype=torch.float32, seed=7)
    save_file(hf_state_dict(src, cfg), str(tmp_path / "model.safetensors"))
    params = load_from_torch_checkpoint(cfg, str(tmp_path), dtype=torch.bfloat16)
    assert params["layers"][0]["mixer"]["A_log"].dtype == torch.bfloat16
    model = Mamba2LMHeadModel(cfg)
    ids = torch.from_numpy(np.random.default_rng(8).integers(0, 300, (3, 20))).cuda()
    a = model.generate(params, ids, max_new_tokens=8, temperature=0, use_graph=True)
    b = model.generate(params, ids, max_new_tokens=8, temperature=0, use_graph=False)
    assert torch.equal(a, b)

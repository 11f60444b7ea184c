"""The Mamba2 language model on MI355X: prefill, and the token-by-token decode
loop that consumes the in-place decode kernels (reference
models/mamba2_lm.py:36-736).

Same config fields, parameter dict structure, call signatures and returns as
the reference (``__call__(params, input_ids) -> logits``, ``generate``).
Parameters are torch tensors on the GPU: ``init_params`` makes random ones of
the architecture, ``load_from_torch_checkpoint`` / ``load_from_pretrained``
read the HF state-spaces checkpoint format (``pytorch_model.bin`` or
safetensors, from local files: there is no download).

Decode, MI355X-first: every layer's conv and SSM state lives in one
(n_layer, ...) tensor that the decode kernels update in place, so a step
allocates no state; the whole step (embedding gather, n_layer x [RMSNorm,
in-projection, conv update, selective state update, gated norm,
out-projection, residual], final norm, LM head) is captured once into a HIP
graph and replayed per token (``generate(..., use_graph=True)``), which
removes the per-kernel launch cost that dominates a small-batch step.  The
reference gets the equivalent from jax.jit + lax.scan over layers
(:667-736).
"""

from __future__ import annotations

import glob
import json
import math
import os
from dataclasses import dataclass

import torch

from ..modules.mamba2 import (MixerDims, _lecun_normal, block_step_fusable, mamba2_block_forward,
                              mamba2_block_step, mamba2_block_step_fused)
from ..ops import linear
from ..ops.rms_norm import rms_norm_gated


@dataclass
class Mamba2Config:
    """Configuration of a Mamba2 language model (reference :36-83)."""
    d_model: int = 2048
    n_layer: int = 48
    vocab_size: int = 50277
    pad_vocab_size_multiple: int = 16
    d_state: int = 128
    d_conv: int = 4
    expand: int = 2
    headdim: int = 64
    ngroups: int = 1
    chunk_size: int = 256
    rmsnorm: bool = True
    norm_before_gate: bool = False
    bias: bool = False
    conv_bias: bool = True
    D_has_hdim: bool = False
    tie_embeddings: bool = True
    residual_in_fp32: bool = True
    dt_limit: tuple = (0.0, float("inf"))

    @property
    def vocab_size_padded(self):
        return math.ceil(self.vocab_size / self.pad_vocab_size_multiple) * self.pad_vocab_size_multiple

    @property
    def d_inner(self):
        return self.expand * self.d_model

    @property
    def nheads(self):
        return self.d_inner // self.headdim

    @property
    def conv_dim(self):
        return self.d_inner + 2 * self.ngroups * self.d_state

    @property
    def d_in_proj(self):
        return 2 * self.d_inner + 2 * self.ngroups * self.d_state + self.nheads

    @classmethod
    def from_pretrained(cls, model_name_or_path: str) -> "Mamba2Config":
        """The config of a local model directory (or its config.json) in the
        HF state-spaces format (reference :84-113, same key map and defaults).
        Hub ids are not fetched: there is no network."""
        path = model_name_or_path
        if os.path.isdir(path):
            path = os.path.join(path, "config.json")
        if not os.path.isfile(path):
            raise FileNotFoundError(f"{model_name_or_path!r}: no local config.json (hub downloads "
                                    "are not supported; pass a local model directory)")
        with open(path) as f:
            data = json.load(f)
        ssm = data.get("ssm_cfg", {})
        return cls(d_model=data.get("d_model", 2048), n_layer=data.get("n_layer", 48),
                   vocab_size=data.get("vocab_size", 50277),
                   pad_vocab_size_multiple=data.get("pad_vocab_size_multiple", 16),
                   d_state=ssm.get("d_state", 128), d_conv=ssm.get("d_conv", 4),
                   expand=ssm.get("expand", 2), headdim=ssm.get("headdim", 64),
                   ngroups=ssm.get("ngroups", 1), chunk_size=ssm.get("chunk_size", 256),
                   rmsnorm=data.get("rms_norm", True),
                   residual_in_fp32=data.get("residual_in_fp32", True),
                   tie_embeddings=data.get("tie_embeddings", True))

    def mixer_dims(self):
        return MixerDims(d_ssm=self.d_inner, d_mlp=0, ngroups=self.ngroups, d_state=self.d_state,
                         headdim=self.headdim, nheads=self.nheads, d_conv=self.d_conv,
                         chunk_size=self.chunk_size, rmsnorm=self.rmsnorm,
                         norm_before_gate=self.norm_before_gate, D_has_hdim=self.D_has_hdim,
                         dt_limit=tuple(self.dt_limit))


# the reference's predefined sizes (:119-125)
MAMBA2_CONFIGS = {
    "mamba2-130m": Mamba2Config(d_model=768, n_layer=24),
    "mamba2-370m": Mamba2Config(d_model=1024, n_layer=48),
    "mamba2-780m": Mamba2Config(d_model=1536, n_layer=48),
    "mamba2-1.3b": Mamba2Config(d_model=2048, n_layer=48),
    "mamba2-2.7b": Mamba2Config(d_model=2560, n_layer=64),
}


def rms_norm(x, weight, eps=1e-5, *, out_dtype=None, residual=None):
    """Plain RMSNorm over the last dimension (reference :136-139), as the HIP
    rms_norm_gated kernel without a gate; out_dtype=torch.bfloat16 stores the
    float32 result in bf16 for a bf16 projection; residual (float32, updated
    in place to residual + x) fuses a pre-norm block's residual add."""
    return rms_norm_gated(x, weight, z=None, eps=eps, out_dtype=out_dtype, residual=residual)


def init_params(cfg: Mamba2Config, dtype=torch.bfloat16, device=None, seed=0):
    """Random parameters of the architecture in the reference's dict layout
    (class docstring of Mamba2LMHeadModel, reference :142-174)."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    g = torch.Generator().manual_seed(seed)
    emb = (torch.randn((cfg.vocab_size_padded, cfg.d_model), generator=g) * 0.02).to(dev, dtype)
    layers = []
    for _ in range(cfg.n_layer):
        u = torch.rand(cfg.nheads, generator=g, dtype=torch.float64)
        dt = torch.exp(u * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp(min=1e-4)
        mixer = {
            "in_proj_kernel": _lecun_normal((cfg.d_model, cfg.d_in_proj), cfg.d_model, g, dev, dtype),
            "conv1d_weight": _lecun_normal((cfg.conv_dim, cfg.d_conv), cfg.d_conv, g, dev, dtype),
            "conv1d_bias": (torch.randn(cfg.conv_dim, generator=g) * 0.02).to(dev, dtype)
            if cfg.conv_bias else None,
            "dt_bias": (dt + torch.log(-torch.expm1(-dt))).to(dev, torch.float32),
            "A_log": torch.log(torch.rand(cfg.nheads, generator=g) * 15 + 1).to(dev, torch.float32),
            "D": torch.ones(cfg.d_inner if cfg.D_has_hdim else cfg.nheads, device=dev),
            "norm_weight": torch.ones(cfg.d_inner, device=dev, dtype=dtype) if cfg.rmsnorm else None,
            # scaled down so that the residual stream stays O(1) over many layers
            "out_proj_kernel": _lecun_normal((cfg.d_inner, cfg.d_model), cfg.d_inner, g, dev, dtype)
            / math.sqrt(2 * cfg.n_layer),
        }
        if cfg.bias:
            mixer["in_proj_bias"] = torch.zeros(cfg.d_in_proj, device=dev, dtype=dtype)
            mixer["out_proj_bias"] = torch.zeros(cfg.d_model, device=dev, dtype=dtype)
        layers.append({"norm_weight": torch.ones(cfg.d_model, device=dev, dtype=dtype),
                       "mixer": mixer})
    return {"embedding": {"weight": emb}, "layers": layers,
            "norm_f_weight": torch.ones(cfg.d_model, device=dev, dtype=dtype),
            "lm_head_weight": emb}


def read_state_dict(path):
    """A checkpoint's tensors on the CPU: ``path`` is a ``pytorch_model.bin``,
    a ``.safetensors`` file, or a directory holding (possibly sharded)
    ``*.safetensors`` or ``pytorch_model*.bin`` files.  Only loaders that
    execute nothing from the file are used (safetensors,
    ``torch.load(weights_only=True)``)."""
    if os.path.isdir(path):
        files = sorted(glob.glob(os.path.join(path, "*.safetensors"))) or \
            sorted(glob.glob(os.path.join(path, "pytorch_model*.bin")))
        if not files:
            raise FileNotFoundError(f"{path}: no *.safetensors or pytorch_model*.bin files")
    elif os.path.isfile(path):
        files = [path]
    else:
        raise FileNotFoundError(path)
    sd = {}
    for f in files:
        if f.endswith(".safetensors"):
            from safetensors.torch import load_file
            sd.update(load_file(f, device="cpu"))
        else:
            sd.update(torch.load(f, map_location="cpu", weights_only=True))
    return sd


def load_from_torch_checkpoint(config: Mamba2Config, checkpoint_path, dtype=torch.float32,
                               device=None):
    """Parameters in the reference's dict layout from an HF state-spaces
    checkpoint (reference :530-601, same key map): Linear weights (out, in)
    become (in, out) kernels, conv1d (ch, 1, k) becomes (ch, k), dt_bias stays
    float32, everything else takes ``dtype``; the LM head is the embedding
    when the config ties them.  ``checkpoint_path``: see ``read_state_dict``
    (the reference reads ``pytorch_model.bin`` only).  ``device``: default
    cuda.  Linear biases are read when the config has them."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    sd = read_state_dict(checkpoint_path) if isinstance(checkpoint_path, (str, os.PathLike)) \
        else checkpoint_path

    def t(key, dt=dtype, op=None):
        v = sd[key]
        if op is not None:
            v = op(v)
        return v.to(dtype=dt).contiguous().to(dev)

    linear_t = lambda v: v.t()
    params = {"embedding": {"weight": t("backbone.embedding.weight")}, "layers": [],
              "norm_f_weight": t("backbone.norm_f.weight")}
    for i in range(config.n_layer):
        pre = f"backbone.layers.{i}.mixer."
        mixer = {
            "in_proj_kernel": t(pre + "in_proj.weight", op=linear_t),
            "conv1d_weight": t(pre + "conv1d.weight", op=lambda v: v.squeeze(1)),
            "conv1d_bias": t(pre + "conv1d.bias") if pre + "conv1d.bias" in sd else None,
            "dt_bias": t(pre + "dt_bias", torch.float32),
            "A_log": t(pre + "A_log"),
            "D": t(pre + "D"),
            "norm_weight": t(pre + "norm.weight") if pre + "norm.weight" in sd else None,
            "out_proj_kernel": t(pre + "out_proj.weight", op=linear_t),
        }
        if config.bias:
            for name in ("in_proj", "out_proj"):
                if pre + name + ".bias" in sd:
                    mixer[name + "_bias"] = t(pre + name + ".bias")
        params["layers"].append({"norm_weight": t(f"backbone.layers.{i}.norm.weight"),
                                 "mixer": mixer})
    params["lm_head_weight"] = params["embedding"]["weight"] if config.tie_embeddings \
        else t("lm_head.weight")
    return params


def load_from_pretrained(model_name: str, dtype=torch.float32, device=None):
    """(model, params, config) from a local model directory holding config.json
    and the weights (reference :604-635, which downloads them from the hub
    first; there is no network here, so a hub id or short name must be a local
    directory)."""
    if not os.path.isdir(model_name):
        raise FileNotFoundError(f"{model_name!r} is not a local model directory (hub downloads "
                                "are not supported)")
    config = Mamba2Config.from_pretrained(model_name)
    params = load_from_torch_checkpoint(config, model_name, dtype=dtype, device=device)
    return Mamba2LMHeadModel(config), params, config


def _sample_token(logits, generator, temperature=1.0, top_k=50):
    """Greedy when temperature == 0, else top-k sampling (reference :648-664)."""
    if temperature == 0:
        return torch.argmax(logits, dim=-1)
    logits = logits.float() / temperature
    if top_k > 0:
        kth = torch.topk(logits, top_k, dim=-1).values[:, -1:]
        logits = torch.where(logits < kth, torch.full_like(logits, -1e10), logits)
    return torch.multinomial(torch.softmax(logits, -1), 1, generator=generator)[:, 0]


class DecodeState:
    """Per-layer decode states stacked over layers, updated in place:
    conv (n_layer, batch, conv_dim, d_conv) and ssm (n_layer, batch, nheads,
    headdim, d_state), both float32."""

    def __init__(self, cfg: Mamba2Config, batch: int, device=None):
        dev = torch.device("cuda") if device is None else torch.device(device)
        self.conv = torch.zeros((cfg.n_layer, batch, cfg.conv_dim, cfg.d_conv), device=dev)
        self.ssm = torch.zeros((cfg.n_layer, batch, cfg.nheads, cfg.headdim, cfg.d_state), device=dev)


class Mamba2LMHeadModel:
    """Mamba2 LM for inference over a parameter dict (reference :142-351)."""

    def __init__(self, config: Mamba2Config):
        self.config = config
        self._prep = None
        # small decode batches (block_step_fusable) run the norms inside the projections
        # (mamba2_block_step_fused) when the parameters allow it
        self.fuse_decode = True

    @staticmethod
    def _sources(params):
        """The tensors _prepared derives its copies from, with the storage
        address and version counter of each: an in-place update of any of
        them (optimizer step, load_state_dict copy) changes the key."""
        ts = [t for lp in params["layers"]
              for t in (lp["mixer"]["A_log"], lp["mixer"]["in_proj_kernel"],
                        lp["mixer"]["out_proj_kernel"])] + [params["lm_head_weight"]]
        return tuple((t.data_ptr(), t._version) for t in ts)

    def _prepared(self, params, head=False):
        """Per-layer mixer dicts with A = -exp(A_log) precomputed, so that a
        decode step launches no kernels for it, and, for bf16 weights,
        K-contiguous copies of the projections ([out, in]) for the decode
        step's skinny GEMM; with head=True the float32 LM head weight (the
        head's float32 matmul).  Cached per parameter dict and rebuilt when
        any source tensor is replaced or updated in place.  The copies cost
        memory: with bf16 weights the projections are held twice (about 5 GB
        at 2.7b) and the float32 head once more (vocab x d_model x 4 bytes)."""
        key = self._sources(params)
        if self._prep is None or self._prep[0] is not params or self._prep[1] != key:
            mixers = []
            for lp in params["layers"]:
                mx = dict(lp["mixer"])
                mx["A"] = -torch.exp(mx["A_log"].float())
                for name in ("in_proj", "out_proj"):
                    k = mx[name + "_kernel"]
                    if k.dtype == torch.bfloat16 and k.shape[0] % 8 == 0:
                        mx[name + "_t"] = k.t().contiguous()
                mixers.append(mx)
            self._prep = (params, key, mixers, {})
        if head:
            extra = self._prep[3]
            if "head32" not in extra:
                w = params["lm_head_weight"]
                extra["head32"] = w if w.dtype == torch.float32 else w.float()
            return extra["head32"]
        return self._prep[2]

    def _run_layers(self, params, x, block, fp32_residual=None):
        """The residual stack (reference :196-211): per layer x = x +
        mixer(rmsnorm(x)).  With a float32 residual (cfg.residual_in_fp32, or
        fp32_residual=True: the decode step's, reference :680) the add is fused
        into the next norm (one kernel per layer boundary).  block(i, xn,
        mixer) runs layer i's mixer.  -> (residual, last mixer output not yet
        added)."""
        cfg = self.config
        layers, mixers = params["layers"], self._prepared(params)
        if cfg.residual_in_fp32 if fp32_residual is None else fp32_residual:
            res = x.float().contiguous()        # a fresh buffer: updated in place
            out = None
            for i, (lp, mx) in enumerate(zip(layers, mixers)):
                dt = mx["in_proj_kernel"].dtype
                xn = rms_norm(res if out is None else out, lp["norm_weight"], out_dtype=dt,
                              residual=None if out is None else res)
                out = block(i, xn, mx)
            return res, out
        for i, (lp, mx) in enumerate(zip(layers, mixers)):
            xn = rms_norm(x.float(), lp["norm_weight"], out_dtype=mx["in_proj_kernel"].dtype)
            x = x + block(i, xn, mx).to(x.dtype)
        return x, None

    def _head(self, params, res, out=None):
        """final norm (with the last residual add) and the LM head -> float32
        logits: the reference multiplies the float32 normalised activations by
        the head weight, which promotes to a float32 matmul (:213-216,
        :732-736).  A decode-sized batch with bf16 weights runs the skinny GEMM
        on the bf16-rounded activations with float32 accumulation and output;
        otherwise the activations stay float32 and the matmul is float32
        throughout."""
        w = params["lm_head_weight"]
        src, resid = (res.float(), None) if out is None else (out, res)
        if res.dim() == 2 and linear.preferred_rows(res.shape[0], res.shape[1], w):
            xn = rms_norm(src, params["norm_f_weight"], out_dtype=w.dtype, residual=resid)
            return linear.linear_skinny(xn, w, out_dtype=torch.float32)
        xn = rms_norm(src, params["norm_f_weight"], residual=resid)
        return xn @ self._prepared(params, head=True).t()

    # -- prefill -------------------------------------------------------------
    def _layers(self, params, x, state=None):
        d = self.config.mixer_dims()

        def block(i, xn, mx):
            if state is None:
                return mamba2_block_forward(xn, mx, d)[0]
            return mamba2_block_forward(xn, mx, d, with_cache=True, conv_state=state.conv[i],
                                        ssm_state=state.ssm[i], inplace=True)[0]
        return self._run_layers(params, x, block)

    def __call__(self, params, input_ids):
        """input_ids (batch, seqlen) -> logits (batch, seqlen, vocab_size_padded)."""
        x = params["embedding"]["weight"][input_ids]
        return self._head(params, *self._layers(params, x))

    def prefill(self, params, input_ids, state: DecodeState):
        """Prefill that leaves every layer's conv / ssm state in ``state``
        (reference _forward_with_cache, :304-351); -> logits of the last token."""
        x = params["embedding"]["weight"][input_ids]
        return self._head(params, *self._layers(params, x, state))[:, -1, :]

    # -- decode ----------------------------------------------------------------
    def _fusable(self, params, batch):
        cfg = self.config
        w = params["lm_head_weight"]
        return (self.fuse_decode and w.dtype == torch.bfloat16
                and w.dim() == 2 and w.shape[1] % 8 == 0 and w.is_cuda
                and all(block_step_fusable(mx, cfg.mixer_dims(), batch, cfg.d_model)
                        for mx in self._prepared(params)))

    def decode_step(self, params, token, state: DecodeState):
        """token (batch,) -> next-token logits (batch, vocab) float32; states in
        place (reference _scan_decode_step, :667-736, whose residual is float32
        whatever residual_in_fp32 says, :680).  Batches of up to 2 rows with
        bf16 projections: each layer's norms run inside its projections
        (mamba2_block_step_fused; 4 kernels per layer), the final norm inside
        the LM head."""
        d = self.config.mixer_dims()
        x = params["embedding"]["weight"][token]
        if self._fusable(params, x.shape[0]):
            res = x.float().contiguous()
            if res.data_ptr() == x.data_ptr():
                res = res.clone()
            for i, (lp, mx) in enumerate(zip(params["layers"], self._prepared(params))):
                mamba2_block_step_fused(res, lp["norm_weight"], mx, d, state.conv[i], state.ssm[i])
            w = params["lm_head_weight"]
            return linear.linear_norm(res, params["norm_f_weight"], w, out_dtype=torch.float32)

        def block(i, xn, mx):
            return mamba2_block_step(xn, mx, d, state.conv[i], state.ssm[i], inplace=True)[0]
        return self._head(params, *self._run_layers(params, x, block, fp32_residual=True))

    def capture_decode(self, params, state: DecodeState, warmup=2):
        """Capture decode_step into a HIP graph over static token / logits
        buffers; returns (graph, token_buffer, logits_buffer).  Replaying it
        advances ``state`` by one token.  The warm-up steps run on copies of
        the states, which are restored before capture."""
        batch = state.conv.shape[1]
        tok = torch.zeros(batch, dtype=torch.long, device=state.conv.device)
        saved = (state.conv.clone(), state.ssm.clone())
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self.decode_step(params, tok, state)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            logits = self.decode_step(params, tok, state)
        state.conv.copy_(saved[0])
        state.ssm.copy_(saved[1])
        return g, tok, logits

    def generate(self, params, input_ids, max_new_tokens: int = 50, temperature: float = 1.0,
                 top_k: int = 50, rng_key=None, use_graph: bool = True):
        """Autoregressive generation (reference :219-302) -> (batch,
        prompt_len + max_new_tokens) token ids.  Batches of any size decode
        together; rng_key: an int seed or a torch.Generator."""
        batch = input_ids.shape[0]
        gen = rng_key if isinstance(rng_key, torch.Generator) else \
            torch.Generator(device=input_ids.device).manual_seed(0 if rng_key is None else int(rng_key))
        state = DecodeState(self.config, batch, input_ids.device)
        logits = self.prefill(params, input_ids, state)
        ids = [input_ids]
        graph = self.capture_decode(params, state) if use_graph else None
        for _ in range(max_new_tokens):
            nxt = _sample_token(logits, gen, temperature, top_k)
            ids.append(nxt[:, None])
            if graph is not None:
                g, tok, out = graph
                tok.copy_(nxt)
                g.replay()
                logits = out
            else:
                logits = self.decode_step(params, nxt, state)
        return torch.cat(ids, dim=1)


__all__ = ["Mamba2Config", "Mamba2LMHeadModel", "DecodeState", "MAMBA2_CONFIGS", "init_params",
           "load_from_pretrained", "load_from_torch_checkpoint", "read_state_dict", "rms_norm"]

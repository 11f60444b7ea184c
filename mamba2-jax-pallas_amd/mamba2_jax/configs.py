"""Benchmark / parity configurations and their seeded synthetic inputs.

The five configurations are the ones the benchmark contract names (c0..c4):
shapes, dtypes and value distributions follow it; seeds are fixed per config
(c0=0 ... c4=4).  Inputs are drawn with ``numpy.random.default_rng`` in float32
and, for bf16 configurations, rounded to bfloat16 (round-to-nearest-even, via
torch's cast) so that the host arrays hold exactly the values the device
tensors will hold.

Distributions (all configs):
  x, dt_raw, z ~ N(0, 1)
  dt_bias = inverse-softplus(dt0), dt0 log-uniform in [1e-3, 1e-1]
            (the Mamba2 dt init, reference modules/mamba2.py:599-616)
  A = -exp(U(log 1, log 16))
  B, C ~ N(0, 1) / sqrt(N)
  D ~ U(0.5, 1.5)
  initial / decode state ~ 0.1 * N(0, 1)
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np


@dataclasses.dataclass(frozen=True)
class SSDConfig:
    name: str
    batch: int
    seqlen: int
    nheads: int
    ngroups: int
    headdim: int
    dstate: int
    chunk_size: int
    dtype: str                 # 'f32' | 'bf16' : dtype of x, dt, B, C, z
    init_state: bool = False
    nseq: int = 0              # > 0: packed variable-length sequences (batch 1)
    min_seqlen: int = 256
    seed: int = 0

    @property
    def nchunks(self):
        return -(-self.seqlen // self.chunk_size)

    @property
    def tokens(self):
        return self.batch * self.seqlen


@dataclasses.dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    nheads: int
    ngroups: int
    headdim: int
    dstate: int
    steps: int
    dtype: str = "bf16"
    seed: int = 4


CONFIGS = {
    "c0": SSDConfig("mamba2-130m", 1, 2048, 24, 1, 64, 128, 256, "f32", seed=0),
    "c1": SSDConfig("mamba2-2.7b", 4, 2048, 80, 1, 64, 128, 256, "bf16",
                    init_state=True, seed=1),
    "c2": SSDConfig("nemotron-h-8b", 1, 4096, 128, 8, 64, 128, 128, "bf16", seed=2),
    "c3": SSDConfig("nemotron-h-47b-varlen", 1, 8192, 256, 8, 64, 256, 128, "bf16",
                    nseq=6, seed=3),
}
DECODE = DecodeConfig("nemotron-h-8b-decode", 64, 128, 8, 64, 128, 256, seed=4)


def round_to(a, dtype):
    """Round a float32 array to the values of ``dtype`` ('f32' | 'bf16')."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == "f32":
        return a
    if dtype == "bf16":
        import torch
        return torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    raise ValueError(f"unsupported dtype {dtype!r}")


def _head_params(rng, nheads):
    dt0 = np.exp(rng.uniform(math.log(1e-3), math.log(1e-1), nheads))
    dt_bias = dt0 + np.log(-np.expm1(-dt0))
    A = -np.exp(rng.uniform(math.log(1.0), math.log(16.0), nheads))
    D = rng.uniform(0.5, 1.5, nheads)
    return (dt_bias.astype(np.float32), A.astype(np.float32), D.astype(np.float32))


def packed_seqlens(rng, total, nseq, min_len):
    """Lengths >= min_len summing to ``total``, drawn from the seed."""
    extra = rng.multinomial(total - nseq * min_len, [1.0 / nseq] * nseq)
    return (min_len + extra).astype(np.int64)


def make_ssd_inputs(cfg: SSDConfig, seed=None, with_z=False):
    """Seeded host inputs (numpy) for one SSD layer forward."""
    rng = np.random.default_rng(cfg.seed if seed is None else seed)
    b, L, H, G, P, N = (cfg.batch, cfg.seqlen, cfg.nheads, cfg.ngroups,
                        cfg.headdim, cfg.dstate)
    dt_bias, A, D = _head_params(rng, H)
    x = rng.standard_normal((b, L, H, P), dtype=np.float32)
    dt = rng.standard_normal((b, L, H), dtype=np.float32)
    B = rng.standard_normal((b, L, G, N), dtype=np.float32) / np.float32(math.sqrt(N))
    C = rng.standard_normal((b, L, G, N), dtype=np.float32) / np.float32(math.sqrt(N))
    out = dict(x=round_to(x, cfg.dtype), dt=round_to(dt, cfg.dtype), A=A,
               B=round_to(B, cfg.dtype), C=round_to(C, cfg.dtype), D=D,
               dt_bias=dt_bias, z=None, initial_states=None, seq_idx=None,
               cu_seqlens=None)
    if cfg.init_state:
        out["initial_states"] = (0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32)
    if cfg.nseq:
        if b != 1:
            raise ValueError("packed sequences need batch == 1")
        lens = packed_seqlens(rng, L, cfg.nseq, cfg.min_seqlen)
        out["cu_seqlens"] = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        out["seq_idx"] = np.repeat(np.arange(cfg.nseq), lens)[None].astype(np.int32)
    if with_z:
        out["z"] = round_to(rng.standard_normal((b, L, H, P), dtype=np.float32), cfg.dtype)
    return out


def make_decode_inputs(cfg: DecodeConfig = DECODE, steps=None, with_z=True):
    """Seeded host inputs (numpy) for ``steps`` consecutive decode steps."""
    rng = np.random.default_rng(cfg.seed)
    b, H, G, P, N = cfg.batch, cfg.nheads, cfg.ngroups, cfg.headdim, cfg.dstate
    T = cfg.steps if steps is None else steps
    dt_bias, A, D = _head_params(rng, H)
    state = (0.1 * rng.standard_normal((b, H, P, N))).astype(np.float32)
    x = rng.standard_normal((T, b, H, P), dtype=np.float32)
    dt = rng.standard_normal((T, b, H), dtype=np.float32)
    B = rng.standard_normal((T, b, G, N), dtype=np.float32) / np.float32(math.sqrt(N))
    C = rng.standard_normal((T, b, G, N), dtype=np.float32) / np.float32(math.sqrt(N))
    z = rng.standard_normal((T, b, H, P), dtype=np.float32) if with_z else None
    return dict(state=state, x=round_to(x, cfg.dtype), dt=dt, A=A,
                B=round_to(B, cfg.dtype), C=round_to(C, cfg.dtype), D=D,
                dt_bias=dt_bias,
                z=None if z is None else round_to(z, cfg.dtype))

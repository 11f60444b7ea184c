"""Write the golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture holds small seeded inputs and the oracle's float64 outputs for
one case of the SSD forward or the decode step.  The reference ships no
vectors of its own (its tests draw inputs from jax.random at run time), so
these pin the oracle against regressions and give the GPU tests fixed
expected values; how the oracle itself is pinned is in tests/test_oracle.py.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mamba2-jax-pallas_amd")]

from mamba2_jax import configs  # noqa: E402
from oracle import ssd_oracle as O  # noqa: E402

SSD_CASES = {
    # name: (config, with_z, D per headdim, varlen)
    "ssd_f32_basic": (configs.SSDConfig("g", 1, 80, 4, 2, 32, 64, 32, "f32",
                                        init_state=True, seed=101), True, False, False),
    "ssd_bf16_groups": (configs.SSDConfig("g", 1, 128, 4, 2, 64, 64, 64, "bf16",
                                          seed=102), False, True, False),
    "ssd_bf16_varlen": (configs.SSDConfig("g", 1, 200, 2, 1, 64, 64, 64, "bf16",
                                          nseq=3, min_seqlen=32, seed=103), True, False, True),
}


def ssd_case(name):
    cfg, with_z, dhp, varlen = SSD_CASES[name]
    d = configs.make_ssd_inputs(cfg, with_z=with_z)
    if dhp:
        d["D"] = np.random.default_rng(cfg.seed).uniform(0.5, 1.5, (cfg.nheads, cfg.headdim)).astype(np.float32)
    res = O.ssd_combined(chunk_size=cfg.chunk_size, dt_softplus=True, return_final_states=True,
                         return_varlen_states=varlen, io_dtype=cfg.dtype, **d)
    out = {k: v for k, v in d.items() if v is not None}
    out["chunk_size"] = np.int32(cfg.chunk_size)
    out["io_dtype"] = np.array(cfg.dtype)
    out["want_out"], out["want_final"] = res[0], res[1]
    if varlen:
        out["want_varlen"] = res[2]
    return out


def ssu_case():
    cfg = configs.DecodeConfig("g", 2, 4, 2, 32, 64, 1, seed=104)
    d = configs.make_decode_inputs(cfg)
    step = {k: (v[0] if k in ("x", "dt", "B", "C", "z") else v) for k, v in d.items()}
    new, y = O.selective_state_update(**step, dt_softplus=True, round_fn=O.round_fn_for("bf16"))
    step["want_state"], step["want_out"] = new, y
    return step


def main():
    for name in SSD_CASES:
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **ssd_case(name))
    np.savez_compressed(os.path.join(HERE, "ssu_bf16_step.npz"), **ssu_case())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()

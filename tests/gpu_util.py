"""Helpers shared by the GPU parity tests (not collected by pytest)."""

import sys

import numpy as np
import torch

from oracle import ssd_oracle as O

DEV = "cuda"
# BASELINE parity bar: max |err| / rms(reference), per input dtype
TOL = {"f32": 1e-3, "bf16": 2e-2}


def tdtype(name):
    return torch.bfloat16 if name == "bf16" else torch.float32


def dev(a, dtype=None):
    """numpy -> GPU tensor (exact for values already representable in dtype)."""
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def host(t):
    return None if t is None else t.detach().float().cpu().numpy().astype(np.float64)


def check(got, want, tol, what):
    e = O.rel_err(host(got) if isinstance(got, torch.Tensor) else got, want)
    print(f"  {what}: max|err|/rms = {e:.3e} (tol {tol:.0e})", flush=True)
    assert np.isfinite(e) and e <= tol, f"{what}: {e:.3e} > {tol:.0e}"
    return e


def seq_idx_from_lengths(seq_lengths):
    return np.stack([np.repeat(np.arange(len(s)), s) for s in seq_lengths]).astype(np.int32)


def announce(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()

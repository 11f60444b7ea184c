"""The Mamba2 mixer layer on MI355X and the SSD dispatch it calls.

``_ssd_combined_fwd`` mirrors reference modules/mamba2.py:42-74: ``use_pallas=True``
(the default) runs the HIP kernels, ``use_pallas=False`` the naive formulation
on the GPU.  Unlike the reference, a failure of the HIP path is raised, never
swallowed into a silent fallback: a fallback would hide parity and performance
failures.

``Mamba2`` is the layer of reference modules/mamba2.py:80-549 as a torch
module over the HIP kernels: prefill (in-projection, causal conv + SiLU, SSD,
gated RMSNorm, out-projection) and the one-token decode step.  Same
constructor attributes, parameter names and shapes, call signature and return
values.  The projections are torch matmuls (hipBLASLt); everything between
them runs in libm2ssd.so:

* the conv writes x, B and C straight into the contiguous layouts the SSD
  kernels read (no split / reshape copies);
* rms_norm_gated reads z in place as a slice of the in-projection output;
* the decode step updates conv_state and ssm_state IN PLACE (what the
  reference gets from JAX buffer donation) and returns them in the new
  inference_params dict, so a decode loop allocates no per-step state.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from ..kernels.ssd_combined import mamba_chunk_scan_combined_fwd as _hip_fwd
from ..ops.causal_conv1d import causal_conv1d, causal_conv1d_update
from ..ops.rms_norm import rms_norm_gated
from ..ops.selective_state_update import selective_state_update
from ..ops.ssd_naive import mamba_chunk_scan_combined_naive


def _ssd_combined_fwd(use_pallas: bool = True, **kwargs):
    """The SSD layer forward: the HIP kernels, or the naive path if use_pallas=False."""
    if use_pallas:
        return _hip_fwd(**kwargs)
    return mamba_chunk_scan_combined_naive(**kwargs)


def _split_last(x, sizes):
    """Consecutive slices of the last dimension (reference modules/mamba2.py:642-652)."""
    out, start = [], 0
    for s in sizes:
        out.append(x[..., start:start + s])
        start += s
    return out


def _lecun_normal(shape, fan_in, gen, device, dtype):
    """Truncated normal (+-2 sigma) with variance 1 / fan_in, as flax's lecun_normal."""
    std = math.sqrt(1.0 / fan_in) / 0.8796256610342398   # stddev of N(0,1) truncated at 2
    t = torch.empty(shape, dtype=torch.float32)
    torch.nn.init.trunc_normal_(t, mean=0.0, std=std, a=-2 * std, b=2 * std, generator=gen)
    return t.to(device=device, dtype=dtype)


class Mamba2(torch.nn.Module):
    """One Mamba2 mixer layer (reference modules/mamba2.py:80-549).

    Parameters (torch.nn.Parameter, reference names): in_proj_kernel
    (d_model, d_in_proj), [in_proj_bias], conv1d_weight (conv_dim, d_conv),
    [conv1d_bias], dt_bias (nheads,) float32, A_log (nheads,), D (nheads,) or
    (d_ssm,), [norm_weight (d_ssm,)], out_proj_kernel (d_inner, d_model),
    [out_proj_bias].  ``param_dtype`` is their dtype (dt_bias stays float32);
    activations follow the parameters' dtype.
    """

    def __init__(self, d_model: int, d_state: int = 128, d_conv: int = 4,
                 conv_init: Optional[float] = None, expand: int = 2, headdim: int = 64,
                 d_ssm: Optional[int] = None, ngroups: int = 1,
                 A_init_range: Tuple[float, float] = (1.0, 16.0), D_has_hdim: bool = False,
                 rmsnorm: bool = True, norm_before_gate: bool = False, dt_min: float = 0.001,
                 dt_max: float = 0.1, dt_init_floor: float = 1e-4,
                 dt_limit: Tuple[float, float] = (0.0, float("inf")), bias: bool = False,
                 conv_bias: bool = True, chunk_size: int = 256, use_mem_eff_path: bool = True,
                 param_dtype=torch.float32, device=None, seed: int = 0):
        super().__init__()
        self.d_model, self.d_state, self.d_conv, self.expand = d_model, d_state, d_conv, expand
        self.headdim, self.ngroups, self.D_has_hdim = headdim, ngroups, D_has_hdim
        self.rmsnorm, self.norm_before_gate = rmsnorm, norm_before_gate
        self.dt_limit, self.chunk_size, self.use_mem_eff_path = tuple(dt_limit), chunk_size, use_mem_eff_path
        # derived sizes (reference modules/mamba2.py:180-204)
        self.d_inner = expand * d_model
        self._d_ssm = self.d_inner if d_ssm is None else d_ssm
        self.d_mlp = self.d_inner - self._d_ssm
        assert self._d_ssm % headdim == 0, f"d_ssm ({self._d_ssm}) must be divisible by headdim ({headdim})"
        self.nheads = self._d_ssm // headdim
        assert self.nheads % ngroups == 0, f"nheads ({self.nheads}) must be divisible by ngroups ({ngroups})"
        self.conv_dim = self._d_ssm + 2 * ngroups * d_state
        self.d_in_proj = 2 * self.d_inner + 2 * ngroups * d_state + self.nheads

        dev = torch.device("cuda") if device is None else torch.device(device)
        g = torch.Generator().manual_seed(seed)
        P = lambda t: torch.nn.Parameter(t, requires_grad=False)
        pd = param_dtype
        self.in_proj_kernel = P(_lecun_normal((d_model, self.d_in_proj), d_model, g, dev, pd))
        self.in_proj_bias = P(torch.zeros(self.d_in_proj, device=dev, dtype=pd)) if bias else None
        self.out_proj_kernel = P(_lecun_normal((self.d_inner, d_model), self.d_inner, g, dev, pd))
        self.out_proj_bias = P(torch.zeros(d_model, device=dev, dtype=pd)) if bias else None
        if conv_init is not None:
            w = (torch.rand((self.conv_dim, d_conv), generator=g) * 2 - 1) * conv_init
            self.conv1d_weight = P(w.to(dev, pd))
        else:
            self.conv1d_weight = P(_lecun_normal((self.conv_dim, d_conv), self.conv_dim, g, dev, pd))
        self.conv1d_bias = P(torch.zeros(self.conv_dim, device=dev, dtype=pd)) if conv_bias else None
        # dt_bias: inverse softplus of log-uniform dt (reference :600-617), float32
        u = torch.rand(self.nheads, generator=g, dtype=torch.float64)
        dt = torch.exp(u * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min)).clamp(min=dt_init_floor)
        self.dt_bias = P((dt + torch.log(-torch.expm1(-dt))).to(dev, torch.float32))
        # A_log = log(uniform(A_init_range)) (reference :620-634)
        A = torch.rand(self.nheads, generator=g, dtype=torch.float64) * (A_init_range[1] - A_init_range[0]) \
            + A_init_range[0]
        self.A_log = P(torch.log(A).to(dev, pd))
        self.D = P(torch.ones(self._d_ssm if D_has_hdim else self.nheads, device=dev, dtype=pd))
        self.norm_weight = P(torch.ones(self._d_ssm, device=dev, dtype=pd)) if rmsnorm else None

    # -- helpers -----------------------------------------------------------
    def _A(self):
        return -torch.exp(self.A_log.float())

    def _D(self):
        return self.D.view(self.nheads, self.headdim) if self.D_has_hdim else self.D

    def _in_proj(self, h):
        z = h @ self.in_proj_kernel
        return z if self.in_proj_bias is None else z + self.in_proj_bias

    def _out(self, y, z, z0, x0):
        """gated RMSNorm, the MLP bypass, out-projection (reference :400-414)."""
        if self.rmsnorm:
            y = rms_norm_gated(y, self.norm_weight, z=z, group_size=self._d_ssm // self.ngroups,
                               norm_before_gate=self.norm_before_gate)
        if self.d_mlp > 0:
            y = torch.cat([torch.nn.functional.silu(z0) * x0, y.to(x0.dtype)], dim=-1)
        y = y.to(self.out_proj_kernel.dtype)
        out = y @ self.out_proj_kernel
        return out if self.out_proj_bias is None else out + self.out_proj_bias

    # -- forward -----------------------------------------------------------
    def forward(self, u, seq_idx=None, cu_seqlens=None, inference_params=None):
        """u (batch, seqlen, d_model) -> out (batch, seqlen, d_model), plus the
        new inference_params dict when inference_params is given
        (reference modules/mamba2.py:163-424)."""
        if inference_params is not None and inference_params.get("seqlen_offset", 0) > 0:
            return self._step(u, inference_params)
        batch, seqlen, _ = u.shape
        G, N, H, Pd = self.ngroups, self.d_state, self.nheads, self.headdim
        zxbcdt = self._in_proj(u.to(self.in_proj_kernel.dtype))
        z0, x0, z, xBC, dt = _split_last(
            zxbcdt, [self.d_mlp, self.d_mlp, self._d_ssm, self.conv_dim, self.nheads])
        new_conv_state = None
        if inference_params is not None:
            # the last d_conv inputs of the conv (left-padded with zeros)
            xT = xBC.transpose(1, 2)
            if seqlen >= self.d_conv:
                new_conv_state = xT[:, :, -self.d_conv:]
            else:
                new_conv_state = torch.nn.functional.pad(xT, (self.d_conv - seqlen, 0))
            cs = inference_params.get("conv_state")
            if cs is not None and tuple(cs.shape) == tuple(new_conv_state.shape):
                cs.copy_(new_conv_state)
                new_conv_state = cs
            else:
                new_conv_state = new_conv_state.contiguous()
        # conv + SiLU into x, B, C (contiguous, the SSD's layouts)
        xs, Bs, Cs = causal_conv1d(xBC.transpose(1, 2), self.conv1d_weight, self.conv1d_bias,
                                   "silu", seq_idx, split_sizes=(self._d_ssm, G * N, G * N))
        x = xs.transpose(1, 2).view(batch, seqlen, H, Pd)
        B = Bs.transpose(1, 2).view(batch, seqlen, G, N)
        C = Cs.transpose(1, 2).view(batch, seqlen, G, N)
        z_scan = None if self.rmsnorm else z.reshape(batch, seqlen, H, Pd)
        return_final = inference_params is not None
        res = _ssd_combined_fwd(x=x, dt=dt, A=self._A(), B=B, C=C, chunk_size=self.chunk_size,
                                D=self._D(), z=z_scan, dt_bias=self.dt_bias, dt_softplus=True,
                                dt_limit=self.dt_limit, seq_idx=seq_idx, cu_seqlens=cu_seqlens,
                                return_final_states=return_final, return_varlen_states=False)
        y, final = (res if return_final else (res, None))
        out = self._out(y.reshape(batch, seqlen, self._d_ssm), z, z0, x0)
        if inference_params is None:
            return out
        ss = inference_params.get("ssm_state")
        if ss is not None and tuple(ss.shape) == tuple(final.shape) and ss.dtype == final.dtype:
            ss.copy_(final)
            final = ss
        return out, {"conv_state": new_conv_state, "ssm_state": final,
                     "seqlen_offset": inference_params.get("seqlen_offset", 0) + seqlen}

    def _step(self, u, inference_params):
        """One decode token (reference modules/mamba2.py:427-549); the states
        in inference_params are updated in place."""
        G, N, H, Pd = self.ngroups, self.d_state, self.nheads, self.headdim
        zxbcdt = self._in_proj(u[:, 0, :].to(self.in_proj_kernel.dtype))
        z0, x0, z, xBC, dt = _split_last(
            zxbcdt, [self.d_mlp, self.d_mlp, self._d_ssm, self.conv_dim, self.nheads])
        conv_state, ssm_state = inference_params["conv_state"], inference_params["ssm_state"]
        conv_state, (x, B, C) = causal_conv1d_update(
            xBC, conv_state, self.conv1d_weight, self.conv1d_bias, "silu",
            split_sizes=(self._d_ssm, G * N, G * N))
        batch = u.shape[0]
        z_step = None if self.rmsnorm else z.reshape(batch, H, Pd)
        ssm_state, y = selective_state_update(
            ssm_state, x.view(batch, H, Pd), dt, self._A(), B.view(batch, G, N), C.view(batch, G, N),
            D=self._D(), z=z_step, dt_bias=self.dt_bias, dt_softplus=True)
        out = self._out(y.reshape(batch, self._d_ssm), z, z0, x0)
        return out[:, None, :], {"conv_state": conv_state, "ssm_state": ssm_state,
                                 "seqlen_offset": inference_params["seqlen_offset"] + 1}


def allocate_inference_cache(batch_size: int, d_model: int, d_state: int = 128, d_conv: int = 4,
                             expand: int = 2, headdim: int = 64, d_ssm: Optional[int] = None,
                             ngroups: int = 1, dtype=torch.float32, device=None):
    """Zero conv / ssm states (reference modules/mamba2.py:556-595)."""
    d_inner = expand * d_model
    d_ssm = d_inner if d_ssm is None else d_ssm
    nheads = d_ssm // headdim
    conv_dim = d_ssm + 2 * ngroups * d_state
    dev = torch.device("cuda") if device is None else torch.device(device)
    return {"conv_state": torch.zeros((batch_size, conv_dim, d_conv), dtype=dtype, device=dev),
            "ssm_state": torch.zeros((batch_size, nheads, headdim, d_state), dtype=dtype, device=dev),
            "seqlen_offset": 0}


__all__ = ["_ssd_combined_fwd", "selective_state_update", "Mamba2", "allocate_inference_cache"]

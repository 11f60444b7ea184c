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
* the decode step returns new conv / ssm states in the new inference_params
  dict and leaves the caller's untouched, as the reference does; with the
  keyword-only ``inplace=True`` it updates them in place instead (what the
  reference gets from JAX buffer donation), so a decode loop that owns its
  states allocates none per step.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from ..kernels.ssd_combined import mamba_chunk_scan_combined_fwd as _hip_fwd
from ..ops import linear as _lin
from ..ops.causal_conv1d import causal_conv1d, causal_conv1d_update, update_from_columns
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

    def dims(self):
        return MixerDims(d_ssm=self._d_ssm, d_mlp=self.d_mlp, ngroups=self.ngroups,
                         d_state=self.d_state, headdim=self.headdim, nheads=self.nheads,
                         d_conv=self.d_conv, chunk_size=self.chunk_size, rmsnorm=self.rmsnorm,
                         norm_before_gate=self.norm_before_gate, D_has_hdim=self.D_has_hdim,
                         dt_limit=self.dt_limit)

    def params(self):
        """The parameters by reference name (absent optional ones as None)."""
        return {k: getattr(self, k) for k in _PARAM_NAMES}

    def forward(self, u, seq_idx=None, cu_seqlens=None, inference_params=None, *, inplace=False):
        """u (batch, seqlen, d_model) -> out (batch, seqlen, d_model), plus the
        new inference_params dict when inference_params is given
        (reference modules/mamba2.py:163-424).  The states in the given
        inference_params are left untouched unless ``inplace`` (then the
        returned dict holds the same, updated, tensors)."""
        if inference_params is not None and inference_params.get("seqlen_offset", 0) > 0:
            conv_state, ssm_state = inference_params["conv_state"], inference_params["ssm_state"]
            out, conv_state, ssm_state = mamba2_block_step(u[:, 0, :], self.params(), self.dims(),
                                                           conv_state, ssm_state, inplace=inplace)
            return out[:, None, :], {"conv_state": conv_state, "ssm_state": ssm_state,
                                     "seqlen_offset": inference_params["seqlen_offset"] + 1}
        if inference_params is None:
            out, _, _ = mamba2_block_forward(u, self.params(), self.dims(), seq_idx, cu_seqlens)
            return out
        out, conv_state, ssm_state = mamba2_block_forward(
            u, self.params(), self.dims(), seq_idx, cu_seqlens, with_cache=True,
            conv_state=inference_params.get("conv_state"),
            ssm_state=inference_params.get("ssm_state"), inplace=inplace)
        return out, {"conv_state": conv_state, "ssm_state": ssm_state,
                     "seqlen_offset": inference_params.get("seqlen_offset", 0) + u.shape[1]}


_PARAM_NAMES = ("in_proj_kernel", "in_proj_bias", "conv1d_weight", "conv1d_bias", "dt_bias",
                "A_log", "D", "norm_weight", "out_proj_kernel", "out_proj_bias")


@dataclass(frozen=True)
class MixerDims:
    """The sizes and flags one mixer layer's computation needs."""
    d_ssm: int
    d_mlp: int
    ngroups: int
    d_state: int
    headdim: int
    nheads: int
    d_conv: int
    chunk_size: int
    rmsnorm: bool = True
    norm_before_gate: bool = False
    D_has_hdim: bool = False
    dt_limit: Tuple[float, float] = (0.0, float("inf"))

    @property
    def conv_dim(self):
        return self.d_ssm + 2 * self.ngroups * self.d_state


def _proj(h, p, name, out_dtype=None):
    """h @ p[name + "_kernel"] (+ bias).  A decode-sized h (<= 16 rows) with a
    K-contiguous bf16 copy p[name + "_t"] ([out, in], prepared by the caller)
    runs the HIP skinny GEMM; anything else is a torch matmul (hipBLASLt).
    out_dtype=torch.float32 with bf16 operands keeps the float32 accumulation
    as the result (no rounding to bf16)."""
    wt, b = p.get(name + "_t"), p.get(name + "_bias")
    if wt is not None and h.dim() == 2 and _lin.preferred(h, wt):
        return _lin.linear_skinny(h, wt, b, out_dtype=out_dtype or wt.dtype)
    w = p[name + "_kernel"]
    if out_dtype == torch.float32 and h.dtype == torch.bfloat16 and w.dtype == torch.bfloat16:
        z = torch.mm(h.reshape(-1, h.shape[-1]), w, out_dtype=torch.float32)
        z = z.reshape(*h.shape[:-1], w.shape[-1])
    else:
        z = h @ w
    z = z if b is None else z + b
    return z if out_dtype is None else z.to(out_dtype)


def _in_proj(h, p):
    return _proj(h, p, "in_proj")


def _mixer_out(y, z, z0, x0, p, d):
    """gated RMSNorm, the MLP bypass, out-projection (reference :400-414).
    Without the MLP bypass the norm stores straight in the projection's dtype.
    The result is float32, as the reference's: its SSD output, and so the
    norm's, is float32, and a float32 activation times a bf16 kernel promotes
    to float32 (the activation itself goes to the bf16 GEMM in bf16)."""
    if d.rmsnorm:
        y = rms_norm_gated(y, p["norm_weight"], z=z, group_size=d.d_ssm // d.ngroups,
                           norm_before_gate=d.norm_before_gate,
                           out_dtype=p["out_proj_kernel"].dtype if d.d_mlp == 0 else None)
    if d.d_mlp > 0:
        y = torch.cat([torch.nn.functional.silu(z0) * x0, y.to(x0.dtype)], dim=-1)
    return _proj(y.to(p["out_proj_kernel"].dtype), p, "out_proj", out_dtype=torch.float32)


def _A(p):
    """A = -exp(A_log) (reference :293), or a precomputed p["A"]."""
    A = p.get("A")
    return -torch.exp(p["A_log"].float()) if A is None else A


def _D(p, d):
    return p["D"].view(d.nheads, d.headdim) if d.D_has_hdim else p["D"]


def mamba2_block_forward(u, p, d, seq_idx=None, cu_seqlens=None, with_cache=False,
                         conv_state=None, ssm_state=None, inplace=False):
    """Prefill of one mixer (reference modules/mamba2.py:296-424) from a
    parameter dict ``p`` (reference names) and MixerDims ``d``.

    -> (out (batch, seqlen, d_model), conv_state, ssm_state); the states are
    None unless with_cache (conv_state: the last d_conv conv inputs,
    left-padded with zeros; ssm_state: the SSD's final states).  They are new
    tensors, or, with ``inplace``, written into the given conv_state /
    ssm_state when their shapes and dtypes match.
    """
    batch, seqlen, _ = u.shape
    G, N, H, Pd = d.ngroups, d.d_state, d.nheads, d.headdim
    zxbcdt = _in_proj(u.to(p["in_proj_kernel"].dtype), p)
    z0, x0, z, xBC, dt = _split_last(zxbcdt, [d.d_mlp, d.d_mlp, d.d_ssm, d.conv_dim, d.nheads])
    new_conv = None
    if with_cache:
        xT = xBC.transpose(1, 2)
        if seqlen >= d.d_conv:
            new_conv = xT[:, :, -d.d_conv:]
        else:
            new_conv = torch.nn.functional.pad(xT, (d.d_conv - seqlen, 0))
        if inplace and conv_state is not None and tuple(conv_state.shape) == tuple(new_conv.shape):
            conv_state.copy_(new_conv)
            new_conv = conv_state
        else:
            new_conv = new_conv.contiguous()
    # conv + SiLU into x, B, C (contiguous, the SSD's layouts)
    xs, Bs, Cs = causal_conv1d(xBC.transpose(1, 2), p["conv1d_weight"], p.get("conv1d_bias"),
                               "silu", seq_idx, split_sizes=(d.d_ssm, G * N, G * N))
    x = xs.transpose(1, 2).view(batch, seqlen, H, Pd)
    B = Bs.transpose(1, 2).view(batch, seqlen, G, N)
    C = Cs.transpose(1, 2).view(batch, seqlen, G, N)
    z_scan = None if d.rmsnorm else z.reshape(batch, seqlen, H, Pd)
    res = _ssd_combined_fwd(x=x, dt=dt, A=_A(p), B=B, C=C, chunk_size=d.chunk_size, D=_D(p, d),
                            z=z_scan, dt_bias=p["dt_bias"], dt_softplus=True, dt_limit=d.dt_limit,
                            seq_idx=seq_idx, cu_seqlens=cu_seqlens,
                            return_final_states=with_cache, return_varlen_states=False)
    y, final = res if with_cache else (res, None)
    out = _mixer_out(y.reshape(batch, seqlen, d.d_ssm), z, z0, x0, p, d)
    if with_cache and inplace and ssm_state is not None \
            and tuple(ssm_state.shape) == tuple(final.shape) and ssm_state.dtype == final.dtype:
        ssm_state.copy_(final)
        final = ssm_state
    return out, new_conv, final


def mamba2_block_step(u_t, p, d, conv_state, ssm_state, inplace=False):
    """One decode token of one mixer (reference modules/mamba2.py:427-549):
    u_t (batch, d_model) -> (out (batch, d_model), new conv_state, new
    ssm_state).  With ``inplace`` the given float32 states are updated in place
    and returned (no per-step state allocation)."""
    G, N, H, Pd = d.ngroups, d.d_state, d.nheads, d.headdim
    batch = u_t.shape[0]
    zxbcdt = _in_proj(u_t.to(p["in_proj_kernel"].dtype), p)
    z0, x0, z, xBC, dt = _split_last(zxbcdt, [d.d_mlp, d.d_mlp, d.d_ssm, d.conv_dim, d.nheads])
    conv_state, (x, B, C) = causal_conv1d_update(
        xBC, conv_state, p["conv1d_weight"], p.get("conv1d_bias"), "silu",
        inplace=inplace, split_sizes=(d.d_ssm, G * N, G * N))
    z_step = None if d.rmsnorm else z.reshape(batch, H, Pd)
    ssm_state, y = selective_state_update(
        ssm_state, x.view(batch, H, Pd), dt, _A(p), B.view(batch, G, N), C.view(batch, G, N),
        D=_D(p, d), z=z_step, dt_bias=p["dt_bias"], dt_softplus=True, inplace=inplace)
    out = _mixer_out(y.reshape(batch, d.d_ssm), z, z0, x0, p, d)
    return out, conv_state, ssm_state


def block_step_fusable(p, d, batch, d_model):
    """True when mamba2_block_step_fused can run this mixer at this batch: bf16
    projections with their [out, in] copies, the gated norm (no MLP bypass),
    and rows the normalising GEMM takes and runs faster than the separate
    kernels (<= 2 rows, 4-element aligned)."""
    return (d.rmsnorm and d.d_mlp == 0 and p.get("in_proj_t") is not None
            and p.get("out_proj_t") is not None and batch <= _lin.NORM_PREFERRED_ROWS
            and batch * max(d_model, d.d_ssm) <= _lin.NORM_MAX_ELEMS and d_model % 8 == 0
            and d.d_ssm % 8 == 0 and (d.d_ssm // d.ngroups) % 4 == 0
            and d.ngroups <= _lin.NORM_MAX_GROUPS and (2 * d.d_ssm + 2 * d.ngroups * d.d_state
                                                        + d.nheads) % 4 == 0)


def mamba2_block_step_fused(res, norm_weight, p, d, conv_state, ssm_state, eps=1e-5):
    """One decode token of a pre-norm residual block, res += mixer(rmsnorm(res))
    (reference models/mamba2_lm.py:205-211 around modules/mamba2.py:427-549),
    in four kernels: the block's RMSNorm runs in the in-projection's prologue,
    the gated norm in the out-projection's, whose epilogue adds the float32
    output (the reference's promotion of a float32 activation times a bf16
    kernel) into res.  res (batch, d_model)
    float32 and the states are updated in place; block_step_fusable must hold.
    The results equal mamba2_block_step's around rms_norm up to the rounding
    of the norms' sums of squares (summed in another order)."""
    G, N, H, Pd = d.ngroups, d.d_state, d.nheads, d.headdim
    batch = res.shape[0]
    odt = p["in_proj_t"].dtype
    if conv_state.dtype == torch.float32 and conv_state.is_contiguous() and d.d_conv == 4:
        # the conv update runs in the in-projection's epilogue on the xBC columns
        cargs, (x, B, C) = update_from_columns(conv_state, p["conv1d_weight"], p.get("conv1d_bias"),
                                               "silu", x_dtype=odt, split_sizes=(d.d_ssm, G * N, G * N))
        zxbcdt = _lin.linear_norm(res, norm_weight, p["in_proj_t"], eps=eps, bias=p.get("in_proj_bias"),
                                  out_dtype=odt, conv_update=(cargs, d.d_ssm))
        _, _, z, _, dt = _split_last(zxbcdt, [0, 0, d.d_ssm, d.conv_dim, d.nheads])
    else:
        zxbcdt = _lin.linear_norm(res, norm_weight, p["in_proj_t"], eps=eps,
                                  bias=p.get("in_proj_bias"), out_dtype=odt)
        _, _, z, xBC, dt = _split_last(zxbcdt, [0, 0, d.d_ssm, d.conv_dim, d.nheads])
        conv_state, (x, B, C) = causal_conv1d_update(
            xBC, conv_state, p["conv1d_weight"], p.get("conv1d_bias"), "silu",
            inplace=True, split_sizes=(d.d_ssm, G * N, G * N))
    ssm_state, y = selective_state_update(
        ssm_state, x.view(batch, H, Pd), dt, _A(p), B.view(batch, G, N), C.view(batch, G, N),
        D=_D(p, d), dt_bias=p["dt_bias"], dt_softplus=True, inplace=True)
    _lin.linear_norm(y.view(batch, d.d_ssm), p["norm_weight"], p["out_proj_t"], z=z,
                     group_size=d.d_ssm // G, norm_before_gate=d.norm_before_gate,
                     bias=p.get("out_proj_bias"), out_dtype=torch.float32, residual=res,
                     store=False)
    return res, conv_state, ssm_state


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


__all__ = ["_ssd_combined_fwd", "selective_state_update", "Mamba2", "MixerDims",
           "mamba2_block_forward", "mamba2_block_step", "mamba2_block_step_fused",
           "block_step_fusable", "allocate_inference_cache"]

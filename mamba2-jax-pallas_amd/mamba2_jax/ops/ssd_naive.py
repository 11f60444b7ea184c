"""The reference's naive SSD forward, as plain torch tensor ops on the GPU.

Restates reference ops/ssd_naive.py:26-397 stage by stage (the einsum
formulation, float32 arithmetic) for device tensors.  It is what
``modules.mamba2._ssd_combined_fwd(use_pallas=False)`` selects explicitly, and
a full-size float32 cross-check for the HIP path; it is never used as a
fallback.  Like the reference it ignores seq_idx / cu_seqlens, and pads the
raw dt before the softplus (so padded positions carry softplus(dt_bias)).
For bf16 inputs it rounds where the reference rounds: CB, the carried states,
the C @ states product and silu(z).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .. import _lib as L


def _r(t, dtype):
    """Round a float32 tensor to `dtype` and back (identity for float32)."""
    return t if dtype == torch.float32 else t.to(dtype).to(torch.float32)


def chunk_cumsum_naive(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                       dt_limit=(0.0, float("inf"))):
    """ssd_naive.py:26-70 -> (dA_cumsum, dt) each (b, H, nc, Q) float32."""
    b, L_, H = dt.shape
    nc = math.ceil(L_ / chunk_size)
    pad = nc * chunk_size - L_
    d = dt.float()
    if pad:
        d = F.pad(d, (0, 0, 0, pad))
    d = d.reshape(b, nc, chunk_size, H).permute(0, 3, 1, 2)
    if dt_bias is not None:
        d = d + dt_bias.float()[None, :, None, None]
    if dt_softplus:
        d = F.softplus(d)
    d = d.clamp(dt_limit[0], dt_limit[1])
    dA = d * A.float()[None, :, None, None]
    return torch.cumsum(dA, dim=-1), d.contiguous()


def chunk_state_naive(B, x, dt, dA_cumsum):
    """ssd_naive.py:77-128 -> (b, nc, H, P, N) float32."""
    b, L_, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    _, _, nc, Q = dt.shape
    T = nc * Q
    xf = F.pad(x.float(), (0, 0, 0, 0, 0, T - L_))
    Bf = F.pad(B.float(), (0, 0, 0, 0, 0, T - L_))
    w = torch.exp(dA_cumsum[..., -1:] - dA_cumsum) * dt                  # (b,H,nc,Q)
    xw = xf.reshape(b, nc, Q, H, P) * w.permute(0, 2, 3, 1)[..., None]    # (b,nc,Q,H,P)
    lhs = xw.permute(0, 1, 3, 4, 2).reshape(b, nc, G, H // G, P, Q).contiguous()
    rhs = Bf.reshape(b, nc, Q, G, N).permute(0, 1, 3, 2, 4)[:, :, :, None].contiguous()
    return torch.matmul(lhs, rhs).reshape(b, nc, H, P, N)


def state_passing_naive(states, dA_chunk_cumsum, initial_states=None):
    """ssd_naive.py:135-182 (pairwise decay) -> (out, final)."""
    b, nc, H, D = states.shape
    init = (torch.zeros((b, H, D), dtype=torch.float32, device=states.device)
            if initial_states is None else initial_states.float())
    st = torch.cat([init[:, None], states.float()], dim=1)              # (b,nc+1,H,D)
    cs = torch.cumsum(F.pad(dA_chunk_cumsum.float(), (1, 0)), dim=-1)   # (b,H,nc+1)
    n1 = nc + 1
    expo = cs[..., :, None] - cs[..., None, :]
    tril = torch.ones((n1, n1), dtype=torch.bool, device=states.device).tril()
    decay = torch.exp(expo.masked_fill(~tril, float("-inf")))          # (b,H,z,c)
    out = torch.matmul(decay, st.permute(0, 2, 1, 3).contiguous())     # (b,H,z,D)
    out = out.permute(0, 2, 1, 3)
    return out[:, :-1], out[:, -1]


def bmm_chunk_naive(C, B, chunk_size):
    """ssd_naive.py:189-216 -> (b, nc, G, Q, Q) float32 (rounded like C.dtype)."""
    b, L_, G, N = C.shape
    nc = math.ceil(L_ / chunk_size)
    T = nc * chunk_size
    Cf = F.pad(C.float(), (0, 0, 0, 0, 0, T - L_)).reshape(b, nc, chunk_size, G, N)
    Bf = F.pad(B.float(), (0, 0, 0, 0, 0, T - L_)).reshape(b, nc, chunk_size, G, N)
    CB = torch.matmul(Cf.permute(0, 1, 3, 2, 4).contiguous(),
                      Bf.permute(0, 1, 3, 4, 2).contiguous())
    return _r(CB, C.dtype)


def chunk_scan_naive(CB, x, dt, dA_cumsum, C, prev_states, D=None, z=None):
    """ssd_naive.py:223-318 -> (out, out_x)."""
    b, L_, H, P = x.shape
    G, N = C.shape[2], C.shape[3]
    _, _, nc, Q = dt.shape
    hpg = H // G
    T = nc * Q
    xf = F.pad(x.float(), (0, 0, 0, 0, 0, T - L_))
    Cf = F.pad(C.float(), (0, 0, 0, 0, 0, T - L_))
    tril = torch.ones((Q, Q), dtype=torch.bool, device=x.device).tril()
    expo = dA_cumsum[..., :, None] - dA_cumsum[..., None, :]             # (b,H,nc,l,s)
    decay = torch.exp(expo.masked_fill(~tril, float("-inf"))).permute(0, 2, 1, 3, 4)
    scores = CB.float().repeat_interleave(hpg, dim=2) * decay           # (b,nc,H,l,s)
    scores = scores * dt.permute(0, 2, 1, 3)[:, :, :, None, :]
    xc = xf.reshape(b, nc, Q, H, P).permute(0, 1, 3, 2, 4).contiguous()  # (b,nc,H,s,P)
    out = torch.matmul(scores.contiguous(), xc)                         # (b,nc,H,l,P)
    ps = _r(prev_states.float(), C.dtype)                               # (b,nc,H,P,N)
    Ch = Cf.reshape(b, nc, Q, G, N).permute(0, 1, 3, 2, 4).repeat_interleave(hpg, dim=2)
    inter = _r(torch.matmul(Ch.contiguous(), ps.transpose(-1, -2).contiguous()), C.dtype)
    out = out + inter * torch.exp(dA_cumsum).permute(0, 2, 1, 3)[..., None]
    out = out.permute(0, 1, 3, 2, 4).reshape(b, T, H, P)[:, :L_]
    if D is not None:
        Df = D.float()
        out = out + x.float() * (Df[None, None, :, None] if Df.dim() == 1 else Df[None, None])
    out_x = None
    if z is not None:
        out_x = out
        out = out * F.silu(z).float()          # silu in z's dtype, as jax.nn.silu
    return out, out_x


def mamba_chunk_scan_combined_naive(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                                    initial_states=None, dt_softplus=False,
                                    dt_limit=(0.0, float("inf")), return_final_states=False,
                                    seq_idx=None, cu_seqlens=None, return_varlen_states=False):
    """ssd_naive.py:325-397.  seq_idx / cu_seqlens / return_varlen_states are
    accepted and ignored, as in the reference."""
    L.device_of(x, dt, A, B, C, D, z, dt_bias, initial_states)
    b, L_, H, P = x.shape
    N = B.shape[3]
    dA, dto = chunk_cumsum_naive(dt, A, chunk_size, dt_bias, dt_softplus, dt_limit)
    st = chunk_state_naive(B, x, dto, dA)
    nc = st.shape[1]
    init = None if initial_states is None else initial_states.reshape(b, H, P * N)
    sp, fin = state_passing_naive(st.reshape(b, nc, H, P * N), dA[..., -1], init)
    sp = sp.reshape(b, nc, H, P, N)
    fin = fin.reshape(b, H, P, N)
    CB = bmm_chunk_naive(C, B, chunk_size)
    out, _ = chunk_scan_naive(CB, x, dto, dA, C, sp, D=D, z=z)
    return (out, fin) if return_final_states else out

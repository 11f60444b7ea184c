"""CPU oracle for the Mamba2 SSD forward and the selective-state-update decode step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline) -- never as a product path.  The product
(``mamba2_jax``) runs the HIP kernels in ``libm2ssd.so`` and has no CPU path.

This is a NumPy restatement of the reference's naive path
(``/root/reference/src/mamba2_jax/ops/ssd_naive.py``), of the seq_idx / varlen
rules its kernel wrappers add, and of ``ops/selective_state_update.py``.  Every
function cites the reference lines it follows.  Arithmetic runs in the dtype
given by ``acc`` (float64 for parity checks, float32 for the CPU baseline).

Reference precision quirks reproduced on purpose (``round_fn``):
  * CB = C @ B^T is an einsum of the input dtype, so bf16 inputs give a bf16 CB
    (ssd_naive.py:214-216);
  * jax.nn.silu(z) keeps z's dtype (ssd_naive.py:316, selective_state_update.py:121);
  * states_passed is cast to C.dtype before the inter-chunk term
    (ssd_naive.py:296, kernels/ssd_combined.py:140);
  * the inter-chunk einsum ``C @ states`` has the input dtype as result type and
    is rounded before the fp32 decay multiply (ssd_naive.py:294-297).
For fp32 inputs ``round_fn`` is the identity.

How each function is pinned (tests/test_oracle.py):
  chunk_cumsum        closed form + prefix sums; dt->-inf gives dA=0; A=0 gives 0
  chunk_state         brute-force outer-product loop; Q=1 closed form
  state_passing       pairwise (ssd_naive) == sequential (test-local) formulation;
                      dA=0 gives prefix sums
  bmm_chunk           float64 matmul per chunk; causal / seq masks by loops
  chunk_scan +        whole SSD == token-by-token recurrence (ssd_sequential);
  ssd_combined        chunk-size invariance
  chunk_state_varlen  packed run == independent per-sequence runs
  selective_state_update  closed form (tests/test_mamba2_ops.py:48-56, 94-103)
                      and 256 steps == SSD prefill over the same tokens
"""

from __future__ import annotations

import math

import numpy as np

INF = float("inf")


# ---------------------------------------------------------------------------
# bf16 emulation (round to nearest even), ml_dtypes is not available
# ---------------------------------------------------------------------------

def bf16_round(a):
    """Round to the nearest bfloat16 value (RNE), returned as float32."""
    a32 = np.ascontiguousarray(a, dtype=np.float32)
    u = a32.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    out = r.view(np.float32).reshape(a32.shape)
    nan = np.isnan(a32)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def identity(a):
    return a


def round_fn_for(dtype_name):
    """The rounding the reference applies for an input dtype.

    'bf16' and 'f32' round to that dtype; None is the identity (exact float64
    arithmetic, used when checking the oracle against other formulations).
    """
    if dtype_name is None:
        return identity
    if dtype_name == "bf16":
        return lambda a: bf16_round(a).astype(np.asarray(a).dtype)
    if dtype_name == "f32":
        return lambda a: np.asarray(a, dtype=np.float32).astype(np.asarray(a).dtype)
    raise ValueError(dtype_name)


def softplus(v):
    """jax.nn.softplus == log(1 + exp(v)), computed stably."""
    return np.logaddexp(v, 0.0)


def silu(v):
    return v / (1.0 + np.exp(-v))


# ---------------------------------------------------------------------------
# 1. chunk_cumsum  (ssd_naive.py:26-70; kernels/chunk_cumsum_fwd.py:213-235)
# ---------------------------------------------------------------------------

def chunk_cumsum(dt, A, chunk_size, dt_bias=None, dt_softplus=False,
                 dt_limit=(0.0, INF), pad="kernel", acc=np.float64):
    """dt (b, L, H) -> (dA_cumsum, dt_out), each (b, H, nc, Q).

    pad="kernel": bias/softplus/clip first, then zero-pad (the kernel wrapper,
    kernels/chunk_cumsum_fwd.py:221-231, and mamba_ssm's Triton kernel): padded
    positions carry dt'=0.
    pad="naive": zero-pad the raw dt first (ssd_naive.py:46-48), so padded
    positions carry softplus(bias).  Only differs when L % Q != 0.
    dA_cumsum = cumsum(dt' * A) as in ssd_naive.py:67-68.
    """
    dt = np.asarray(dt, dtype=acc)
    A = np.asarray(A, dtype=acc)
    b, L, H = dt.shape
    nc = -(-L // chunk_size)
    padl = nc * chunk_size - L

    def process(v):
        if dt_bias is not None:
            v = v + np.asarray(dt_bias, dtype=acc)[None, None, :]
        if dt_softplus:
            v = softplus(v)
        return np.clip(v, dt_limit[0], dt_limit[1])

    if pad == "naive":
        v = process(np.pad(dt, ((0, 0), (0, padl), (0, 0))))
    elif pad == "kernel":
        v = np.pad(process(dt), ((0, 0), (0, padl), (0, 0)))
    else:
        raise ValueError(pad)
    dt_out = v.reshape(b, nc, chunk_size, H).transpose(0, 3, 1, 2)
    dA = dt_out * A[None, :, None, None]
    return np.cumsum(dA, axis=-1), np.ascontiguousarray(dt_out)


# ---------------------------------------------------------------------------
# seq_idx helpers (the seq_idx rules of reference kernels/chunk_state_fwd.py:239-269,
# kernels/state_passing_fwd.py:208-225, kernels/chunk_scan_fwd.py:294-322)
# ---------------------------------------------------------------------------

def _pad_seq(seq_idx, nc, chunk_size):
    """Pad seq_idx with -1 to nc*Q (chunk_state_fwd.py:231-232)."""
    seq_idx = np.asarray(seq_idx)
    L = seq_idx.shape[1]
    return np.pad(seq_idx, ((0, 0), (0, nc * chunk_size - L)), constant_values=-1)


def _chunk_end_seq(seq_idx, nc, chunk_size):
    """seq_idx at the last valid position of each chunk (chunk_state_fwd.py:256-259)."""
    L = seq_idx.shape[1]
    ends = np.minimum(np.arange(1, nc + 1) * chunk_size, L) - 1
    return np.asarray(seq_idx)[:, ends]  # (b, nc)


# ---------------------------------------------------------------------------
# 2. chunk_state  (ssd_naive.py:77-128; seq_idx: chunk_state_fwd.py:245-269)
# ---------------------------------------------------------------------------

def chunk_state(B, x, dt, dA_cumsum, seq_idx=None, decay_clamp=False, acc=np.float64):
    """states[b,c,h,p,n] = sum_l exp(dA[-1]-dA[l]) * dt[l] * x[l,p] * B[l,n].

    ``decay_clamp`` clamps the exponent at 0 as the reference's chunk_state
    kernel does (kernels/chunk_state_fwd.py:251); its naive path
    (ops/ssd_naive.py:113-115) does not.  The two differ only where dA_cumsum
    increases within a chunk (dt' * A > 0 somewhere).
    """
    x = np.asarray(x, dtype=acc)
    B = np.asarray(B, dtype=acc)
    dt = np.asarray(dt, dtype=acc)
    dA_cumsum = np.asarray(dA_cumsum, dtype=acc)
    b, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    _, _, nc, Q = dt.shape
    hpg = H // G
    T = nc * Q
    if L < T:
        x = np.pad(x, ((0, 0), (0, T - L), (0, 0), (0, 0)))
        B = np.pad(B, ((0, 0), (0, T - L), (0, 0), (0, 0)))
    expo = dA_cumsum[:, :, :, -1:] - dA_cumsum
    decay = np.exp(np.minimum(expo, 0.0) if decay_clamp else expo)   # (b,H,nc,Q)
    w = decay * dt
    if seq_idx is not None:
        last = _chunk_end_seq(seq_idx, nc, Q)                      # (b,nc)
        sp = _pad_seq(seq_idx, nc, Q).reshape(b, nc, Q)
        keep = (last[:, :, None] >= 0) & (sp == last[:, :, None])  # (b,nc,Q)
        w = np.where(keep[:, None, :, :], w, 0.0)
    # einsum "bclhn,bhcl,bhcl,bclhp->bchpn" as grouped batched matmuls
    xc = x.reshape(b, nc, Q, G, hpg, P)
    Bc = B.reshape(b, nc, Q, G, N)
    wt = w.transpose(0, 2, 3, 1).reshape(b, nc, Q, G, hpg)       # (b,nc,Q,G,hpg)
    xw = xc * wt[..., None]                                        # (b,nc,Q,G,hpg,P)
    lhs = xw.transpose(0, 1, 3, 4, 5, 2)                           # (b,nc,G,hpg,P,Q)
    rhs = Bc.transpose(0, 1, 3, 2, 4)[:, :, :, None]               # (b,nc,G,1,Q,N)
    st = np.matmul(lhs, rhs)                                       # (b,nc,G,hpg,P,N)
    return st.reshape(b, nc, H, P, N)


# ---------------------------------------------------------------------------
# 3. state_passing
#    pairwise:   ssd_naive.py:135-182
#    sequential: tests/test_state_passing_and_bmm.py:92-138 (seq_idx resets,
#                prev seq = 0 for chunk 0; kernels/state_passing_fwd.py:208-225)
# ---------------------------------------------------------------------------

def state_passing(states, dA_chunk_cumsum, initial_states=None, seq_idx=None,
                  chunk_size=None, method=None, acc=np.float64):
    """Returns (out (b,nc,H,D) = state entering each chunk, final (b,H,D))."""
    states = np.asarray(states, dtype=acc)
    dAc = np.asarray(dA_chunk_cumsum, dtype=acc)
    b, nc, H, D = states.shape
    if method is None:
        method = "sequential" if seq_idx is not None else "pairwise"
    init = (np.zeros((b, H, D), acc) if initial_states is None
            else np.asarray(initial_states, dtype=acc))
    if method == "pairwise":
        if seq_idx is not None:
            raise ValueError("the pairwise (ssd_naive) form has no seq_idx")
        st = np.concatenate([init[:, None], states], axis=1)       # (b,nc+1,H,D)
        cs = np.cumsum(np.pad(dAc, ((0, 0), (0, 0), (1, 0))), axis=-1)  # (b,H,nc+1)
        n1 = nc + 1
        expo = cs[:, :, :, None] - cs[:, :, None, :]
        expo = np.where(np.tril(np.ones((n1, n1), bool))[None, None], expo, -np.inf)
        decay = np.exp(expo)                                       # (b,H,z,c)
        # einsum "bhzc,bchd->bzhd"
        out = np.matmul(decay, st.transpose(0, 2, 1, 3))           # (b,H,z,D)
        out = out.transpose(0, 2, 1, 3)
        return out[:, :-1], out[:, -1]
    if method != "sequential":
        raise ValueError(method)
    scale_mask = np.ones((b, nc), acc)
    if seq_idx is not None:
        ends = _chunk_end_seq(seq_idx, nc, chunk_size)
        prev = np.concatenate([np.zeros((b, 1), ends.dtype), ends[:, :-1]], axis=1)
        scale_mask = (ends == prev).astype(acc)
    run = init.copy()
    outs = []
    for c in range(nc):
        outs.append(run.copy())
        scale = np.exp(dAc[:, :, c]) * scale_mask[:, c][:, None]
        run = scale[:, :, None] * run + states[:, c]
    return np.stack(outs, axis=1), run


# ---------------------------------------------------------------------------
# 4. bmm_chunk  (ssd_naive.py:189-216; masks: kernels/bmm_chunk_fwd.py:348-372)
# ---------------------------------------------------------------------------

def bmm_chunk(C, B, chunk_size, seq_idx=None, causal=False, round_fn=identity,
              acc=np.float64):
    """CB[b,c,g,l,s] = sum_n C[b,cQ+l,g,n] * B[b,cQ+s,g,n]."""
    C = np.asarray(C, dtype=acc)
    B = np.asarray(B, dtype=acc)
    b, L, G, N = C.shape
    Q = chunk_size
    nc = -(-L // Q)
    T = nc * Q
    if L < T:
        C = np.pad(C, ((0, 0), (0, T - L), (0, 0), (0, 0)))
        B = np.pad(B, ((0, 0), (0, T - L), (0, 0), (0, 0)))
    Cc = C.reshape(b, nc, Q, G, N).transpose(0, 1, 3, 2, 4)
    Bc = B.reshape(b, nc, Q, G, N).transpose(0, 1, 3, 4, 2)
    CB = round_fn(np.matmul(Cc, Bc))
    if causal:
        CB = np.where(np.tril(np.ones((Q, Q), bool))[None, None, None], CB, 0.0)
    if seq_idx is not None:
        sp = _pad_seq(seq_idx, nc, Q).reshape(b, nc, Q)
        m = sp[:, :, :, None] == sp[:, :, None, :]
        CB = np.where(m[:, :, None], CB, 0.0)
    return CB


# ---------------------------------------------------------------------------
# 5. chunk_scan  (ssd_naive.py:223-318; seq_idx: chunk_scan_fwd.py:294-322)
# ---------------------------------------------------------------------------

def chunk_scan(CB, x, dt, dA_cumsum, C, prev_states, D=None, z=None,
               seq_idx=None, round_fn=identity, acc=np.float64):
    """Returns (out (b,L,H,P), out_x or None).

    prev_states is rounded to C's dtype (``round_fn``) before use, and the
    C @ states product is rounded to that dtype before the exp(dA) multiply,
    as the naive path does.  With seq_idx, rows whose sequence differs from the
    one that ended the previous chunk get no inter-chunk term; CB is used as
    given (the kernel wrapper expects it masked upstream).
    """
    CB = np.asarray(CB, dtype=acc)
    x = np.asarray(x, dtype=acc)
    dt = np.asarray(dt, dtype=acc)
    dA = np.asarray(dA_cumsum, dtype=acc)
    C = np.asarray(C, dtype=acc)
    b, L, H, P = x.shape
    G, N = C.shape[2], C.shape[3]
    _, _, nc, Q = dt.shape
    hpg = H // G
    T = nc * Q
    xp = np.pad(x, ((0, 0), (0, T - L), (0, 0), (0, 0))) if L < T else x
    Cp = np.pad(C, ((0, 0), (0, T - L), (0, 0), (0, 0))) if L < T else C
    # Part A: intra-chunk, decay masked before exp (ssd_naive.py:263-282)
    expo = dA[:, :, :, :, None] - dA[:, :, :, None, :]            # (b,H,nc,l,s)
    expo = np.where(np.tril(np.ones((Q, Q), bool)), expo, -np.inf)
    decay = np.exp(expo).transpose(0, 2, 1, 3, 4)                 # (b,nc,H,l,s)
    CBh = np.repeat(CB, hpg, axis=2)                               # (b,nc,H,l,s)
    dtt = dt.transpose(0, 2, 1, 3)                                 # (b,nc,H,s)
    scores = CBh * decay * dtt[:, :, :, None, :]
    xc = xp.reshape(b, nc, Q, H, P).transpose(0, 1, 3, 2, 4)       # (b,nc,H,s,P)
    out_intra = np.matmul(scores, xc)                              # (b,nc,H,l,P)
    # Part B: inter-chunk (ssd_naive.py:285-297)
    ps = round_fn(np.asarray(prev_states, dtype=acc))              # (b,nc,H,P,N)
    Cc = Cp.reshape(b, nc, Q, G, N).transpose(0, 1, 3, 2, 4)       # (b,nc,G,l,N)
    Ch = np.repeat(Cc, hpg, axis=2)                                # (b,nc,H,l,N)
    inter = round_fn(np.matmul(Ch, ps.transpose(0, 1, 2, 4, 3)))   # (b,nc,H,l,P)
    sdec = np.exp(dA).transpose(0, 2, 1, 3)                        # (b,nc,H,l)
    if seq_idx is not None:
        sp = _pad_seq(seq_idx, nc, Q)
        prev_pos = np.arange(nc) * Q - 1
        seq_prev = np.where(prev_pos >= 0, sp[:, np.maximum(prev_pos, 0)], 0)
        same = sp.reshape(b, nc, Q) == seq_prev[:, :, None]        # (b,nc,Q)
        sdec = np.where(same[:, :, None, :], sdec, 0.0)
    out = out_intra + inter * sdec[..., None]
    out = out.transpose(0, 1, 3, 2, 4).reshape(b, T, H, P)[:, :L]
    if D is not None:
        D = np.asarray(D, dtype=acc)
        Db = D[None, None, :, None] if D.ndim == 1 else D[None, None]
        out = out + x * Db
    out_x = None
    if z is not None:
        out_x = out
        # jax.nn.silu(z) keeps z's dtype (ssd_naive.py:316)
        out = out * round_fn(silu(np.asarray(z, dtype=acc)))
    return out, out_x


# ---------------------------------------------------------------------------
# 6. chunk_state_varlen  (kernels/chunk_state_fwd.py:448-597;
#                         tests/test_chunk_scan_and_varlen.py:504-589)
# ---------------------------------------------------------------------------

def chunk_state_varlen(B, x, dt, dA_cumsum, cu_seqlens, chunk_states,
                       acc=np.float64):
    """Final state of each packed sequence, (nseq, H, P, N)."""
    B = np.asarray(B, dtype=acc)
    x = np.asarray(x, dtype=acc)
    dt = np.asarray(dt, dtype=acc)
    dA = np.asarray(dA_cumsum, dtype=acc)
    cs = np.asarray(chunk_states, dtype=acc)
    Ltot, H, P = x.shape
    _, nc, Q = dt.shape
    G, N = B.shape[1], B.shape[2]
    hpg = H // G
    cu = [int(v) for v in np.asarray(cu_seqlens)]
    res = []
    for s in range(len(cu) - 1):
        start, end = cu[s], cu[s + 1]
        lc = (end - 1) // Q
        c0 = lc * Q
        lim = end - c0
        sin = max(start - c0, 0)
        dAl = dA[:, lc]                                            # (H,Q)
        last = dAl[:, lim - 1]                                     # (H,)
        w = np.exp(np.minimum(last[:, None] - dAl, 0.0)) * dt[:, lc]
        pos = np.arange(Q)
        w = np.where(((pos >= sin) & (pos < lim))[None], w, 0.0)
        xs = np.zeros((Q, H, P), acc)
        Bs = np.zeros((Q, G, N), acc)
        n_avail = min(lim, Ltot - c0)
        xs[:n_avail] = x[c0:c0 + n_avail]
        Bs[:n_avail] = B[c0:c0 + n_avail]
        st = np.empty((H, P, N), acc)
        for h in range(H):
            st[h] = (xs[:, h, :] * w[h][:, None]).T @ Bs[:, h // hpg, :]
        if start < c0:
            st = st + cs[lc] * np.exp(last)[:, None, None]
        res.append(st)
    return np.stack(res, axis=0)


# ---------------------------------------------------------------------------
# Combined forward  (kernels/ssd_combined.py:46-203; naive ssd_naive.py:325-397)
# ---------------------------------------------------------------------------

def ssd_combined(x, dt, A, B, C, chunk_size, D=None, z=None, dt_bias=None,
                 initial_states=None, seq_idx=None, cu_seqlens=None,
                 dt_softplus=False, dt_limit=(0.0, INF),
                 return_final_states=False, return_varlen_states=False,
                 io_dtype="f32", pad="kernel", decay_clamp=False, acc=np.float64,
                 passed_jitter=0.0, jitter_seed=0):
    """The five-stage SSD forward with the reference's return arity.

    ``io_dtype`` names the dtype of x/B/C ('f32' or 'bf16'); the inputs must
    already hold values of that dtype.  It selects the rounding applied where
    the reference casts to C.dtype.  ``decay_clamp``: see chunk_state.
    ``passed_jitter`` (tests only) multiplies the passed states by
    1 + passed_jitter * N(0, 1) (seed ``jitter_seed``) before their rounding to
    C.dtype: with a jitter far below any fp32 summation-order difference, the
    change it causes measures how far one rounding flip at that point (which
    the reference makes, kernels/ssd_combined.py:140) moves the results.
    """
    rf = round_fn_for(io_dtype)
    b, L, H, P = np.shape(x)
    G, N = np.shape(B)[2], np.shape(B)[3]
    if not return_varlen_states:
        cu_seqlens = None
    dA, dto = chunk_cumsum(dt, A, chunk_size, dt_bias, dt_softplus, dt_limit,
                           pad=pad, acc=acc)
    st = chunk_state(B, x, dto, dA, seq_idx=seq_idx, decay_clamp=decay_clamp, acc=acc)
    nc = st.shape[1]
    init = None if initial_states is None else np.asarray(
        initial_states, dtype=acc).reshape(b, H, P * N)
    sp, fin = state_passing(st.reshape(b, nc, H, P * N), dA[:, :, :, -1],
                            initial_states=init, seq_idx=seq_idx,
                            chunk_size=chunk_size, acc=acc)
    sp = sp.reshape(b, nc, H, P, N)
    if passed_jitter:
        sp = sp * (1.0 + passed_jitter * np.random.default_rng(jitter_seed).standard_normal(sp.shape))
    sp = rf(sp)                                  # out_dtype = C.dtype
    fin = fin.reshape(b, H, P, N)
    CB = bmm_chunk(C, B, chunk_size, seq_idx=seq_idx, round_fn=rf, acc=acc)
    out, _ = chunk_scan(CB, x, dto, dA, C, sp, D=D, z=z, seq_idx=seq_idx,
                        round_fn=rf, acc=acc)
    varlen = None
    if cu_seqlens is not None:
        if b != 1:
            raise ValueError("cu_seqlens for varlen states needs batch == 1")
        varlen = chunk_state_varlen(np.asarray(B)[0], np.asarray(x)[0], dto[0],
                                    dA[0], cu_seqlens, sp[0], acc=acc)
    if not return_varlen_states:
        return (out, fin) if return_final_states else out
    return (out, fin, varlen) if return_final_states else (out, varlen)


# ---------------------------------------------------------------------------
# Independent formulation: token-by-token recurrence
# (the identity the reference's prefill-vs-step test relies on,
#  tests/test_mamba2_vs_torch.py:312-408)
# ---------------------------------------------------------------------------

def ssd_sequential(x, dt, A, B, C, D=None, z=None, dt_bias=None,
                   initial_states=None, seq_idx=None, dt_softplus=False,
                   dt_limit=(0.0, INF), acc=np.float64):
    """h_t = exp(dt'_t A) h_{t-1} + dt'_t x_t B_t^T ; y_t = h_t C_t + D x_t.

    With seq_idx the state restarts at zero whenever seq_idx[t] differs from
    seq_idx[t-1] (seq_idx[-1] := 0, the id the initial state belongs to).
    Returns (y (b,L,H,P), final state (b,H,P,N)).
    """
    x = np.asarray(x, dtype=acc)
    dt = np.asarray(dt, dtype=acc)
    A = np.asarray(A, dtype=acc)
    B = np.asarray(B, dtype=acc)
    C = np.asarray(C, dtype=acc)
    b, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    if dt_bias is not None:
        dt = dt + np.asarray(dt_bias, dtype=acc)[None, None]
    if dt_softplus:
        dt = softplus(dt)
    dt = np.clip(dt, dt_limit[0], dt_limit[1])
    h = (np.zeros((b, H, P, N), acc) if initial_states is None
         else np.asarray(initial_states, dtype=acc).copy())
    Bh = np.repeat(B, hpg, axis=2)
    Ch = np.repeat(C, hpg, axis=2)
    ys = np.empty((b, L, H, P), acc)
    prev = np.zeros(b, dtype=np.int64)
    for t in range(L):
        if seq_idx is not None:
            cur = np.asarray(seq_idx)[:, t]
            h = h * (cur == prev)[:, None, None, None]
            prev = cur
        da = np.exp(dt[:, t] * A[None])                             # (b,H)
        h = (h * da[:, :, None, None]
             + (dt[:, t][:, :, None, None] * x[:, t][:, :, :, None]
                * Bh[:, t][:, :, None, :]))
        ys[:, t] = np.einsum("bhpn,bhn->bhp", h, Ch[:, t])
    if D is not None:
        D = np.asarray(D, dtype=acc)
        ys = ys + x * (D[None, None, :, None] if D.ndim == 1 else D[None, None])
    if z is not None:
        ys = ys * silu(np.asarray(z, dtype=acc))
    return ys, h


# ---------------------------------------------------------------------------
# Decode step  (ops/selective_state_update.py:68-123)
# ---------------------------------------------------------------------------

def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
                           dt_softplus=False, round_fn=identity, acc=np.float64):
    """Returns (new_state (b,H,P,N), out (b,H,P)); no dt_limit clamp.

    ``round_fn`` rounds silu(z) to z's dtype, as jax.nn.silu does (:121).
    """
    state = np.asarray(state, dtype=acc)
    x = np.asarray(x, dtype=acc)
    dt = np.asarray(dt, dtype=acc)
    A = np.asarray(A, dtype=acc)
    B = np.asarray(B, dtype=acc)
    C = np.asarray(C, dtype=acc)
    b, H, P, N = state.shape
    G = B.shape[1]
    hpg = H // G
    if dt_bias is not None:
        dt = dt + np.asarray(dt_bias, dtype=acc)
    if dt_softplus:
        dt = softplus(dt)
    if dt.ndim == 2:
        dt = dt[:, :, None]
    Bh = np.repeat(B, hpg, axis=1)
    Ch = np.repeat(C, hpg, axis=1)
    if A.ndim == 1:
        dA = np.exp(dt[:, :, :, None] * A[None, :, None, None])
    else:
        dA = np.exp(dt[:, :, :, None] * A[None])
    dBx = dt[:, :, :, None] * Bh[:, :, None, :] * x[:, :, :, None]
    new = state * dA + dBx
    out = np.sum(new * Ch[:, :, None, :], axis=-1)
    if D is not None:
        D = np.asarray(D, dtype=acc)
        out = out + (D[None, :, None] if D.ndim == 1 else D[None]) * x
    if z is not None:
        out = out * round_fn(silu(np.asarray(z, dtype=acc)))
    return new, out


def rel_err(got, want):
    """max |got - want| / rms(want): the BASELINE parity measure."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    rms = math.sqrt(float(np.mean(want * want))) or 1.0
    return float(np.max(np.abs(got - want))) / rms

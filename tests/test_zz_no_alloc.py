"""m2_ssd_combined_noalloc (the combined forward over the library's static
scratch, for callers that cannot allocate) against m2_ssd_combined (the same
kernels over a caller workspace), both called through the C ABI: identical
outputs, bit for bit, on consecutive calls whose sizes shrink (the scratch
keeps the previous call's contents), and the size limit enforced.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import announce
from mamba2_jax import _lib as L
from mamba2_jax import configs


def _args(t, chunk_size, dtype, fin=None, vs=None, nseq=0):
    """SsdCombinedArgs for the tensors in t (laid out as the Python wrapper
    passes them) with the outputs given."""
    b, Lq, H, P = t["x"].shape
    G, N = t["B"].shape[2], t["B"].shape[3]
    return L.SsdCombinedArgs(
        x=L.ptr(t["x"]), dt=L.ptr(t["dt"]), A=L.ptr(t["A"]), B=L.ptr(t["B"]), C=L.ptr(t["C"]),
        D=L.ptr(t.get("D")), z=L.ptr(t.get("z")), dt_bias=L.ptr(t.get("dt_bias")),
        initial_states=L.ptr(t.get("init")), seq_idx=L.ptr(t.get("seq")),
        cu_seqlens=L.ptr(t.get("cu")), out=L.ptr(t["out"]), final_states=L.ptr(fin),
        varlen_states=L.ptr(vs), batch=b, seqlen=Lq, nheads=H, headdim=P, ngroups=G, dstate=N,
        chunk_size=chunk_size, nseq=nseq, dtype=dtype, dt_dtype=L.dtype_code(t["dt"], "dt"),
        D_has_hdim=int(t.get("D") is not None and t["D"].dim() == 2), dt_softplus=1,
        dt_min=0.0, dt_max=float("inf"), stage_events=None)


def _inputs(rng, b, Lq, H, G, P, N, io, extras=False):
    dt = torch.bfloat16 if io == "bf16" else torch.float32
    g = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).cuda()
    t = {"x": g(b, Lq, H, P).to(dt), "dt": g(b, Lq, H).to(dt),
         "A": -torch.exp(torch.from_numpy(rng.uniform(0, np.log(16), H).astype(np.float32))).cuda(),
         "B": (g(b, Lq, G, N) / np.sqrt(N)).to(dt), "C": (g(b, Lq, G, N) / np.sqrt(N)).to(dt),
         "D": torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).cuda(),
         "dt_bias": torch.from_numpy(rng.uniform(-5, -2, H).astype(np.float32)).cuda()}
    if extras:
        t["D"] = torch.from_numpy(rng.uniform(0.5, 1.5, (H, P)).astype(np.float32)).cuda()
        t["z"] = g(b, Lq, H, P).to(dt)
        t["init"] = 0.1 * g(b, H, P, N)
        lens = [Lq // 3, Lq - Lq // 3]
        t["seq"] = torch.from_numpy(np.repeat(np.arange(2), lens).astype(np.int32)[None].repeat(b, 0)).cuda()
    t["out"] = torch.empty((b, Lq, H, P), dtype=torch.float32, device="cuda")
    return t


def _run_both(t, chunk_size, io):
    """(out, final) from m2_ssd_combined (torch workspace) and from
    m2_ssd_combined_noalloc; the noalloc call runs second, with its outputs
    pre-filled with NaN so that every element must be written."""
    lib = L.load_library()
    code = L.M2_BF16 if io == "bf16" else L.M2_F32
    b, Lq, H, P = t["x"].shape
    N = t["B"].shape[3]
    fin_w = torch.empty((b, H, P, N), dtype=torch.float32, device="cuda")
    a = _args(t, chunk_size, code, fin=fin_w)
    need = lib.m2_ssd_combined_workspace_size(ctypes.byref(a))
    assert 0 < need <= L.NOALLOC_SCRATCH_BYTES, need
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    a.workspace, a.workspace_bytes = ws.data_ptr(), need
    stream = torch.cuda.current_stream().cuda_stream
    L.call("m2_ssd_combined", a, stream)
    torch.cuda.synchronize()
    out_w = t["out"].clone()
    t["out"].fill_(float("nan"))
    fin_n = torch.full_like(fin_w, float("nan"))
    an = _args(t, chunk_size, code, fin=fin_n)      # workspace fields left NULL / 0
    L.call("m2_ssd_combined_noalloc", an, stream)
    torch.cuda.synchronize()
    return (out_w, fin_w), (t["out"], fin_n)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point():
    rng = np.random.default_rng(2024)
    cases = [
        # (b, L, H, G, P, N, chunk, io, extras): shrinking sizes, so every call
        # after the first finds the scratch holding a larger previous call's data
        (1, 4096, 128, 8, 64, 128, 128, "bf16", False),     # the nemotron-h-8b layer (fused kernels)
        (2, 1000, 16, 2, 64, 128, 128, "bf16", True),       # ragged L, init, z, D per head dim, seq_idx
        (1, 520, 8, 1, 64, 64, 256, "f32", False),          # float32: the staged kernels
    ]
    for (b, Lq, H, G, P, N, Q, io, ex) in cases:
        announce("noalloc vs workspace", b, Lq, H, G, P, N, Q, io, ex)
        t = _inputs(rng, b, Lq, H, G, P, N, io, ex)
        (ow, fw), (on, fn) = _run_both(t, Q, io)
        assert torch.equal(ow, on), "outputs differ"
        assert torch.equal(fw, fn), "final states differ"


@pytest.mark.gpu
def test_noalloc_rejects_oversized_problem():
    """A problem whose workspace exceeds the static scratch is refused with
    M2_ERR_WORKSPACE before anything runs (the nemotron-h-47b shape of config
    c3 needs ~570 MB)."""
    cfg = configs.CONFIGS["c3"]
    t = {k: torch.empty(1, device="cuda") for k in ("x", "dt", "A", "B", "C", "out")}
    a = L.SsdCombinedArgs(x=L.ptr(t["x"]), dt=L.ptr(t["dt"]), A=L.ptr(t["A"]), B=L.ptr(t["B"]),
                          C=L.ptr(t["C"]), out=L.ptr(t["out"]), batch=1, seqlen=cfg.seqlen,
                          nheads=cfg.nheads, headdim=cfg.headdim, ngroups=cfg.ngroups,
                          dstate=cfg.dstate, chunk_size=cfg.chunk_size, dtype=L.M2_BF16,
                          dt_dtype=L.M2_BF16, dt_softplus=1, dt_max=float("inf"))
    lib = L.load_library()
    assert lib.m2_ssd_combined_workspace_size(ctypes.byref(a)) > L.NOALLOC_SCRATCH_BYTES
    with pytest.raises(L.M2Error) as e:
        L.call("m2_ssd_combined_noalloc", a, torch.cuda.current_stream().cuda_stream)
    assert e.value.code == -4 and "static scratch" in str(e.value)


@pytest.mark.gpu
def test_noalloc_under_graph_capture():
    """m2_ssd_combined_noalloc captured in a HIP graph after
    m2_ssd_combined_noalloc_prepare (the first call on a device looks the
    scratch up, which a capturing stream must not see): every replay, with an
    eager noalloc call on other inputs between replays (it overwrites the
    shared scratch), equals the workspace entry point bit for bit."""
    announce("noalloc under graph capture")
    lib = L.load_library()
    assert lib.m2_ssd_combined_noalloc_prepare() == 0
    rng = np.random.default_rng(77)
    t = _inputs(rng, 1, 1000, 16, 2, 64, 128, "bf16", True)
    (ow, fw), _ = _run_both(t, 128, "bf16")
    other = _inputs(rng, 1, 700, 8, 1, 64, 64, "bf16", False)
    out = torch.full_like(ow, float("nan"))
    fin = torch.full_like(fw, float("nan"))
    an = _args(dict(t, out=out), 128, L.M2_BF16, fin=fin)
    ao = _args(other, 128, L.M2_BF16)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        L.call("m2_ssd_combined_noalloc", an, torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        L.call("m2_ssd_combined_noalloc", ao, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        fin.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ow), f"replay {r}: outputs differ"
        assert torch.equal(fin, fw), f"replay {r}: final states differ"

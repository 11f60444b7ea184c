"""The C-ABI boundary, checked without a GPU.

* libm2ssd.so loads and exports every function include/m2ssd.h declares;
* the ctypes structs in mamba2_jax._lib match the header's layout (gcc
  compiles a probe against the header and prints sizeof / offsetof);
* host-side argument validation rejects bad calls before any GPU work.
"""

import ctypes
import os
import re
import subprocess

import pytest
import torch

from mamba2_jax import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "m2ssd.h")

STRUCT_NAMES = {
    "ChunkCumsumArgs": "m2_chunk_cumsum_args",
    "ChunkStateArgs": "m2_chunk_state_args",
    "StatePassingArgs": "m2_state_passing_args",
    "BmmChunkArgs": "m2_bmm_chunk_args",
    "ChunkScanArgs": "m2_chunk_scan_args",
    "ChunkStateVarlenArgs": "m2_chunk_state_varlen_args",
    "SsdCombinedArgs": "m2_ssd_combined_args",
    "SsuArgs": "m2_ssu_args",
    "ConvOut": "m2_conv_out",
    "CausalConv1dArgs": "m2_causal_conv1d_args",
    "CausalConv1dUpdateArgs": "m2_causal_conv1d_update_args",
    "RmsNormGatedArgs": "m2_rms_norm_gated_args",
    "SkinnyGemmArgs": "m2_skinny_gemm_args",
    "SkinnyGemmNormArgs": "m2_skinny_gemm_norm_args",
}


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(m2_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_function():
    lib = L.load_library()
    names = declared_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), f"{n} declared in m2ssd.h but not exported"
    assert set(names) == set(L.ENTRY_POINTS) | set(L.OTHER_SYMBOLS)
    assert lib.m2_abi_version() == L.ABI_VERSION


def test_nm_shows_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for n in declared_functions():
        assert n in syms


def test_struct_layout_matches_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"',
             "int main(void) {"]
    for py, c in STRUCT_NAMES.items():
        st = getattr(L, py)
        lines.append(f'printf("{py} size %zu\\n", sizeof({c}));')
        for fname, _ in st._fields_:
            lines.append(f'printf("{py}.{fname} %zu\\n", offsetof({c}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run(
        [str(exe)], capture_output=True, text=True, check=True).stdout.splitlines())
    for py in STRUCT_NAMES:
        st = getattr(L, py)
        assert int(got[f"{py} size"]) == ctypes.sizeof(st), py
        for fname, _ in st._fields_:
            assert int(got[f"{py}.{fname}"]) == getattr(st, fname).offset, f"{py}.{fname}"


def test_noalloc_scratch_size_matches_header():
    src = open(HEADER).read()
    m = re.search(r"#define M2_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", src)
    assert m and int(m.group(1)) << int(m.group(2)) == L.NOALLOC_SCRATCH_BYTES


def test_noalloc_rejects_oversized_problem_without_gpu():
    """The size check runs on the host before any device call: the c3 shape
    (~570 MB of workspace) is refused with M2_ERR_WORKSPACE."""
    lib = L.load_library()
    a = L.SsdCombinedArgs(batch=1, seqlen=8192, nheads=256, headdim=64, ngroups=8, dstate=256,
                          chunk_size=128, dtype=L.M2_BF16, dt_dtype=L.M2_BF16, x=16, dt=16, A=16,
                          B=16, C=16, out=16)
    assert lib.m2_ssd_combined_workspace_size(ctypes.byref(a)) > L.NOALLOC_SCRATCH_BYTES
    assert lib.m2_ssd_combined_noalloc(ctypes.byref(a), None) == -4
    assert b"static scratch" in lib.m2_last_error()


def test_null_args_are_rejected_without_gpu():
    lib = L.load_library()
    for name, st in L.ENTRY_POINTS.items():
        rc = getattr(lib, name)(None, None)
        assert rc == -1, name
        assert b"NULL" in lib.m2_last_error()


def test_invalid_sizes_are_rejected_without_gpu():
    lib = L.load_library()
    a = L.ChunkStateArgs(batch=1, seqlen=128, nheads=6, headdim=64, ngroups=4, dstate=64,
                         chunk_size=64, dtype=L.M2_BF16, x=16, B=16, dt=16, dA_cumsum=16, states=16)
    assert lib.m2_chunk_state(ctypes.byref(a), None) == -1          # 6 % 4 != 0
    assert b"multiple of ngroups" in lib.m2_last_error()
    a.ngroups, a.chunk_size = 2, 100
    assert lib.m2_chunk_state(ctypes.byref(a), None) == -2          # chunk 100 unsupported
    c = L.SsdCombinedArgs(batch=1, seqlen=128, nheads=4, headdim=64, ngroups=1, dstate=64,
                          chunk_size=64, dtype=L.M2_F32, x=16, dt=16, A=16, B=16, C=16, out=16)
    need = lib.m2_ssd_combined_workspace_size(ctypes.byref(c))
    assert need > 0
    c.workspace, c.workspace_bytes = 16, need - 1
    assert lib.m2_ssd_combined(ctypes.byref(c), None) == -4
    assert b"workspace" in lib.m2_last_error()


def test_python_wrappers_reject_cpu_tensors_and_bad_shapes():
    from mamba2_jax.kernels import chunk_cumsum_fwd, mamba_chunk_scan_combined_fwd
    dt = torch.zeros(1, 8, 2)
    with pytest.raises(ValueError, match="no CPU path"):
        chunk_cumsum_fwd(dt, torch.zeros(2), 4)
    with pytest.raises(AssertionError):
        # shape errors are AssertionError (like the reference's asserts) and ValueError
        from mamba2_jax._lib import require
        require(False, "x")
    with pytest.raises(ValueError):
        mamba_chunk_scan_combined_fwd(torch.zeros(1, 8, 2, 4), dt, torch.zeros(2),
                                      torch.zeros(1, 8, 1, 4), torch.zeros(1, 8, 1, 4), 4)


def test_dispatch_override_hook_without_gpu():
    """The testing hook m2_set_dispatch_override: unknown knobs and values are
    refused, the previous value comes back, the context manager restores it."""
    lib = L.load_library()
    assert lib.m2_set_dispatch_override(7, 1) == -1
    assert lib.m2_set_dispatch_override(0, 9) == -1
    assert lib.m2_set_dispatch_override(0, 2) == 0
    assert lib.m2_set_dispatch_override(0, 0) == 2
    with L.dispatch_override("states_split", "pair128"):
        with L.dispatch_override("f32_states", "staged"):
            assert lib.m2_set_dispatch_override(1, 2) == 2
        assert lib.m2_set_dispatch_override(0, 3) == 3
    assert lib.m2_set_dispatch_override(0, 0) == 0
    assert lib.m2_set_dispatch_override(1, 0) == 0
    assert lib.m2_set_dispatch_override(3, 66) == -1
    with L.dispatch_override("f32_scan", "per_head"):
        assert lib.m2_set_dispatch_override(3, 3) == 1
    assert lib.m2_set_dispatch_override(3, 0) == 0      # restored on exit
    with L.dispatch_override("f32_scan", "group16"):
        assert lib.m2_set_dispatch_override(3, 17) == 17
    assert lib.m2_set_dispatch_override(3, 0) == 0
    # the knob numbers of the header are the ones the Python table uses
    hdr = open(HEADER).read()
    defs = {n.lower(): int(v) for n, v in re.findall(r"#define M2_KNOB_(\w+)\s+(\d+)", hdr)}
    assert defs == {k: v[0] for k, v in L.KNOBS.items()}

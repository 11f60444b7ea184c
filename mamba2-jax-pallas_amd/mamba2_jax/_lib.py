"""ctypes binding of libm2ssd.so (include/m2ssd.h) and device-tensor plumbing.

The library is the product: there is no CPU path.  If it is missing, or a
tensor is not on a GPU, calls raise -- they never fall back to anything else.
torch provides device memory, the current stream and the HIP runtime that the
library shares (torch is imported first so that libm2ssd.so binds to the
libamdhip64 already loaded by torch).
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libm2ssd.so")

M2_F32 = 0
M2_BF16 = 1
ABI_VERSION = 5
# bytes of the static scratch m2_ssd_combined_noalloc runs in (M2_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 128 << 20

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class ChunkCumsumArgs(ctypes.Structure):
    _fields_ = [("dt", _c_p), ("A", _c_p), ("dt_bias", _c_p), ("dA_cumsum", _c_p),
                ("dt_out", _c_p), ("batch", _i64), ("seqlen", _i64), ("nheads", _i64),
                ("chunk_size", _i64), ("dt_dtype", _i32), ("dt_softplus", _i32),
                ("dt_min", _f32), ("dt_max", _f32)]


class ChunkStateArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("B", _c_p), ("dt", _c_p), ("dA_cumsum", _c_p),
                ("seq_idx", _c_p), ("states", _c_p), ("batch", _i64), ("seqlen", _i64),
                ("nheads", _i64), ("headdim", _i64), ("ngroups", _i64), ("dstate", _i64),
                ("chunk_size", _i64), ("dtype", _i32)]


class StatePassingArgs(ctypes.Structure):
    _fields_ = [("states", _c_p), ("dA_chunk_cumsum", _c_p), ("dA_stride_batch", _i64),
                ("dA_stride_head", _i64), ("dA_stride_chunk", _i64),
                ("initial_states", _c_p), ("seq_idx", _c_p), ("out", _c_p),
                ("final_states", _c_p), ("batch", _i64), ("nchunks", _i64),
                ("nheads", _i64), ("dim", _i64), ("seqlen", _i64), ("chunk_size", _i64),
                ("out_dtype", _i32)]


class BmmChunkArgs(ctypes.Structure):
    _fields_ = [("a", _c_p), ("b", _c_p), ("seq_idx", _c_p), ("out", _c_p),
                ("batch", _i64), ("seqlen", _i64), ("ngroups", _i64), ("k", _i64),
                ("chunk_size", _i64), ("dtype", _i32), ("out_dtype", _i32), ("causal", _i32)]


class ChunkScanArgs(ctypes.Structure):
    _fields_ = [("cb", _c_p), ("x", _c_p), ("dt", _c_p), ("dA_cumsum", _c_p), ("C", _c_p),
                ("states", _c_p), ("D", _c_p), ("z", _c_p), ("seq_idx", _c_p),
                ("out", _c_p), ("out_x", _c_p), ("batch", _i64), ("seqlen", _i64),
                ("nheads", _i64), ("headdim", _i64), ("ngroups", _i64), ("dstate", _i64),
                ("chunk_size", _i64), ("dtype", _i32), ("cb_dtype", _i32),
                ("states_dtype", _i32), ("D_has_hdim", _i32)]


class ChunkStateVarlenArgs(ctypes.Structure):
    _fields_ = [("B", _c_p), ("x", _c_p), ("dt", _c_p), ("dA_cumsum", _c_p),
                ("cu_seqlens", _c_p), ("chunk_states", _c_p), ("out", _c_p),
                ("seqlen", _i64), ("nseq", _i64), ("nheads", _i64), ("headdim", _i64),
                ("ngroups", _i64), ("dstate", _i64), ("nchunks", _i64), ("chunk_size", _i64),
                ("dtype", _i32), ("states_dtype", _i32)]


class SsdCombinedArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("dt", _c_p), ("A", _c_p), ("B", _c_p), ("C", _c_p),
                ("D", _c_p), ("z", _c_p), ("dt_bias", _c_p), ("initial_states", _c_p),
                ("seq_idx", _c_p), ("cu_seqlens", _c_p), ("out", _c_p),
                ("final_states", _c_p), ("varlen_states", _c_p), ("workspace", _c_p),
                ("workspace_bytes", ctypes.c_size_t), ("batch", _i64), ("seqlen", _i64),
                ("nheads", _i64), ("headdim", _i64), ("ngroups", _i64), ("dstate", _i64),
                ("chunk_size", _i64), ("nseq", _i64), ("dtype", _i32), ("dt_dtype", _i32),
                ("D_has_hdim", _i32), ("dt_softplus", _i32), ("dt_min", _f32),
                ("dt_max", _f32), ("stage_events", _c_p)]


class SsuArgs(ctypes.Structure):
    _fields_ = [("state", _c_p), ("x", _c_p), ("dt", _c_p), ("A", _c_p), ("B", _c_p),
                ("C", _c_p), ("D", _c_p), ("z", _c_p), ("dt_bias", _c_p), ("out", _c_p),
                ("batch", _i64), ("nheads", _i64), ("headdim", _i64), ("ngroups", _i64),
                ("dstate", _i64), ("dtype", _i32), ("dt_dtype", _i32),
                ("dt_has_hdim", _i32), ("A_full", _i32), ("D_has_hdim", _i32),
                ("dt_bias_has_hdim", _i32), ("dt_softplus", _i32), ("new_state", _c_p)]


class ConvOut(ctypes.Structure):
    _fields_ = [("ptr", _c_p), ("c_begin", _i64), ("stride_batch", _i64),
                ("stride_dim", _i64), ("stride_time", _i64)]


class CausalConv1dArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("x_stride_batch", _i64), ("x_stride_dim", _i64),
                ("x_stride_time", _i64), ("weight", _c_p), ("bias", _c_p), ("seq_idx", _c_p),
                ("out", ConvOut * 3), ("batch", _i64), ("dim", _i64), ("seqlen", _i64),
                ("width", _i64), ("nout", _i32), ("x_dtype", _i32), ("w_dtype", _i32),
                ("bias_dtype", _i32), ("out_dtype", _i32), ("silu", _i32)]


class CausalConv1dUpdateArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("x_stride_batch", _i64), ("conv_state", _c_p),
                ("new_state", _c_p), ("weight", _c_p), ("bias", _c_p), ("out", ConvOut * 3),
                ("batch", _i64), ("dim", _i64), ("width", _i64), ("nout", _i32),
                ("x_dtype", _i32), ("state_dtype", _i32), ("new_state_dtype", _i32),
                ("w_dtype", _i32), ("bias_dtype", _i32), ("out_dtype", _i32), ("silu", _i32)]


class RmsNormGatedArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("z", _c_p), ("weight", _c_p), ("out", _c_p),
                ("x_row_stride", _i64), ("z_row_stride", _i64), ("out_row_stride", _i64),
                ("rows", _i64), ("hidden", _i64), ("group_size", _i64), ("eps", _f32),
                ("x_dtype", _i32), ("z_dtype", _i32), ("w_dtype", _i32), ("out_dtype", _i32),
                ("norm_before_gate", _i32), ("residual", _c_p), ("residual_row_stride", _i64)]


class SkinnyGemmArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("w", _c_p), ("bias", _c_p), ("y", _c_p), ("M", _i64), ("N", _i64),
                ("K", _i64), ("ldx", _i64), ("ldw", _i64), ("ldy", _i64), ("x_dtype", _i32),
                ("w_dtype", _i32), ("bias_dtype", _i32), ("y_dtype", _i32)]


class SkinnyGemmNormArgs(ctypes.Structure):
    _fields_ = [("x", _c_p), ("z", _c_p), ("norm_weight", _c_p), ("x_row_stride", _i64),
                ("z_row_stride", _i64), ("group_size", _i64), ("eps", ctypes.c_float),
                ("x_dtype", _i32), ("z_dtype", _i32), ("norm_weight_dtype", _i32),
                ("norm_before_gate", _i32), ("w", _c_p), ("bias", _c_p), ("y", _c_p),
                ("residual", _c_p), ("M", _i64), ("N", _i64), ("K", _i64), ("ldw", _i64),
                ("ldy", _i64), ("residual_row_stride", _i64), ("w_dtype", _i32),
                ("bias_dtype", _i32), ("y_dtype", _i32), ("with_conv", _i32),
                ("conv_begin", _i64), ("conv", CausalConv1dUpdateArgs)]


# entry point name -> argument struct (every function declared in m2ssd.h)
ENTRY_POINTS = {
    "m2_chunk_cumsum": ChunkCumsumArgs,
    "m2_chunk_state": ChunkStateArgs,
    "m2_state_passing": StatePassingArgs,
    "m2_bmm_chunk": BmmChunkArgs,
    "m2_chunk_scan": ChunkScanArgs,
    "m2_chunk_state_varlen": ChunkStateVarlenArgs,
    "m2_ssd_combined": SsdCombinedArgs,
    "m2_ssd_combined_noalloc": SsdCombinedArgs,
    "m2_selective_state_update": SsuArgs,
    "m2_causal_conv1d": CausalConv1dArgs,
    "m2_causal_conv1d_update": CausalConv1dUpdateArgs,
    "m2_rms_norm_gated": RmsNormGatedArgs,
    "m2_skinny_gemm": SkinnyGemmArgs,
    "m2_skinny_gemm_norm": SkinnyGemmNormArgs,
}
OTHER_SYMBOLS = ("m2_ssd_combined_workspace_size", "m2_last_error", "m2_abi_version",
                 "m2_set_dispatch_override", "m2_ssd_combined_noalloc_prepare")

# testing hook m2_set_dispatch_override: knob name -> (M2_KNOB_*, {choice: value})
KNOBS = {
    "states_split": (0, {"halves": 1, "pair64": 2, "pair128": 3}),
    "f32_states": (1, {"fused": 1, "staged": 2}),
    "oneshot_heads": (2, {"1": 1}),
    "f32_scan": (3, {"per_head": 1, **{f"group{n}": n + 1 for n in range(1, 65)}}),
}


class M2Error(RuntimeError):
    """A non-zero return code from libm2ssd.so."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


class M2ShapeError(AssertionError, ValueError):
    """Bad shapes / arguments.  An AssertionError like the reference's asserts,
    and a ValueError."""


_lock = threading.Lock()
_lib = None


def load_library(path=LIB_PATH):
    """Load libm2ssd.so once and declare its functions."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise ImportError(
                f"{path} is missing: build the HIP library first "
                "(python mamba2-jax-pallas_amd/build.py or __graft_entry__.build())")
        lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        for name, st in ENTRY_POINTS.items():
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(st), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        lib.m2_ssd_combined_workspace_size.argtypes = [ctypes.POINTER(SsdCombinedArgs)]
        lib.m2_ssd_combined_workspace_size.restype = ctypes.c_size_t
        lib.m2_last_error.argtypes = []
        lib.m2_last_error.restype = ctypes.c_char_p
        lib.m2_abi_version.argtypes = []
        lib.m2_abi_version.restype = ctypes.c_int
        lib.m2_set_dispatch_override.argtypes = [ctypes.c_int, ctypes.c_int]
        lib.m2_set_dispatch_override.restype = ctypes.c_int
        lib.m2_ssd_combined_noalloc_prepare.argtypes = []
        lib.m2_ssd_combined_noalloc_prepare.restype = ctypes.c_int
        if lib.m2_abi_version() != ABI_VERSION:
            raise ImportError(f"{path}: ABI version {lib.m2_abi_version()} != {ABI_VERSION}")
        _lib = lib
        return lib


_fns = {}


def call(name, args, stream):
    """Call entry point `name` with a filled argument struct on `stream`."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load_library(), name)
    rc = fn(ctypes.byref(args), stream)
    if rc != 0:
        raise M2Error(name, rc, load_library().m2_last_error().decode(errors="replace"))


# Bumped on every override change: results cached against the library's
# shape-based choices (the combined forward's workspace size) include it.
_override_epoch = 0


@contextlib.contextmanager
def dispatch_override(knob, choice):
    """Testing hook: force one of the library's shape-based kernel choices
    (KNOBS) inside the block, process-wide; the automatic choice is restored
    after it.  A forced choice the shape cannot take is ignored by the library."""
    global _override_epoch
    lib = load_library()
    k, values = KNOBS[knob]
    prev = lib.m2_set_dispatch_override(k, values[choice])
    if prev < 0:
        raise M2Error("m2_set_dispatch_override", prev, lib.m2_last_error().decode())
    _override_epoch += 1
    try:
        yield
    finally:
        lib.m2_set_dispatch_override(k, prev)
        _override_epoch += 1


def override_epoch():
    return _override_epoch


# ---------------------------------------------------------------------------
# tensor plumbing
# ---------------------------------------------------------------------------

_DTYPE_CODE = {torch.float32: M2_F32, torch.bfloat16: M2_BF16}


def dtype_code(t, what):
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: dtype {t.dtype} is not supported (float32 or bfloat16)") from None


def torch_dtype(d):
    """Accept torch dtypes and common names ('float32', 'bfloat16', jnp-like objects)."""
    if d is None or isinstance(d, torch.dtype):
        return d
    name = getattr(d, "name", None) or getattr(d, "__name__", None) or str(d)
    name = name.replace("torch.", "").replace("jnp.", "")
    table = {"float32": torch.float32, "f32": torch.float32, "bfloat16": torch.bfloat16,
             "bf16": torch.bfloat16}
    if name not in table:
        raise TypeError(f"dtype {d!r} is not supported (float32 or bfloat16)")
    return table[name]


def require(cond, msg):
    """Raise M2ShapeError(msg) unless cond; msg may be a callable that builds
    the message (formatted only on failure)."""
    if not cond:
        raise M2ShapeError(msg() if callable(msg) else msg)


def device_of(*tensors):
    """The common GPU device of the given tensors (None entries ignored)."""
    first, idx = None, -1
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if not t.is_cuda:
            raise ValueError(
                f"tensor on {t.device}: the HIP kernels need GPU tensors (there is no CPU path)")
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise ValueError(f"tensors on different devices: {first.device} and {t.device}")
    if first is None:
        raise ValueError("no GPU tensor given")
    return first.device


def dev_contig(t, dtype=None):
    """Contiguous (and 16-byte aligned) version of t, optionally cast."""
    if t is None:
        return None
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def ptr(t):
    return 0 if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device):
    """The raw handle of `device`'s current stream."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream

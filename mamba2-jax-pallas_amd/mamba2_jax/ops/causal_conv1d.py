"""causal_conv1d / causal_conv1d_update on MI355X: the depthwise causal
convolution in front of the SSD (prefill) and its one-token update (decode),
as HIP kernels in libm2ssd.so (m2_causal_conv1d, m2_causal_conv1d_update).

Drop-in for reference ops/causal_conv1d.py:18-139: same names, arguments,
shapes and result dtypes (bf16 only when x, weight and bias are all bf16), the
same sequence-boundary mask (:142-193, which zeroes the last width - 1 inputs
before every sequence start for all outputs).  Differences, all documented:

* the result keeps the memory layout of x: a (batch, d, seqlen) view of a
  channels-last (batch, seqlen, d) buffer -- what ``xBC.transpose(1, 2)``
  gives in the Mamba2 layer -- comes back as the same kind of view, so the
  transpose back to (batch, seqlen, d) is free;
* ``split_sizes`` (keyword only, not in the reference) writes consecutive
  channel ranges of the result into separate tensors, e.g. x, B and C of an
  SSD layer in the contiguous layouts the SSD kernels read, with no copy;
* causal_conv1d_update returns a new conv state and leaves the caller's
  untouched, as the reference does; a decode loop that owns its state passes
  the keyword-only ``inplace=True`` to have it updated in place (when its dtype
  is the new state's), what JAX's buffer donation gives.
"""

from __future__ import annotations

import torch

from .. import _lib as L

_MAX_WIDTH = 8


def _result_dtype(*dts):
    dts = [d for d in dts if d is not None]
    return torch.bfloat16 if all(d == torch.bfloat16 for d in dts) else torch.float32


def _float_tensor(t, what):
    if t is None:
        return None
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return L.dev_contig(t)


def _weight(weight, dim, what="weight"):
    if weight.dim() == 3:
        L.require(weight.shape[1] == 1, f"{what} must be (d, width) or (d, 1, width)")
        weight = weight[:, 0, :]
    L.require(weight.dim() == 2 and weight.shape[0] == dim,
              f"{what}.shape={tuple(weight.shape)} does not match d={dim}")
    width = int(weight.shape[1])
    L.require(1 <= width <= _MAX_WIDTH, f"kernel width {width} is not in 1..{_MAX_WIDTH}")
    return _float_tensor(weight, what), width


def _splits(dim, split_sizes):
    if split_sizes is None:
        return [dim]
    sizes = [int(s) for s in split_sizes]
    L.require(1 <= len(sizes) <= 3 and all(s > 0 for s in sizes) and sum(sizes) == dim,
              f"split_sizes={sizes} must be 1..3 positive sizes summing to d={dim}")
    return sizes


def causal_conv1d(x, weight, bias=None, activation=None, seq_idx=None, *, split_sizes=None):
    """-> out (batch, d, seqlen), or a tuple of (batch, d_j, seqlen) parts with split_sizes.

    x (batch, d, seqlen) (any strides; unit channel stride or unit time stride
    are the fast layouts); weight (d, width) or (d, 1, width); bias (d,);
    activation "silu" or None (anything else: no activation, as the
    reference); seq_idx (batch, seqlen) integer.
    out[t] = silu?(sum_i weight[:, i] * xm[t - width + 1 + i] + bias).
    """
    dev = L.device_of(x, weight, bias, seq_idx)
    L.require(x.dim() == 3, "x must be (batch, d, seqlen)")
    batch, dim, seqlen = (int(v) for v in x.shape)
    L.require(batch > 0 and dim > 0 and seqlen > 0, f"x.shape={tuple(x.shape)} has an empty dim")
    w, width = _weight(weight, dim)
    if bias is not None:
        L.require(tuple(bias.shape) == (dim,), f"bias.shape={tuple(bias.shape)}")
    b_c = _float_tensor(bias, "bias")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if x.data_ptr() % 16 and x.stride(1) == 1:
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    elif x.data_ptr() % 16:
        x = x.contiguous()
    seq = None
    if seq_idx is not None:
        L.require(tuple(seq_idx.shape) == (batch, seqlen), f"seq_idx.shape={tuple(seq_idx.shape)}")
        seq = L.dev_contig(seq_idx, torch.int32)
    odt = _result_dtype(x.dtype, w.dtype, None if b_c is None else b_c.dtype)
    sizes = _splits(dim, split_sizes)
    # the result keeps x's layout: channels-last when x's channel stride is 1
    channels_last = x.stride(1) == 1 and x.stride(2) != 1
    parts, outs, c0 = [], (L.ConvOut * 3)(), 0
    for j, dj in enumerate(sizes):
        if channels_last:
            buf = torch.empty((batch, seqlen, dj), dtype=odt, device=dev)
            part = buf.transpose(1, 2)
        else:
            part = torch.empty((batch, dj, seqlen), dtype=odt, device=dev)
        outs[j] = L.ConvOut(L.ptr(part), c0, part.stride(0), part.stride(1), part.stride(2))
        parts.append(part)
        c0 += dj
    args = L.CausalConv1dArgs(
        x=L.ptr(x), x_stride_batch=x.stride(0), x_stride_dim=x.stride(1),
        x_stride_time=x.stride(2), weight=L.ptr(w), bias=L.ptr(b_c), seq_idx=L.ptr(seq),
        out=outs, batch=batch, dim=dim, seqlen=seqlen, width=width, nout=len(sizes),
        x_dtype=L.dtype_code(x, "x"), w_dtype=L.dtype_code(w, "weight"),
        bias_dtype=L.M2_F32 if b_c is None else L.dtype_code(b_c, "bias"),
        out_dtype=L.dtype_code(parts[0], "out"), silu=int(activation == "silu"))
    with torch.cuda.device(dev):
        L.call("m2_causal_conv1d", args, L.stream_of(dev))
    return parts[0] if split_sizes is None else tuple(parts)


def update_from_columns(conv_state, weight, bias=None, activation=None, *, x_dtype=torch.bfloat16,
                        split_sizes=None):
    """The arguments of an in-place decode conv update whose new inputs are
    produced by another kernel (the in-projection's epilogue, see
    ops.linear.linear_norm): -> (CausalConv1dUpdateArgs with x unset, out
    parts).  conv_state (batch, d, width) float32 contiguous."""
    dev = L.device_of(conv_state, weight, bias)
    L.require(conv_state.dim() == 3 and conv_state.dtype == torch.float32 and conv_state.is_contiguous(),
              "conv_state must be a contiguous float32 (batch, d, width) tensor")
    batch, dim, width = (int(v) for v in conv_state.shape)
    w, kw = _weight(weight, dim)
    L.require(kw == width, f"weight width {kw} != conv_state width {width}")
    if bias is not None:
        L.require(tuple(bias.shape) == (dim,), f"bias.shape={tuple(bias.shape)}")
    b_c = _float_tensor(bias, "bias")
    nsdt = _result_dtype(torch.float32, x_dtype)
    odt = _result_dtype(nsdt, w.dtype, None if b_c is None else b_c.dtype)
    sizes = _splits(dim, split_sizes)
    parts, outs, c0 = [], (L.ConvOut * 3)(), 0
    for j, dj in enumerate(sizes):
        part = torch.empty((batch, dj), dtype=odt, device=dev)
        outs[j] = L.ConvOut(L.ptr(part), c0, part.stride(0), 1, 0)
        parts.append(part)
        c0 += dj
    args = L.CausalConv1dUpdateArgs(
        x=None, x_stride_batch=0, conv_state=L.ptr(conv_state), new_state=L.ptr(conv_state),
        weight=L.ptr(w), bias=L.ptr(b_c), out=outs, batch=batch, dim=dim, width=width,
        nout=len(sizes), x_dtype=L.M2_BF16 if x_dtype == torch.bfloat16 else L.M2_F32,
        state_dtype=L.M2_F32, new_state_dtype=L.M2_F32, w_dtype=L.dtype_code(w, "weight"),
        bias_dtype=L.M2_F32 if b_c is None else L.dtype_code(b_c, "bias"),
        out_dtype=L.dtype_code(parts[0], "out"), silu=int(activation == "silu"))
    # keep the converted operands alive as long as the arguments
    args._keep = (w, b_c)
    return args, (parts[0] if split_sizes is None else tuple(parts))


def causal_conv1d_update(x_new, conv_state, weight, bias=None, activation=None, *,
                         inplace=False, split_sizes=None):
    """-> (new_conv_state (batch, d, width), out (batch, d)) (out: a tuple of
    (batch, d_j) parts with split_sizes).

    new_conv_state = concat(conv_state[:, :, 1:], x_new[:, :, None]);
    out = silu?(sum(new_conv_state * weight, -1) + bias).
    """
    dev = L.device_of(x_new, conv_state, weight, bias)
    L.require(conv_state.dim() == 3, "conv_state must be (batch, d, width)")
    batch, dim, width = (int(v) for v in conv_state.shape)
    L.require(tuple(x_new.shape) == (batch, dim), f"x_new.shape={tuple(x_new.shape)}")
    w, kw = _weight(weight, dim)
    L.require(kw == width, f"weight width {kw} != conv_state width {width}")
    if bias is not None:
        L.require(tuple(bias.shape) == (dim,), f"bias.shape={tuple(bias.shape)}")
    b_c = _float_tensor(bias, "bias")
    if x_new.dtype not in (torch.float32, torch.bfloat16):
        x_new = x_new.float()
    if x_new.stride(1) != 1:
        x_new = x_new.contiguous()
    st = conv_state if conv_state.dtype in (torch.float32, torch.bfloat16) else conv_state.float()
    nsdt = _result_dtype(st.dtype, x_new.dtype)
    if inplace and st is conv_state and st.dtype == nsdt and st.is_contiguous():
        new_state = st
    else:
        st = st.contiguous()
        new_state = torch.empty((batch, dim, width), dtype=nsdt, device=dev)
    odt = _result_dtype(nsdt, w.dtype, None if b_c is None else b_c.dtype)
    sizes = _splits(dim, split_sizes)
    parts, outs, c0 = [], (L.ConvOut * 3)(), 0
    for j, dj in enumerate(sizes):
        part = torch.empty((batch, dj), dtype=odt, device=dev)
        outs[j] = L.ConvOut(L.ptr(part), c0, part.stride(0), 1, 0)
        parts.append(part)
        c0 += dj
    args = L.CausalConv1dUpdateArgs(
        x=L.ptr(x_new), x_stride_batch=x_new.stride(0), conv_state=L.ptr(st),
        new_state=L.ptr(new_state), weight=L.ptr(w), bias=L.ptr(b_c), out=outs, batch=batch,
        dim=dim, width=width, nout=len(sizes), x_dtype=L.dtype_code(x_new, "x_new"),
        state_dtype=L.dtype_code(st, "conv_state"), new_state_dtype=L.dtype_code(new_state, "state"),
        w_dtype=L.dtype_code(w, "weight"),
        bias_dtype=L.M2_F32 if b_c is None else L.dtype_code(b_c, "bias"),
        out_dtype=L.dtype_code(parts[0], "out"), silu=int(activation == "silu"))
    with torch.cuda.device(dev):
        L.call("m2_causal_conv1d_update", args, L.stream_of(dev))
    return new_state, (parts[0] if split_sizes is None else tuple(parts))


__all__ = ["causal_conv1d", "causal_conv1d_update", "update_from_columns"]

"""The row-op call surface of the reference (src/rowops.py, compile_rowop.py)
on libwxhip.so's row kernels.

Reference design entry points (rowops.py:221-330), same names and keyword
arguments, operating on device tensors (torch, bf16 unless noted) instead of
IRON tensors; each writes c_out and returns it:

  layer_norm(a_in, c_out, *, rows, cols)                 'ln'  (no affine)
  softmax_row / softmax_row2 / softmax_row3 / softmax_row4(a_in, c_out, *, rows, cols)
  softmax_row3_win / softmax_row4_win / softmax_row4r_win(..., valid)
  gelu_row4(...)          'g4'  poly4, truncating rounding
  gelu_row4_rne(...)      'g4r' poly4, RNE
  gelu_row4f(a_in fp32, c_out, *, rows, cols, out_cols=0)   'g4f' fp32 in,
                          bf16 written as a `cols`-wide band of an
                          `out_cols`-wide c_out (rowops.py:80-88)

Every softmax variant computes the same exact-fp32 softmax: the reference's
variants differ only in how the AIE LUT exp and the reciprocal are rounded
(kernels/softmax_row*.cc), which a GPU need not imitate. The op codes 'gl',
'g2', 'g3' (tanh / logistic / 5-piece GELU, kernels/gelu_row*.cc) are
superseded variants the reference keeps for A/B only and are not built:
they raise ``NotImplementedError``. Row widths need not be multiples of 16.
"""
import numpy as np

from . import _lib as L

# rowop op code -> (kind, variant) ; compile_rowop.py:12-19
OPS = {
    "ln": ("ln", None),
    "sm": ("softmax", None), "s2": ("softmax", None), "s3": ("softmax", None),
    "s4": ("softmax", None), "s3w": ("softmax", None), "s4w": ("softmax", None),
    "s4rw": ("softmax", None),
    "g4": ("gelu", L.WXH_GELU_POLY4_TRUNC), "g4r": ("gelu", L.WXH_GELU_POLY4_RNE),
    "g4f": ("gelu", L.WXH_GELU_POLY4_RNE),
    "gl": ("absent", None), "g2": ("absent", None), "g3": ("absent", None),
}
GELU_VARIANT = {"g4": L.WXH_GELU_POLY4_TRUNC, "g4r": L.WXH_GELU_POLY4_RNE,
                "g4f": L.WXH_GELU_POLY4_RNE, "erf": L.WXH_GELU_ERF}


def _torch():
    import torch
    return torch


def as_device_bf16(dev, buf, rows, cols):
    """uint16 bf16 bits (numpy) or a bf16 torch tensor -> device bf16 [rows, cols]."""
    torch = _torch()
    if isinstance(buf, np.ndarray):
        if buf.dtype != np.uint16:
            raise TypeError("bf16 buffers are passed as uint16 bit arrays")
        t = torch.from_numpy(np.ascontiguousarray(buf).reshape(rows, cols).view(np.int16))
        return t.view(torch.bfloat16).to(dev.device)
    if buf.dtype != torch.bfloat16:
        raise TypeError(f"expected a bf16 tensor, got {buf.dtype}")
    return buf.reshape(rows, cols).to(dev.device)


def bits_to_numpy(t):
    """bf16 torch tensor -> uint16 numpy bit array."""
    torch = _torch()
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def run_op(dev, op, x, valid=None, out=None):
    """Apply rowop `op` to the device tensor x [rows, cols]; returns bf16."""
    kind, variant = OPS.get(op, ("unknown", None))
    if kind == "unknown":
        raise ValueError(f"unknown rowop {op!r}; known: {sorted(OPS)}")
    if kind == "absent":
        raise NotImplementedError(
            f"rowop {op!r} is a superseded GELU variant that is not built here; "
            f"use g4r/g4/g4f (poly4) or the erf GELU")
    if kind == "ln":
        return dev.layer_norm(x, out=out)
    if kind == "softmax":
        return dev.softmax_rows(x, valid=valid, out=out)
    return dev.gelu(x, variant, out=out)


_DEV = None  # the Device the design-level entry points run on


def _dev_of(t):
    global _DEV
    if _DEV is None or _DEV.device != t.device:
        from .device import Device
        _DEV = Device(t.device.index or 0)
    return _DEV


def _rows(a_in, c_out, rows, cols):
    return a_in.reshape(rows, cols), c_out.reshape(rows, cols)


def layer_norm(a_in, c_out, *, rows, cols):
    x, y = _rows(a_in, c_out, rows, cols)
    _dev_of(x).layer_norm(x, out=y)
    return c_out


def _softmax(a_in, c_out, rows, cols, valid=0):
    x, y = _rows(a_in, c_out, rows, cols)
    _dev_of(x).softmax_rows(x, valid=valid or cols, out=y)
    return c_out


def softmax_row(a_in, c_out, *, rows, cols):
    return _softmax(a_in, c_out, rows, cols)


softmax_row2 = softmax_row3 = softmax_row4 = softmax_row


def softmax_row3_win(a_in, c_out, *, rows, cols, valid):
    return _softmax(a_in, c_out, rows, cols, valid)


softmax_row4_win = softmax_row4r_win = softmax_row3_win


def _gelu(a_in, c_out, rows, cols, variant, out_cols=0):
    x = a_in.reshape(rows, cols)
    if out_cols:
        # c_out is the `out_cols`-wide buffer or a band view of it
        y = c_out if c_out.dim() == 2 else c_out.reshape(rows, out_cols)
        if y.shape[0] != rows or y.shape[1] < cols:
            raise ValueError(f"c_out {tuple(c_out.shape)} cannot hold a {rows}x{cols} band")
        y = y[:, :cols]
    else:
        y = c_out.reshape(rows, cols)
    _dev_of(x).gelu(x, variant, out=y)
    return c_out


def gelu_row4(a_in, c_out, *, rows, cols):
    return _gelu(a_in, c_out, rows, cols, L.WXH_GELU_POLY4_TRUNC)


def gelu_row4_rne(a_in, c_out, *, rows, cols):
    return _gelu(a_in, c_out, rows, cols, L.WXH_GELU_POLY4_RNE)


def gelu_row4f(a_in, c_out, *, rows, cols, out_cols=0):
    return _gelu(a_in, c_out, rows, cols, L.WXH_GELU_POLY4_RNE, out_cols)


def _absent(name):
    def f(*a, **k):
        raise NotImplementedError(f"rowops.{name} is a superseded variant not built here")
    f.__name__ = name
    return f


gelu_row = _absent("gelu_row")
gelu_row2 = _absent("gelu_row2")
gelu_row3 = _absent("gelu_row3")

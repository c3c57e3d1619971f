"""bf16 bit helpers for the oracle (numpy has no bf16 dtype and ml_dtypes is
not installed).

A bf16 value is carried as its uint16 bit pattern: the top half of the fp32
pattern. Two fp32 -> bf16 roundings are used by the reference kernels:

* round-to-nearest-even (RNE): ``aie::set_rounding(conv_even)`` in
  kernels/gelu_row4_rne.cc:49 and kernels/gelu_row4f.cc:64, and what torch's
  ``.to(torch.bfloat16)`` does;
* truncation toward zero: the AIE2 default, inherited by kernels/gelu_row4.cc
  (no set_rounding call, gelu_row4.cc:44-61).

NaN handling follows the usual convention (quiet the NaN, keep the sign); no
hot-path input is NaN.
"""
import numpy as np


def f32_bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def round_rne(x):
    """fp32 -> bf16 bits (uint16), round to nearest, ties to even."""
    u = f32_bits(x).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r = np.where(nan, ((f32_bits(x) >> 16) | 0x40).astype(np.uint32), r)
    return r.astype(np.uint16)


def round_trunc(x):
    """fp32 -> bf16 bits (uint16), truncation toward zero."""
    return (f32_bits(x) >> 16).astype(np.uint16)


def to_f32(b):
    """bf16 bits (uint16) -> fp32 values."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rb(x, mode="rne"):
    """Round fp32 values to bf16 and return them as fp32 (exactly representable)."""
    return to_f32(round_rne(x) if mode == "rne" else round_trunc(x))


def ulp_diff(a_bits, b_bits):
    """Distance in bf16 units-in-the-last-place between two bf16 bit arrays.

    Maps the sign-magnitude patterns onto a monotone integer line, so +0 and -0
    are 0 apart and the step across zero counts like any other step.
    """
    def line(b):
        b = np.asarray(b, dtype=np.uint16).astype(np.int64)
        mag = b & 0x7FFF
        return np.where(b & 0x8000, -mag, mag)
    return np.abs(line(a_bits) - line(b_bits))

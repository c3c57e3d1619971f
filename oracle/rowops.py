"""Row-wise definitions the GPU row kernels are gated against (CPU, numpy).

Each function returns float64 (or the bf16 bits for the bit-exact poly4), so a
test rounds the exact value once, RNE, and compares bf16 bit patterns within
1 ulp. Reference lines restated:

* LayerNorm           src/npu_whisper_encoder.py:278-281 (population variance,
                      eps 1e-5, affine after the normalisation)
* erf-GELU            src/npu_whisper_encoder.py:284-287 (exact erf
                      formulation, "torch nn.GELU() default")
* A&S erf-GELU        src/npu_whisper_encoder.py:284-300 (the reference's own
                      fp32 numpy evaluation through Abramowitz-Stegun 7.1.26)
* poly4 GELU          kernels/gelu_poly4_eval.inc:27-65 with the constants of
                      kernels/gelu_poly4_coeffs.h:4-13; input rounding of
                      kernels/gelu_row4f.cc:58-84 (g4f), RNE of
                      kernels/gelu_row4_rne.cc:44-66 (g4r), truncation of
                      kernels/gelu_row4.cc:44-61 (g4)
* softmax             src/npu_whisper_encoder.py:416-419 and
                      src/rawxrt.py:156-159; the `valid` window of
                      src/rowops.py:60-73 (only the first `valid` columns of a
                      row are read and written)
"""
import math

import numpy as np

from . import bf16 as B

# --- poly4 constants (kernels/gelu_poly4_coeffs.h:4-13; every one is bf16-exact)
POLY4_BREAK = (1.0, 2.0, 4.0)
POLY4_SHIFT = (0.5, 1.5, 3.0)
POLY4_SCALE = (2.0, 2.0, 1.0)
POLY4_COEF = (
    (-0.0020446777, -0.013000488, 0.077148438, -0.06640625, -0.15429688),
    (0.0021514893, -0.0071716309, -0.0040283203, 0.063964844, -0.10009766),
    (-0.0029296875, 0.010681152, -0.015869141, 0.012023926, -0.0040283203),
)


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    """(x - mean) / sqrt(var + eps) * gamma + beta over the last axis, float64.

    npu_whisper_encoder.py:278-281: mean and population variance of the row,
    eps inside the square root. gamma/beta None means the plain normalisation
    of kernels/layer_norm_gb.cc:48-86 (no affine).
    """
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, dtype=np.float64)
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)
    return y


def _erfc(z):
    from scipy.special import erfc
    return erfc(z)


def gelu_erf(x):
    """Exact erf-GELU 0.5*x*(1+erf(x/sqrt2)), float64.

    npu_whisper_encoder.py:284-287 defines GELU as the exact erf formulation.
    Written as 0.5*x*erfc(-x/sqrt2), which is the same function without the
    cancellation of 1+erf(...) for very negative x.
    """
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * _erfc(-x / math.sqrt(2.0))


def gelu_erf_as_f32(x):
    """The reference's numpy GELU exactly as it evaluates: fp32 numpy with the
    Abramowitz-Stegun 7.1.26 erf (npu_whisper_encoder.py:284-300).

    Reported beside the gate only: for x < -4.8 it is more than 1 bf16 ulp from
    the exact GELU (1 - erf cancels), where |GELU| < 3.1e-6.
    """
    x = np.asarray(x, dtype=np.float32)
    a1, a2, a3, a4, a5, p = (0.254829592, -0.284496736, 1.421413741,
                             -1.453152027, 1.061405429, 0.3275911)
    z = x / np.float32(math.sqrt(2.0))
    sign = np.sign(z)
    az = np.abs(z)
    t = 1.0 / (1.0 + p * az)
    y = 1.0 - (((((a5 * t + a4) * t) + a3) * t + a2) * t + a1) * t * np.exp(-az * az)
    erf = (sign * y).astype(np.float32)
    return (0.5 * x * (1.0 + erf)).astype(np.float32)


def gelu_poly4(x, mode="rne", f32_input=False):
    """Bit-exact poly4 GELU; returns bf16 bits (uint16).

    x           fp32 values (f32_input=True, the g4f kernel) or values that are
                already bf16 (g4/g4r: pass the bf16 bits through bf16.to_f32)
    mode        "rne" (g4r, g4f) or "trunc" (g4) -- the rounding used at every
                fp32 -> bf16 point below

    gelu_poly4_eval.inc:27-65, per element:
      s = |x|; q = 0
      for p = 2, 1, 0:                          (innermost piece wins)
        u   = rb(rb(s - SHIFT[p]) * SCALE[p])
        acc = COEF[p][0]
        for k = 1..4: acc = fp32(COEF[p][k] + rb(acc) * u)
        if s < BREAK[p]: q = rb(acc)
      out = rb(max(x, 0) + q)
    g4f first rounds its fp32 input to bf16 RNE (gelu_row4f.cc:64-78).
    """
    f32 = np.float32
    x = np.asarray(x, dtype=np.float32)
    if f32_input:
        x = B.rb(x, "rne")
    else:
        if not np.array_equal(B.rb(x, "trunc"), x):
            raise ValueError("gelu_poly4: bf16-input variant got non-bf16 values")

    def rb(v):
        return B.rb(v.astype(np.float32), mode)

    s = np.abs(x)
    q = np.zeros_like(x)
    for p in (2, 1, 0):
        u = rb(rb(s - f32(POLY4_SHIFT[p])) * f32(POLY4_SCALE[p]))
        acc = np.full_like(x, f32(POLY4_COEF[p][0]))
        for k in range(1, 5):
            acc = (f32(POLY4_COEF[p][k]) + rb(acc) * u).astype(np.float32)
        q = np.where(s < f32(POLY4_BREAK[p]), rb(acc), q)
    out = (np.maximum(x, f32(0.0)) + q).astype(np.float32)
    return B.round_rne(out) if mode == "rne" else B.round_trunc(out)


def softmax(x, valid=None):
    """Row softmax over the last axis in float64 (npu_whisper_encoder.py:416-419).

    valid: only the first `valid` columns take part (rowops.py:60-73); the
    returned array then has `valid` columns.
    """
    x = np.asarray(x, dtype=np.float64)
    if valid is not None:
        x = x[..., :valid]
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)

"""The int8 oracle (oracle/int8.py) pinned on the CPU.

Pins, chosen so that a wrong axis for a scale, a missing zero-row rule, a
rounding mode other than half-to-even or a scale applied twice fails one:
* closed forms: rows whose maximum is 127 have scale 1, so their codes are
  the values and the product is the exact integer product;
* round half to even on .5 codes (numpy's rint, the reference's rounding);
* a brute-force element-by-element restatement on tiny inputs;
* invariance under power-of-two scaling of A and of B (exact in fp32);
* the encoder: in "fp32" mode encoder_int8 is the fp32 encoder (equal to
  encoder_torch), and in "perchan" it stays close to it.
"""
import numpy as np
import pytest

from oracle import encoder as OE
from oracle import int8 as OQ
from wxhip import synth


def test_quantize_rows_closed_forms():
    x = np.array([[0.0, 63.5, 127.0, -127.0],      # max 127: scale 1, codes = rint(x)
                  [0.0, 0.0, 0.0, 0.0],            # all zero: scale 1, codes 0
                  [0.5, 1.5, 2.5, 127.0],          # half to even: 0, 2, 2
                  [-2.5, -0.5, 3.5, -127.0]], np.float32)
    q, s = OQ.quantize_rows(x)
    np.testing.assert_array_equal(s, [1, 1, 1, 1])
    np.testing.assert_array_equal(q, [[0, 64, 127, -127], [0, 0, 0, 0], [0, 2, 2, 127],
                                      [-2, 0, 4, -127]])
    y = np.array([[1.0, -2.0, 0.25]], np.float32)
    q, s = OQ.quantize_rows(y)
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    np.testing.assert_array_equal(q, [[64, -127, 16]])  # 63.5 -> 64, 15.875 -> 16


def test_q_matmul_scale_one_is_the_integer_product():
    rng = np.random.default_rng(0)
    A = rng.integers(-127, 128, (7, 40)).astype(np.float32)
    B = rng.integers(-127, 128, (40, 9)).astype(np.float32)
    A[:, 0] = 127.0  # every row's max |.| is 127
    B[0, :] = -127.0  # every column's max |.| is 127
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(OQ.q_matmul(A, B), want)
    bias = rng.normal(size=9).astype(np.float32)
    np.testing.assert_array_equal(OQ.q_matmul(A, B, bias), want + bias)


def _brute(A, B, bias, mode):
    M, K = A.shape
    N = B.shape[1]
    f = np.float32
    sa = [max(abs(float(v)) for v in A[m]) for m in range(M)]
    sa = [f(f(s) / f(127.0)) if s else f(1.0) for s in sa]
    if mode == "pertensor":
        t = max(abs(float(v)) for v in B.ravel())
        sw = [f(f(t) / f(127.0)) if t else f(1.0)] * N
    else:
        sw = [max(abs(float(B[k, n])) for k in range(K)) for n in range(N)]
        sw = [f(f(s) / f(127.0)) if s else f(1.0) for s in sw]
    qa = [[int(round(float(f(A[m, k]) / sa[m]))) for k in range(K)] for m in range(M)]
    qb = [[int(round(float(f(B[k, n]) / sw[n]))) for n in range(N)] for k in range(K)]
    out = np.empty((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            acc = sum(qa[m][k] * qb[k][n] for k in range(K))
            out[m, n] = f(f(f(acc) * sa[m]) * sw[n]) + (bias[n] if bias is not None else f(0))
    return out


@pytest.mark.parametrize("mode", ["perchan", "pertensor"])
def test_q_matmul_matches_brute_force(mode):
    rng = np.random.default_rng(3)
    A = rng.normal(0, 2, (5, 24)).astype(np.float32)
    A[2] = 0.0
    B = (rng.normal(0, 0.05, (24, 6)) * rng.uniform(0.2, 3, 6)).astype(np.float32)
    bias = rng.normal(size=6).astype(np.float32)
    np.testing.assert_array_equal(OQ.q_matmul(A, B, bias, mode), _brute(A, B, bias, mode))


def test_q_matmul_power_of_two_invariance():
    rng = np.random.default_rng(4)
    A = rng.normal(size=(9, 64)).astype(np.float32)
    B = rng.normal(size=(64, 11)).astype(np.float32)
    r = OQ.q_matmul(A, B)
    np.testing.assert_array_equal(OQ.q_matmul(A * 8, B), r * 8)
    np.testing.assert_array_equal(OQ.q_matmul(A, B / 4), r / 4)


def test_quantize_cols_is_quantize_rows_of_the_transpose():
    rng = np.random.default_rng(5)
    B = rng.normal(size=(50, 7)).astype(np.float32)
    q, s = OQ.quantize_cols(B)
    qt, st = OQ.quantize_rows(B.T)
    np.testing.assert_array_equal(q, qt.T)
    np.testing.assert_array_equal(s, st)


def test_encoder_int8_fp32_mode_is_the_fp32_encoder_and_perchan_stays_close():
    W = synth.make_weights("tiny")
    mel = synth.make_mel(80, 400, 0)
    ref = OE.encoder_torch(W, mel)
    f = OQ.encoder_int8(W, mel, mode="fp32")
    assert np.abs(f - ref).max() < 2e-3
    q = OQ.encoder_int8(W, mel, mode="perchan")
    c = float((q * ref).sum() / np.linalg.norm(q) / np.linalg.norm(ref))
    assert 0.99 < c < 0.99999, c  # quantisation noise is there, and small


def _rn32(fr):
    """A rational rounded to the nearest binary32 (ties to even)."""
    from fractions import Fraction
    a = np.float32(float(fr))
    cands = [a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(-np.inf))]
    return min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.float32(c).view(np.uint32)) & 1))


def test_quantiser_quotient_is_the_correctly_rounded_division():
    """The device quantisers (quant_quotient in csrc/common.h) form x / s as
    q0 = RN(x r), then RN(q0 + RN(x - q0 s) r) with r = RN(1 / s) and both
    steps as single-rounding FMAs (emulated here in exact rational
    arithmetic), for s in [2^-100, 2^100]. That must equal numpy's float32
    x / s, which the oracle's rint(x / s) uses, on quotients next to the
    half-integers where rint turns, and on random ones; scales across the
    whole allowed range."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    for it in range(3000):
        m = np.float32(2.0 ** rng.choice([rng.uniform(-20, 20), rng.uniform(-92, -80),
                                          rng.uniform(80, 92)]) * rng.uniform(1, 2))
        s = np.float32(m / np.float32(127.0))
        assert 2.0 ** -100 <= s <= 2.0 ** 100
        r = np.float32(np.float32(1.0) / s)
        if it % 2:
            x = np.float32((int(rng.integers(-127, 127)) + 0.5) * float(s))
            x = np.float32(x + int(rng.integers(-1, 2)) * np.spacing(x))
        else:
            x = np.float32(rng.uniform(-1, 1) * float(m))
        q0 = np.float32(x * r)
        e = _rn32(-Fraction(float(q0)) * Fraction(float(s)) + Fraction(float(x)))
        q1 = _rn32(Fraction(float(e)) * Fraction(float(r)) + Fraction(float(q0)))
        assert q1 == np.float32(x / s), (x, s, q1, np.float32(x / s))

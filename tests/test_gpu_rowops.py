"""GPU parity of the row kernels against the CPU oracle (oracle/rowops.py).

Gate: within 1 bf16 ulp per element of the exact definition (LayerNorm,
erf-GELU, softmax), bit-exact for the poly4 GELU variants. Inputs are the
standalone row-op workloads (LN [1500,1280], GELU [1500,5120], softmax
[30000,1500]) plus edge shapes.
"""
import numpy as np
import pytest
import torch

from conftest import bits, case, report, to_dev_bf16
from oracle import bf16 as OB
from oracle import rowops as OR
from wxhip import _lib as L
from wxhip import synth

pytestmark = pytest.mark.gpu

ULP = 1


def _ulps(got_bits, want_f64):
    want = OB.round_rne(np.asarray(want_f64, np.float64).astype(np.float32))
    return OB.ulp_diff(got_bits, want)


def _ln_check(got_bits, x, g=None, b=None):
    """LayerNorm gate: within 1 bf16 ulp of the exact value, except where the
    output cancels (x_hat*gamma ~ -beta): no fp32 evaluation can hold 1 ulp of
    a result 2^7 times smaller than its terms, so there the bound is 2^-16 of
    the terms' magnitude (a few fp32 ulps of it). Returns how many elements
    needed that allowance."""
    xh = OR.layer_norm(x)
    gg = 1.0 if g is None else np.asarray(g, np.float64)
    bb = 0.0 if b is None else np.asarray(b, np.float64)
    exact = xh * gg + bb
    mag = np.abs(xh * gg) + np.abs(bb)
    d = _ulps(got_bits, exact)
    ok1 = d <= ULP
    err = np.abs(OB.to_f32(got_bits).astype(np.float64) - exact)
    ok2 = (np.abs(exact) < 2 ** -7 * mag) & (err <= 2 ** -16 * mag)
    assert (ok1 | ok2).all(), f"max {d[~(ok1 | ok2)].max()} ulp outside the bound"
    n = int((~ok1).sum())
    # the allowance is for isolated cancellations, not a looser gate: at most
    # 0.1 % of the elements may need it
    assert n <= 1e-3 * d.size, f"{n} of {d.size} elements needed the cancellation allowance"
    return n


@pytest.fixture(scope="module")
def inputs():
    return synth.rowop_inputs(seed=0)


def test_layernorm_bf16_affine_rowop_shape(dev, inputs):
    case("layernorm bf16 [1500,1280] gamma/beta")
    x = OB.rb(inputs["ln_x"])
    g, b = inputs["ln_gamma"], inputs["ln_beta"]
    y = dev.layer_norm(to_dev_bf16(x, dev), torch.from_numpy(g).to(dev.device),
                       torch.from_numpy(b).to(dev.device))
    n = _ln_check(bits(y), x, g, b)
    report("layernorm_rowop_shape_allowance", elements=int(x.size), allowance=n)


@pytest.mark.parametrize("rows,cols", [(1, 8), (7, 384), (33, 768), (1500, 1280), (5, 4096)])
def test_layernorm_shapes_fp32_in(dev, rows, cols):
    case(f"layernorm fp32 in {rows}x{cols}")
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.normal(0.5, 3, (rows, cols))).astype(np.float32)
    g = rng.normal(1, 0.1, cols).astype(np.float32)
    b = rng.normal(0, 0.1, cols).astype(np.float32)
    y = dev.layer_norm(torch.from_numpy(x).to(dev.device), torch.from_numpy(g).to(dev.device),
                       torch.from_numpy(b).to(dev.device))
    _ln_check(bits(y), x, g, b)
    # fp32 output path: within a few fp32 ulps of the fp64 value
    yf = dev.layer_norm(torch.from_numpy(x).to(dev.device), torch.from_numpy(g).to(dev.device),
                        torch.from_numpy(b).to(dev.device), out_dtype=torch.float32)
    np.testing.assert_allclose(yf.cpu().numpy(), OR.layer_norm(x, g, b), rtol=2e-5, atol=2e-5)


def test_layernorm_no_affine_and_fused_residual(dev):
    case("layernorm 'ln' no affine + fused residual")
    rng = np.random.default_rng(3)
    x = OB.rb(rng.normal(0, 1, (512, 1280)).astype(np.float32))
    y = dev.layer_norm(to_dev_bf16(x, dev))
    assert _ulps(bits(y), OR.layer_norm(x)).max() <= ULP
    # invariant of the normalisation: per-row mean 0, variance 1 (before bf16)
    yf = dev.layer_norm(to_dev_bf16(x, dev), out_dtype=torch.float32).cpu().numpy()
    assert np.abs(yf.mean(1)).max() < 1e-5 and np.abs(yf.var(1) - 1).max() < 1e-3
    r = rng.normal(0, 1, (512, 1280)).astype(np.float32)
    s = torch.empty(512, 1280, dtype=torch.float32, device=dev.device)
    xs = torch.from_numpy(OB.to_f32(OB.round_rne(x))).to(dev.device)
    y2 = dev.layer_norm(xs, resid=torch.from_numpy(r).to(dev.device), sum_out=s)
    np.testing.assert_array_equal(s.cpu().numpy(), (x + r).astype(np.float32))
    assert _ulps(bits(y2), OR.layer_norm((x + r).astype(np.float32))).max() <= ULP


def test_gelu_erf_rowop_shape(dev, inputs):
    case("gelu erf bf16 [1500,5120]")
    x = OB.rb(inputs["gelu_x"])
    y = dev.gelu(to_dev_bf16(x, dev), L.WXH_GELU_ERF)
    d = _ulps(bits(y), OR.gelu_erf(x))
    assert d.max() <= ULP, f"max {d.max()} ulp at x={x.ravel()[d.argmax()]}"


def test_gelu_erf_tails_fp32_in(dev):
    case("gelu erf fp32 tails")
    x = np.concatenate([np.linspace(-20, 20, 40001), [-1e30, -88.0, -13.5, -5.0, 0.0,
                                                      1e-30, 1e30]]).astype(np.float32)
    y = dev.gelu(torch.from_numpy(x[None]).to(dev.device), L.WXH_GELU_ERF)
    d = _ulps(bits(y)[0], OR.gelu_erf(x))
    assert d.max() <= ULP, f"max {d.max()} ulp at x={x[d.argmax()]}"


@pytest.mark.parametrize("op,mode", [("g4r", "rne"), ("g4", "trunc")])
def test_gelu_poly4_bit_exact_all_bf16(dev, op, mode):
    case(f"gelu poly4 {op} over every finite bf16")
    allbits = np.arange(65536, dtype=np.uint16)
    x = OB.to_f32(allbits)
    x = x[np.isfinite(x)].reshape(1, -1)
    variant = {"g4r": L.WXH_GELU_POLY4_RNE, "g4": L.WXH_GELU_POLY4_TRUNC}[op]
    y = dev.gelu(torch.from_numpy(x).to(dev.device).to(torch.bfloat16), variant)
    with np.errstate(all="ignore"):
        want = OR.gelu_poly4(x, mode=mode)
    got = bits(y)
    bad = np.nonzero(got != want)[1]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[0, bad[:5]]}"


def test_gelu_poly4_f32_input_band(dev, inputs):
    """g4f: fp32 accumulator in, bf16 out as a column band of a wider buffer
    (the fc1 chunk -> fc2 A write of rawxrt.py:487-516)."""
    case("gelu poly4 g4f fp32 in, banded out")
    x = inputs["gelu_x"][:, :1280].copy()
    wide = torch.zeros(1500, 5120, dtype=torch.bfloat16, device=dev.device)
    dev.gelu(torch.from_numpy(x).to(dev.device), L.WXH_GELU_POLY4_RNE, out=wide[:, 1280:2560])
    got = bits(wide)
    want = OR.gelu_poly4(x, mode="rne", f32_input=True)
    np.testing.assert_array_equal(got[:, 1280:2560], want)
    assert (got[:, :1280] == 0).all() and (got[:, 2560:] == 0).all()


@pytest.mark.parametrize("variant", ["erf", "g4r", "g4"])
def test_gelu_odd_width_scalar_path(dev, variant):
    """Widths and strides that are not multiples of 8 take the one-element
    path (with its own copy of the poly4 table)."""
    case(f"gelu {variant} odd width 13x37")
    rng = np.random.default_rng(5)
    x = OB.rb(rng.normal(0, 3, (13, 37)).astype(np.float32))
    code = {"erf": L.WXH_GELU_ERF, "g4r": L.WXH_GELU_POLY4_RNE,
            "g4": L.WXH_GELU_POLY4_TRUNC}[variant]
    y = dev.gelu(to_dev_bf16(x, dev), code)
    if variant == "erf":
        assert _ulps(bits(y), OR.gelu_erf(x)).max() <= ULP
    else:
        np.testing.assert_array_equal(bits(y), OR.gelu_poly4(x, mode="rne" if variant == "g4r" else "trunc"))


def test_gelu_strided_bands_and_tiny_inputs(dev):
    """Row-strided input and output (the 32-bit chunk-index path) on values
    around the poly4 table's ends: 0, denormals, 2^-10 and its neighbours,
    the breaks 1, 2, 4 and beyond."""
    case("gelu strided bands, table ends")
    pts = np.array([0.0, 1e-40, 1e-30, 2.0 ** -11, 2.0 ** -10, 2.0 ** -10 * 1.0078125,
                    2.0 ** -9, 0.5, 0.99609375, 1.0, 1.9921875, 2.0, 3.984375, 4.0,
                    4.03125, 7.0, 1e4], np.float32)
    row = OB.rb(np.concatenate([pts, -pts, np.linspace(-6, 6, 1024 - 2 * pts.size)]).astype(np.float32))
    x = np.tile(row, (24, 1))
    xd = torch.zeros(24, 1032, dtype=torch.bfloat16, device=dev.device)
    xd[:, 8:1032] = to_dev_bf16(x, dev)
    for variant, mode in ((L.WXH_GELU_POLY4_RNE, "rne"), (L.WXH_GELU_POLY4_TRUNC, "trunc")):
        out = torch.zeros(24, 1040, dtype=torch.bfloat16, device=dev.device)
        dev.gelu(xd[:, 8:1032], variant, out=out[:, 16:1040])
        np.testing.assert_array_equal(bits(out)[:, 16:], OR.gelu_poly4(x, mode=mode))
        assert (bits(out)[:, :16] == 0).all()
    out = torch.zeros(24, 1040, dtype=torch.bfloat16, device=dev.device)
    dev.gelu(xd[:, 8:1032], L.WXH_GELU_ERF, out=out[:, 16:1040])
    assert _ulps(bits(out)[:, 16:], OR.gelu_erf(x)).max() <= ULP


def test_softmax_rowop_shape(dev, inputs):
    case("softmax bf16 [30000,1500]")
    x = OB.rb(inputs["sm_x"])
    y = dev.softmax_rows(to_dev_bf16(x, dev))
    d = _ulps(bits(y), OR.softmax(x))
    assert d.max() <= ULP, f"max {d.max()} ulp, {int((d > 0).sum())} differ"


@pytest.mark.parametrize("rows,cols,valid", [(20 * 4, 1536, 1500), (9, 1504, 1504),
                                             (5, 37, 37), (6, 5000, 4999), (3, 16, 1)])
def test_softmax_window_and_widths(dev, rows, cols, valid):
    case(f"softmax {rows}x{cols} valid={valid}")
    rng = np.random.default_rng(cols)
    x = OB.rb(rng.normal(0, 6, (rows, cols)).astype(np.float32))
    sentinel = torch.full((rows, cols), 7.0, dtype=torch.bfloat16, device=dev.device)
    y = dev.softmax_rows(to_dev_bf16(x, dev), valid=valid, out=sentinel)
    got = bits(y)
    d = _ulps(got[:, :valid], OR.softmax(x, valid=valid))
    assert d.max() <= ULP
    # columns past the window are neither read nor written (rowops.py:60-73)
    assert (OB.to_f32(got[:, valid:]) == 7.0).all()


def test_softmax_overflow_and_uniform(dev):
    case("softmax logits +200 and constant rows")
    rng = np.random.default_rng(9)
    x = OB.rb((rng.normal(0, 6, (512, 512)) + 200).astype(np.float32))
    y = dev.softmax_rows(to_dev_bf16(x, dev))
    assert _ulps(bits(y), OR.softmax(x)).max() <= ULP
    c = torch.full((4, 1500), -3.0, dtype=torch.bfloat16, device=dev.device)
    p = dev.softmax_rows(c).float().cpu().numpy()
    np.testing.assert_array_equal(p, np.full((4, 1500), OB.rb(np.float32(1 / 1500))[0]))


def test_rowop_surface_codes(dev):
    """HipRT.rowop with the reference's op codes."""
    import wxhip
    case("rowop codes")
    rt = wxhip.HipRT()
    rng = np.random.default_rng(11)
    x = OB.rb(rng.normal(0, 3, (64, 256)).astype(np.float32))
    xb = OB.round_rne(x)
    assert (rt.rowop("g4r", xb, 64, 256) == OR.gelu_poly4(x, "rne")).all()
    assert (rt.rowop("g4", xb, 64, 256) == OR.gelu_poly4(x, "trunc")).all()
    assert OB.ulp_diff(rt.rowop("s4w", xb, 64, 256), OB.round_rne(OR.softmax(x).astype(np.float32))).max() <= 1
    assert OB.ulp_diff(rt.rowop("ln", xb, 64, 256), OB.round_rne(OR.layer_norm(x).astype(np.float32))).max() <= 1
    with pytest.raises(NotImplementedError):
        rt.rowop("g3", xb, 64, 256)
    with pytest.raises(ValueError):
        rt.rowop("zz", xb, 64, 256)

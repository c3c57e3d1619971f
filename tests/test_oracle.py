"""Pins for the CPU oracle (oracle/), CPU only.

Each oracle function is checked against something other than its own
formula: a library routine (torch), an independent restatement (oracle/poly4.c,
the numpy encoder twin), closed forms and invariants, and the committed golden
fixtures in tests/golden/. A plausible slip -- dropped term, wrong sign or
index, transposed operand, wrong rounding -- fails at least one of these.
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bf16 as OB
from oracle import encoder as OE
from oracle import rowops as OR
from oracle.build import poly4_gelu_c
from wxhip import synth

GOLDEN = Path(__file__).resolve().parent / "golden"
ALL_BF16 = OB.to_f32(np.arange(65536, dtype=np.uint16))
FINITE = ALL_BF16[np.isfinite(ALL_BF16)]


# ----------------------------------------------------------------- bf16

def test_bf16_rne_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 10, 200000), rng.normal(0, 1e-30, 1000),
                        [0.0, -0.0, 1e38, -1e38, 3.4e38]]).astype(np.float32)
    # exact ties: low 16 bits = 0x8000, both parities of the kept lsb
    ties = ((np.arange(1000, dtype=np.uint32) << 16) | 0x3f808000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(OB.round_rne(x), want)


def test_bf16_trunc_and_ulp():
    x = np.array([1.0, 1.0078125 + 2 ** -9, -2.5], np.float32)
    assert (OB.to_f32(OB.round_trunc(x)) == np.array([1.0, 1.0078125, -2.5], np.float32)).all()
    a = OB.round_rne(np.array([1.0, -0.0, 0.0], np.float32))
    b = OB.round_rne(np.array([1.0078125, 0.0, -1e-45], np.float32))
    assert list(OB.ulp_diff(a, b)) == [1, 0, 0]


# ----------------------------------------------------------------- poly4

@pytest.mark.parametrize("mode", ["rne", "trunc"])
def test_poly4_numpy_equals_c_restatement_on_every_bf16(mode):
    with np.errstate(all="ignore"):
        a = OR.gelu_poly4(FINITE, mode=mode)
    np.testing.assert_array_equal(a, poly4_gelu_c(FINITE, mode=mode))


def test_poly4_g4f_numpy_equals_c_on_fp32():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 3, 500000), rng.uniform(-5, 5, 200000)]).astype(np.float32)
    np.testing.assert_array_equal(OR.gelu_poly4(x, "rne", f32_input=True),
                                  poly4_gelu_c(x, "rne", f32_input=True))
    # g4f == g4r on the RNE-rounded input (gelu_row4f.cc:1-12)
    np.testing.assert_array_equal(OR.gelu_poly4(x, "rne", f32_input=True),
                                  OR.gelu_poly4(OB.rb(x), "rne"))


def test_poly4_matches_committed_golden():
    g = np.load(GOLDEN / "poly4_all_bf16.npz")
    with np.errstate(all="ignore"):
        np.testing.assert_array_equal(OR.gelu_poly4(FINITE, "rne"), g["rne"])
        np.testing.assert_array_equal(OR.gelu_poly4(FINITE, "trunc"), g["trunc"])


def test_poly4_against_exact_gelu_and_invariants():
    with np.errstate(all="ignore"):
        y = OB.to_f32(OR.gelu_poly4(FINITE, "rne"))
    exact = OR.gelu_erf(FINITE)
    small = np.abs(FINITE) < 8
    err = np.abs(y[small] - exact[small])
    # the minimax fit's published quality: ~7.8e-3 worst case, and not exact
    assert 5e-3 < err.max() < 8e-3
    # q = 0 beyond the last break: GELU(x) = relu(x) exactly for |x| >= 4
    big = np.abs(FINITE) >= 4
    np.testing.assert_array_equal(y[big], np.maximum(FINITE[big], 0))
    assert np.isfinite(y).all()
    # q depends on |x| only: out(x) - out(-x) = x up to the final roundings
    x = FINITE[(np.abs(FINITE) < 4) & (np.abs(FINITE) > 1e-3)]
    with np.errstate(all="ignore"):
        d = OB.to_f32(OR.gelu_poly4(x, "rne")) - OB.to_f32(OR.gelu_poly4(-x, "rne"))
    assert np.abs(d - x).max() <= 2 ** -7 * np.abs(x).max()


# ----------------------------------------------------------------- erf GELU, LN, softmax

def test_gelu_erf_vs_torch_and_normal_cdf():
    # torch's GELU (exact-erf form) where 1 + erf does not cancel
    x = np.linspace(-5, 10, 150001)
    want = F.gelu(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(OR.gelu_erf(x), want, rtol=1e-9, atol=1e-300)
    # everywhere, including the far tail: GELU(x) = x * Phi(x), Phi = scipy ndtr
    from scipy.special import ndtr
    x = np.linspace(-30, 30, 300001)
    np.testing.assert_allclose(OR.gelu_erf(x), x * ndtr(x), rtol=1e-12, atol=1e-300)
    assert OR.gelu_erf(np.array([0.0]))[0] == 0.0


def test_gelu_as_f32_is_the_reference_formula():
    """The A&S fp32 twin stays within A&S 7.1.26's |eps| <= 1.5e-7 (scaled)
    of the exact GELU, and differs from it only in the far negative tail."""
    x = OB.rb(np.linspace(-6, 6, 100001).astype(np.float32))
    a = OR.gelu_erf_as_f32(x).astype(np.float64)
    e = OR.gelu_erf(x)
    assert np.abs(a - e).max() < 1e-6
    tail = x < -4.8
    big = OB.ulp_diff(OB.round_rne(a.astype(np.float32)), OB.round_rne(e.astype(np.float32))) > 1
    assert not big[~tail].any()


def test_layer_norm_vs_torch_and_invariants():
    rng = np.random.default_rng(1)
    x = rng.normal(2, 3, (64, 1280))
    g, b = rng.normal(1, 0.1, 1280), rng.normal(0, 0.1, 1280)
    want = F.layer_norm(torch.from_numpy(x), (1280,), torch.from_numpy(g), torch.from_numpy(b),
                        1e-5).numpy()
    np.testing.assert_allclose(OR.layer_norm(x, g, b), want, rtol=1e-10, atol=1e-10)
    y = OR.layer_norm(x)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(1), 1 - 1e-5 / (x.var(1) + 1e-5), rtol=1e-9)


def test_softmax_vs_torch_and_invariants():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 6, (100, 1536))
    np.testing.assert_allclose(OR.softmax(x), torch.softmax(torch.from_numpy(x), -1).numpy(),
                               rtol=1e-12, atol=1e-300)
    p = OR.softmax(x)
    np.testing.assert_allclose(p.sum(1), 1, rtol=1e-12)
    np.testing.assert_allclose(OR.softmax(x + 200.0), p, rtol=1e-9)
    np.testing.assert_allclose(OR.softmax(x, valid=1500), OR.softmax(x[:, :1500]))
    # the reference's rowop gate (test_rowops.py:35-53): rel L2 < 0.02
    xb = OB.rb(x.astype(np.float32))
    ref32 = np.exp(xb - xb.max(1, keepdims=True))
    ref32 /= ref32.sum(1, keepdims=True)
    assert np.linalg.norm(OR.softmax(xb) - ref32) / np.linalg.norm(ref32) < 1e-5


# ----------------------------------------------------------------- encoder

def test_sinusoids_closed_form():
    pe = synth.sinusoids(1500, 384)
    inc = math.log(10000) / (192 - 1)
    for t, i in [(0, 0), (7, 3), (1499, 191), (123, 100)]:
        assert abs(pe[t, i] - math.sin(t * math.exp(-inc * i))) < 1e-6
        assert abs(pe[t, 192 + i] - math.cos(t * math.exp(-inc * i))) < 1e-6


def test_im2col_conv_equals_conv1d():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (5, 17)).astype(np.float32)
    w = rng.normal(0, 1, (4, 5, 3)).astype(np.float32)
    for stride in (1, 2):
        got = OE.im2col(x, 3, stride, 1) @ w.reshape(4, 15).T
        want = F.conv1d(torch.from_numpy(x)[None], torch.from_numpy(w), stride=stride,
                        padding=1)[0].numpy().T
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_attention_known_answers_in_oracle():
    """Known answers of the attention step (HISTORY.md:220-223), run through
    the oracle encoder's own attention: with Wk = 0 every score is equal, so
    each head's output is the column mean of v."""
    W = synth.make_weights("tiny", n_layer=1)
    W["w.blocks.0.attn.key.weight"][:] = 0
    mel = synth.make_mel(80, 64, seed=0)
    # reproduce the block input to read v, then check o = mean(v)
    t = {k: torch.from_numpy(v) for k, v in W.items()}
    x = F.gelu(F.conv1d(torch.from_numpy(mel)[None], t["w.conv1.weight"], t["w.conv1.bias"], padding=1))
    x = F.gelu(F.conv1d(x, t["w.conv2.weight"], t["w.conv2.bias"], stride=2, padding=1))
    x = x.permute(0, 2, 1)[0] + t["w.positional_embedding"][:32]
    h = F.layer_norm(x, (384,), t["w.blocks.0.attn_ln.weight"], t["w.blocks.0.attn_ln.bias"], 1e-5)
    v = F.linear(h, t["w.blocks.0.attn.value.weight"], t["w.blocks.0.attn.value.bias"])
    o = v.mean(0, keepdim=True).expand_as(v)
    x1 = x + F.linear(o, t["w.blocks.0.attn.out.weight"], t["w.blocks.0.attn.out.bias"])
    h2 = F.layer_norm(x1, (384,), t["w.blocks.0.mlp_ln.weight"], t["w.blocks.0.mlp_ln.bias"], 1e-5)
    x2 = x1 + F.linear(F.gelu(F.linear(h2, t["w.blocks.0.mlp.0.weight"], t["w.blocks.0.mlp.0.bias"])),
                       t["w.blocks.0.mlp.2.weight"], t["w.blocks.0.mlp.2.bias"])
    want = F.layer_norm(x2, (384,), t["w.ln_post.weight"], t["w.ln_post.bias"], 1e-5).numpy()
    np.testing.assert_allclose(OE.encoder_torch(W, mel), want, rtol=1e-4, atol=1e-4)


def test_encoder_attention_matches_sdpa():
    """The oracle's head split / scale (hd^-1/4 on q and k) equals torch's
    scaled_dot_product_attention with 1/sqrt(hd)."""
    rng = np.random.default_rng(5)
    q, k, v = (torch.from_numpy(rng.normal(0, 1, (1, 6, 40, 64))) for _ in range(3))
    s = 64 ** -0.25
    mine = torch.softmax((q * s) @ (k * s).transpose(-1, -2), -1) @ v
    np.testing.assert_allclose(mine.numpy(), F.scaled_dot_product_attention(q, k, v).numpy(),
                               rtol=1e-10, atol=1e-12)


def test_encoder_torch_equals_numpy_twin():
    W = synth.make_weights("tiny", n_layer=2)
    mel = synth.make_mel(80, 400, seed=3)
    a = OE.encoder_torch(W, mel)
    b = OE.encoder_numpy(W, mel)
    assert a.shape == (200, 384)
    np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-4)


def test_encoder_matches_committed_golden():
    g = np.load(GOLDEN / "encoder_tiny_2layer_ctx50.npz")
    W = synth.make_weights("tiny", n_layer=2)
    mel = synth.make_mel(80, 100, seed=0)
    np.testing.assert_array_equal(mel, g["mel"])
    np.testing.assert_allclose(OE.encoder_torch(W, mel), g["out"], rtol=1e-5, atol=1e-5)


def test_encoder_batch_axis():
    W = synth.make_weights("tiny", n_layer=1)
    mels = synth.make_mel_batch(2, 80, 120)
    both = OE.encoder_torch(W, mels)
    for i in range(2):
        np.testing.assert_allclose(both[i], OE.encoder_torch(W, mels[i]), rtol=1e-5, atol=1e-5)

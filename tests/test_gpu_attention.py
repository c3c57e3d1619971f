"""GPU parity of the fused flash attention (wxh_attention) against the closed
form softmax((q s)(k s)^T) v per head in fp64, on the bf16-rounded operands
(the reference's attention chain semantics, rawxrt.py:813-891 and
npu_whisper_encoder.py:491-511), plus its known answers (K = 0 -> column mean
of V; V = ones -> ones, HISTORY.md:220-223).

Tolerance: P is rounded to bf16 before P.V (the reference rounds its scores
and probabilities to bf16 too), so elements agree to ~1e-2 relative of |V|;
cosine >= 0.99995 against fp64.
"""
import numpy as np
import pytest
import torch

from conftest import case, cosine
from oracle import bf16 as OB
from wxhip import _lib as L

pytestmark = pytest.mark.gpu


def _ref(q, k, v, nh, scale):
    """fp64 closed form, q/k/v [B, T, nh*64]."""
    B, T, d = q.shape
    hd = d // nh
    out = np.empty((B, T, d))
    for b in range(B):
        for h in range(nh):
            sl = slice(h * hd, (h + 1) * hd)
            s = (q[b, :, sl].astype(np.float64) @ k[b, :, sl].astype(np.float64).T) * scale
            s -= s.max(1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(1, keepdims=True)
            out[b, :, sl] = p @ v[b, :, sl].astype(np.float64)
    return out


@pytest.fixture
def nosplit(dev):
    """nosplit(mode) sets the device's key split (WXH_TUNE_ATTN_KEYSPLIT):
    "nosplit" the one-group kernel, else automatic; reset after the test."""
    yield lambda mode: dev.set_tuning(L.WXH_TUNE_ATTN_KEYSPLIT, int(mode == "nosplit"))
    dev.set_tuning(L.WXH_TUNE_ATTN_KEYSPLIT, 0)


def _run(dev, q, k, v, nh, scale, out_dtype=torch.float32):
    B, T, d = q.shape
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a.reshape(B * T, d))).to(dev.device)
    Q, K, Vt = dev.pack_qkv(f(q), f(k), f(v), B, T, nh)
    return dev.attention(Q, K, Vt, B, nh, T, scale, out_dtype=out_dtype).cpu().float().numpy().reshape(B, T, d)


# Fewer than 256 workgroups (every shape but the batch-4 one) split each
# workgroup's keys over two wave groups; "nosplit" forces the one-part kernel.
@pytest.mark.parametrize("B,T,nh,mode", [(1, 1500, 20, ""), (2, 512, 6, ""), (1, 100, 2, ""),
                                         (3, 65, 1, ""), (1, 1, 1, ""), (4, 1500, 20, ""),
                                         (1, 1500, 20, "nosplit"), (3, 65, 1, "nosplit")])
def test_attention_vs_closed_form(dev, B, T, nh, mode, nosplit):
    case(f"attention B={B} T={T} nh={nh} {mode}")
    nosplit(mode)
    rng = np.random.default_rng(T + nh)
    d = nh * 64
    q, k, v = (OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32)) for _ in range(3))
    scale = 1.0 / 8.0
    got = _run(dev, q, k, v, nh, scale)
    ref = _ref(q, k, v, nh, scale)
    assert np.isfinite(got).all()
    assert cosine(got, ref) >= 0.99995, cosine(got, ref)
    assert np.abs(got - ref).max() <= 2e-2 * np.abs(v).max()


def test_attention_known_answers(dev):
    """K = 0 gives uniform P, so O = column mean of V; V = 1 gives O = 1."""
    case("attention known answers")
    B, T, nh = 1, 1500, 4
    d = nh * 64
    rng = np.random.default_rng(1)
    q = OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32))
    v = OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32))
    got = _run(dev, q, np.zeros_like(q), v, nh, 0.125)
    want = v.astype(np.float64).mean(1, keepdims=True)
    assert np.abs(got - want).max() < 4e-3
    ones = _run(dev, q, OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32)),
                np.ones_like(q), nh, 0.125)
    np.testing.assert_allclose(ones, 1.0, atol=1e-2)


def test_attention_large_logits_masked_tail(dev):
    """Big scores stay finite, and padded keys (T = 1500 -> 1536) get no mass:
    compare against the closed form with exactly T keys."""
    case("attention large logits")
    B, T, nh = 1, 1500, 2
    d = nh * 64
    rng = np.random.default_rng(4)
    q, k = (OB.rb(rng.normal(0, 4, (B, T, d)).astype(np.float32)) for _ in range(2))
    v = OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32))
    got = _run(dev, q, k, v, nh, 0.125)
    ref = _ref(q, k, v, nh, 0.125)
    assert np.isfinite(got).all() and cosine(got, ref) >= 0.9999


@pytest.mark.parametrize("mode", ["", "nosplit"])
def test_attention_late_max_and_negative_scores(dev, mode, nosplit):
    """The running exp2 reference has to move on a late key block (the last
    50 keys score ~2^30 above the first block's maximum, so that block's
    exps overflow the fast path and are redone), and has to settle far below
    zero when every score is about -80 (identical keys: O = column mean of V).
    Both against the fp64 closed form."""
    case(f"attention late max / negative scores {mode}")
    nosplit(mode)
    B, T, nh = 1, 1500, 2
    d = nh * 64
    rng = np.random.default_rng(8)
    q = OB.rb((np.abs(rng.normal(0, 1, (B, T, d))) + 0.5).astype(np.float32))
    k = OB.rb(rng.normal(0, 0.1, (B, T, d)).astype(np.float32))
    k[:, T - 50:] = OB.rb(2.0 + rng.normal(0, 0.1, (B, 50, d)).astype(np.float32))
    v = OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32))
    got = _run(dev, q, k, v, nh, 0.125)
    ref = _ref(q, k, v, nh, 0.125)
    assert np.isfinite(got).all()
    assert cosine(got, ref) >= 0.99995, cosine(got, ref)
    assert np.abs(got - ref).max() <= 2e-2 * np.abs(v).max()
    kneg = np.full_like(k, -8.0)
    got = _run(dev, q, kneg, v, nh, 0.125)
    want = v.astype(np.float64).mean(1, keepdims=True)
    assert np.isfinite(got).all() and np.abs(got - want).max() < 4e-3


def test_attention_bf16_out_and_batch_independence(dev):
    """Batch item b of a batched call equals the same item run alone, bit for bit."""
    case("attention batch independence")
    B, T, nh = 3, 300, 3
    d = nh * 64
    rng = np.random.default_rng(6)
    q, k, v = (OB.rb(rng.normal(0, 1, (B, T, d)).astype(np.float32)) for _ in range(3))
    allb = _run(dev, q, k, v, nh, 0.125, out_dtype=torch.bfloat16)
    for b in range(B):
        one = _run(dev, q[b:b + 1], k[b:b + 1], v[b:b + 1], nh, 0.125, out_dtype=torch.bfloat16)
        np.testing.assert_array_equal(allb[b], one[0])


def test_hiprt_attn_chain_and_host_path(dev):
    """RawRT.attn_chain contract (q, k, v fp32 [ctx, d], n_head, scale=hd^-1/4)
    and the device-routed per-head path agree."""
    import wxhip
    case("HipRT.attn_chain")
    rt = wxhip.HipRT()
    rng = np.random.default_rng(8)
    ctx, nh = 1500, 6
    q, k, v = (rng.normal(0, 1, (ctx, nh * 64)).astype(np.float32) for _ in range(3))
    scale = 64 ** -0.25
    o1 = rt.attn_chain(q, k, v, nh, scale)
    ref = _ref(OB.rb(q)[None], OB.rb(k)[None], OB.rb(v)[None], nh, scale * scale)[0]
    assert cosine(o1, ref) >= 0.99995
    o2 = rt._attn_host(q, k, v, nh, scale)
    assert cosine(o2, ref) >= 0.9999
    assert rt.chain_ok and not rt.fallbacks

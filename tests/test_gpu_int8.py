"""The int8 GEMM path on the GPU against the int8 oracle (oracle/int8.py,
the reference's quantised matmul of bench/probe_int8_decode.py:48-74).

Gates:
* wxh_quantize_rows: codes and scales bit-identical to the oracle (the
  division is the correctly rounded fp32 one, rint is half-to-even);
* wxh_gemm_i8: bit-identical fp32 results on the oracle's codes for every
  tile configuration (128x128 with 2 and 3 slots, 256x256), edge tiles and
  the residual epilogue; bf16 outputs equal RNE of those values; the GELU
  epilogues within 1 bf16 ulp / 3e-4 relative of the exact GELU of them;
* the q_matmul plug: bit-identical to the oracle's q_matmul;
* the encoder (HipEncoder int8=True; attention stays bf16 MFMA, the
  oracle's is fp32): cosine >= 0.999 against the oracle's int8 encoder at
  tiny depth, and the bf16 path unchanged after switching back.
"""
import numpy as np
import pytest
import torch

from conftest import case, cosine, report
from oracle import int8 as OQ
from oracle import rowops as OR
from wxhip import _lib as L
from wxhip import synth

pytestmark = pytest.mark.gpu


def _t(x, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev.device)
    return t if dtype is None else t.to(dtype)


@pytest.mark.parametrize("rows,cols,pad", [(1, 8, 8), (37, 240, 256), (1500, 1280, 1280),
                                           (300, 5120, 5120), (64, 1152, 1280)])
def test_quantize_rows_bit_exact(dev, rows, cols, pad):
    case(f"quantize_rows {rows}x{cols} pad {pad}")
    rng = np.random.default_rng(rows + cols)
    x = (rng.normal(0, 1, (rows, cols)) * rng.uniform(1e-3, 50, (rows, 1))).astype(np.float32)
    x[0, : min(8, cols)] = [0.5, -1.5, 2.5, 127, 63.5, -63.5, 0, 1][: min(8, cols)]
    if rows > 2:
        x[2] = 0.0  # an all-zero row: scale 1, codes 0
    q, s = dev.quantize_rows(_t(x, dev), cols_pad=pad)
    wq, ws = OQ.quantize_rows(x)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)
    qn = q.cpu().numpy()
    np.testing.assert_array_equal(qn[:, :cols], wq)
    assert (qn[:, cols:] == 0).all()
    # bf16 input: the oracle on the bf16 values
    xb = _t(x, dev, torch.bfloat16)
    q2, s2 = dev.quantize_rows(xb, cols_pad=pad)
    wq2, ws2 = OQ.quantize_rows(xb.float().cpu().numpy())
    np.testing.assert_array_equal(s2.cpu().numpy(), ws2)
    np.testing.assert_array_equal(q2.cpu().numpy()[:, :cols], wq2)


def test_quantize_per_tensor(dev):
    case("quantize per tensor")
    rng = np.random.default_rng(9)
    B = rng.normal(0, 0.02, (384, 1536)).astype(np.float32)
    q, s = dev.quantize_rows(_t(B, dev), per_tensor=True)
    wq, ws = OQ.quantize_cols(B.T, per_tensor=True)
    assert s.numel() == 1 and s.item() == ws[0]
    np.testing.assert_array_equal(q.cpu().numpy(), wq.T)
    z = torch.zeros(16, 64, device=dev.device)
    qz, sz = dev.quantize_rows(z, per_tensor=True)
    assert sz.item() == 1.0 and (qz == 0).all()


def _i8_case(rng, M, N, K):
    qa = rng.integers(-127, 128, (M, K)).astype(np.int8)
    qw = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = rng.uniform(1e-3, 0.1, M).astype(np.float32)
    sw = rng.uniform(1e-4, 0.01, N).astype(np.float32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    r = OQ.int_matmul(qa, qw.T).astype(np.float32)
    want = (r * sa[:, None] * sw[None, :] + bias).astype(np.float32)
    return qa, qw, sa, sw, bias, want


@pytest.mark.parametrize("M,N,K", [
    (100, 200, 128),     # partial tiles (128x64, 3-slot ring)
    (1500, 1280, 1280),  # batch-1 out-proj shape: 120 tiles of 128x128 -> 128x64 tiles
    (1000, 1000, 1152),  # 128x64 tiles with 128-element K-steps (K % 256 != 0)
    (1000, 1000, 256),   # 256-element K-steps: one step, fewer than the ring's slots
    (1000, 1000, 512),   # two steps
    (1500, 2560, 1280),  # 240 tiles: 128x128, 8 waves, 3-slot ring
    (1500, 5120, 1280),  # batch-1 fc1 shape: 128x128, 2-slot ring
    (4000, 4096, 256),   # >= 256 tiles of 256x256 (edge rows)
    (6000, 1280, 5120),  # long K
])
def test_gemm_i8_bit_exact(dev, M, N, K):
    case(f"gemm_i8 {M}x{N}x{K}")
    rng = np.random.default_rng(M + N + K)
    qa, qw, sa, sw, bias, want = _i8_case(rng, M, N, K)
    A, Wt = _t(qa, dev), _t(qw, dev)
    SA, SW, b = _t(sa, dev), _t(sw, dev), _t(bias, dev)
    got = dev.gemm_i8(A, SA, Wt, SW, b, L.WXH_EPI_F32).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    # residual: out += result (fp32 add of the same value)
    x0 = rng.normal(0, 1, (M, N)).astype(np.float32)
    x = _t(x0, dev)
    dev.gemm_i8(A, SA, Wt, SW, b, L.WXH_EPI_RESID_F32, out=x)
    np.testing.assert_array_equal(x.cpu().numpy(), x0 + want)
    # bf16 out: RNE of the fp32 result
    got16 = dev.gemm_i8(A, SA, Wt, SW, b, L.WXH_EPI_BF16)
    np.testing.assert_array_equal(got16.float().cpu().numpy(),
                                  torch.from_numpy(want).to(torch.bfloat16).float().numpy())
    # GELU epilogues: the project's erf-GELU of the fp32 result, whose fitted
    # tail term has relative error < 2.8e-4 (so the fp32 output is within
    # 3e-4 relative; bf16 outputs within 1 ulp). The GELU input must be the
    # rounded r*sa*sw plus the bias: fused into one FMA it differs by an ulp,
    # which near cancellation shows here as a relative error of 1e-2.
    g32 = dev.gemm_i8(A, SA, Wt, SW, b, L.WXH_EPI_F32_GELU_ERF).cpu().numpy()
    exact = OR.gelu_erf(want.astype(np.float64))
    # (relative error is meaningful where the result is a normal fp32 number;
    # below ~1e-38, for x < -13, fp32 denormals carry few bits)
    err = np.where(np.abs(exact) > 1e-35, np.abs(g32 - exact) / np.maximum(np.abs(exact), 1e-30), 0)
    k = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() < 3e-4, (float(err.max()), float(want[k]), float(g32[k]), float(exact[k]))
    assert np.abs(g32 - exact)[np.abs(exact) <= 1e-35].max(initial=0) < 1e-35
    g16 = dev.gemm_i8(A, SA, Wt, SW, b, L.WXH_EPI_BF16_GELU_ERF).float().cpu().numpy()
    assert np.abs(g16 - exact).max() <= np.abs(exact).max() * 2 ** -8


def test_gemm_i8_rejects_unpadded_k(dev):
    case("gemm_i8 K % 128 != 0")
    A = torch.zeros(16, 120, dtype=torch.int8, device=dev.device)
    W = torch.zeros(16, 120, dtype=torch.int8, device=dev.device)
    s = torch.ones(16, device=dev.device)
    with pytest.raises(L.WxhError):
        dev.gemm_i8(A, s, W, s)


@pytest.mark.parametrize("mode", ["perchan", "pertensor"])
def test_q_matmul_plug_matches_oracle(dev, mode):
    import wxhip
    from wxhip import int8 as Q
    case(f"q_matmul plug {mode}")
    rng = np.random.default_rng(1)
    A = rng.normal(0, 1.5, (300, 240)).astype(np.float32)  # K = 240: zero-padded to 256
    B = rng.normal(0, 0.02, (240, 384)).astype(np.float32)
    bias = rng.normal(0, 0.1, 384).astype(np.float32)
    qm = Q.q_matmul_factory(mode, rt=wxhip.HipRT())
    np.testing.assert_array_equal(qm(A, B, bias), OQ.q_matmul(A, B, bias, mode))
    np.testing.assert_array_equal(qm(A, B), OQ.q_matmul(A, B, None, mode))  # cached B
    assert qm.stats["n"] == 2


def test_encoder_int8_tiny_against_oracle(dev):
    import wxhip
    case("encoder int8 tiny (4 layers, ctx 1500)")
    W = synth.make_weights("tiny")
    mel = synth.make_mel(80, 3000, 0)
    enc = wxhip.HipEncoder(dev, W, int8=True)
    got = enc.forward(_t(mel, dev)).cpu().numpy()
    ref = OQ.encoder_int8(W, mel)
    c = cosine(got, ref)
    from oracle import encoder as OE
    c32 = cosine(got, OE.encoder_torch(W, mel))
    report("encoder_int8_tiny", cosine_vs_int8_oracle=c, cosine_vs_fp32_oracle=c32)
    assert got.shape == (1500, 384) and np.isfinite(got).all()
    assert c >= 0.999, c
    # back to bf16: the same result as an encoder built without int8
    enc.set_int8(False)
    b16 = enc.forward(_t(mel, dev)).cpu().numpy()
    ref16 = wxhip.HipEncoder(dev, W).forward(_t(mel, dev)).cpu().numpy()
    np.testing.assert_array_equal(b16, ref16)
    enc.set_int8(True)
    np.testing.assert_array_equal(enc.forward(_t(mel, dev)).cpu().numpy(), got)


def test_encoder_int8_batch_and_mirror(dev):
    """Batch items are independent in the int8 graph, and the reference's
    entry point with the q_matmul plug (the probe's call) lands on the same
    features as the oracle."""
    import wxhip
    from wxhip import encoder as E
    from wxhip import int8 as Q
    case("encoder int8 batch 2 ctx 512 + q_matmul mirror")
    W = synth.make_weights("tiny")
    mels = np.stack([synth.make_mel(80, 1024, s) for s in (3, 4)])
    enc = wxhip.HipEncoder(dev, W, int8=True)
    got = enc.forward(_t(mels, dev)).cpu().numpy()
    for b in range(2):
        one = enc.forward(_t(mels[b], dev)).cpu().numpy()
        assert cosine(got[b], one) >= 0.99999
        ref = OQ.encoder_int8(W, mels[b])
        assert cosine(got[b], ref) >= 0.999
    rt = wxhip.HipRT()
    qm = Q.q_matmul_factory("perchan", rt=rt)
    out = E.encoder(W, mels[0], qm, rt.matmul, n_layer=4, n_head=6,
                    attn_fn=rt.attn_chain, fold_bias=False)
    c = cosine(out, OQ.encoder_int8(W, mels[0]))
    report("encoder_int8_mirror", cosine=c, gemms=qm.stats["n"])
    assert qm.stats["n"] == 2 + 4 * 6 and c >= 0.999

"""CPU checks of the drop-in module's host-side logic (no GPU).

* im2col against the oracle's restatement of npu_whisper_encoder.py:422-431
  and against torch's conv1d, for both conv strides;
* zero_bias keeps one read-only zero array per width (the identity the
  reference's weight cache relies on, :308-315);
* prepare_mlp_chunks follows the width rule of :383-396 (d-wide chunks when
  d divides N, even pieces otherwise, an explicit `chunk`, nothing for
  widths that fit) and the chunks rebuild fc1 exactly;
* which device path encoder() takes for each argument combination the
  reference's callers use (graph, and with which GELUs, or op by op).
"""
import numpy as np
import pytest

from oracle import encoder as OE
from wxhip import encoder as E
from wxhip import synth
from wxhip.hiprt import HipRT


@pytest.mark.parametrize("C,T,stride", [(80, 3000, 1), (384, 3000, 2), (5, 7, 1), (3, 8, 2),
                                        (4, 1, 1), (2, 9, 2)])
def test_im2col_matches_reference_layout_and_conv1d(C, T, stride):
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(C * 31 + T)
    x = rng.normal(0, 1, (C, T)).astype(np.float32)
    got = E.im2col(x, 3, stride, 1)
    np.testing.assert_array_equal(got, OE.im2col(x, 3, stride, 1))
    assert got.flags.c_contiguous and got.dtype == np.float32
    w = rng.normal(0, 1, (6, C, 3)).astype(np.float32)
    conv = F.conv1d(torch.from_numpy(x)[None], torch.from_numpy(w), stride=stride, padding=1)
    np.testing.assert_allclose(got @ w.reshape(6, C * 3).T, conv[0].numpy().T,
                               rtol=1e-5, atol=1e-4)


def test_zero_bias_identity_and_read_only():
    a, b = E.zero_bias(384), E.zero_bias(384)
    assert a is b and a.dtype == np.float32 and a.shape == (384,) and not a.any()
    assert E.zero_bias(1280) is not a
    with pytest.raises(ValueError):
        a[0] = 1.0


def _w(d, n_layer=2, ffn=None):
    W = synth.add_transposed(synth.make_weights(
        {"n_mels": 8, "d": d, "n_head": d // 64, "n_layer": n_layer, "n_ctx": 16}))
    if ffn is not None:   # a non-Whisper fc1 width, for the uneven-piece rule
        rng = np.random.default_rng(1)
        for L in range(n_layer):
            p = f"w.blocks.{L}."
            W[p + "mlp.0.weight_T"] = rng.normal(0, 0.02, (d, ffn)).astype(np.float32)
            W[p + "mlp.0.bias"] = rng.normal(0, 0.02, ffn).astype(np.float32)
    return W


@pytest.mark.parametrize("d,ffn,chunk,widths", [
    (1280, None, 0, [1280] * 4),          # large-v3: d divides 5120
    (384, None, 0, None),                 # tiny: 1536 fits, nothing made
    (384, None, 768, [768, 768]),         # explicit chunk
    (384, None, 1000, [1000, 536]),       # explicit chunk with a tail
    (1280, 5000, 0, [2500, 2500]),        # d does not divide: even pieces
    (1280, 9000, 0, [3000, 3000, 3000]),
])
def test_prepare_mlp_chunks_rule(d, ffn, chunk, widths):
    W = _w(d, ffn=ffn)
    made = E.prepare_mlp_chunks(W, 2, d, chunk)
    for L in range(2):
        p = f"w.blocks.{L}."
        if widths is None:
            assert p + "mlp.0.parts" not in W
            continue
        parts = W[p + "mlp.0.parts"]
        assert [wc.shape[1] for wc, _ in parts] == widths
        np.testing.assert_array_equal(np.hstack([wc for wc, _ in parts]), W[p + "mlp.0.weight_T"])
        np.testing.assert_array_equal(np.concatenate([bc for _, bc in parts]), W[p + "mlp.0.bias"])
        assert all(wc.flags.c_contiguous and bc.flags.c_contiguous for wc, bc in parts)
    n_parts = 0 if widths is None else len(widths)
    assert len(made) == 2 * 2 * n_parts
    if n_parts:   # weight, bias, weight, bias, ... in chunk order
        assert made[0] is W["w.blocks.0.mlp.0.parts"][0][0]
        assert made[1] is W["w.blocks.0.mlp.0.parts"][0][1]


@pytest.fixture
def rt():
    """A HipRT without a device: only what the path choice reads."""
    r = object.__new__(HipRT)
    r.graph_ok = r.chain_ok = r.mlp_ok = True
    return r


def test_graph_plan(rt, monkeypatch):
    W = _w(384, n_layer=1)
    Wp = _w(1280, n_layer=1)
    E.prepare_mlp_chunks(Wp, 1, 1280)
    plan = lambda W_, **kw: E._plan(rt, W_, kw.get("mm", rt.matmul), kw.get("attn_mm", rt.matmul),
                                    kw.get("attn_fn"), kw.get("mlp_fn"), kw.get("fused_gelu", False))
    # the module's own gelu: erf everywhere
    assert plan(W) == ("erf", "erf")
    assert plan(W, attn_fn=rt.attn_chain) == ("erf", "erf")
    # the reference callers' E.gelu = rt.gelu (GELU_OP g4r): poly4 convs; the
    # host MLP GELU follows it, the device MLP plug follows GELU_F32_OP
    monkeypatch.setattr(E, "gelu", rt.gelu)
    assert plan(W) == ("poly4", "poly4")
    assert plan(W, mlp_fn=rt.mlp) == ("poly4", "poly4")          # no chunks: host MLP GELU
    assert plan(Wp, mlp_fn=rt.mlp) == ("poly4", "poly4")
    monkeypatch.setattr(rt, "GELU_F32_OP", "erf", raising=False)
    assert plan(Wp, mlp_fn=rt.mlp) == ("poly4", "erf")
    assert plan(Wp) == ("poly4", "poly4")                        # chunks, no plug: host GELU
    monkeypatch.setattr(rt, "GELU_OP", "g4", raising=False)      # truncating poly4: no graph form
    assert plan(W) is None
    monkeypatch.setattr(rt, "GELU_OP", "erf", raising=False)
    assert plan(W) == ("erf", "erf")
    # any other gelu, plug or overridden stage runs op by op
    monkeypatch.setattr(E, "gelu", lambda x: x)
    assert plan(W) is None
    monkeypatch.setattr(E, "gelu", E._OWN_GELU)
    assert plan(W, attn_fn=lambda *a: None) is None
    assert plan(W, mm=lambda *a, **k: None) is None
    assert plan(W, fused_gelu=True) == ("erf", "erf")
    rt.graph_ok = False
    assert plan(W) is None
    rt.graph_ok = True
    rt._mlp_dev = lambda *a: None
    assert plan(W) is None

"""The drop-in surface as the reference's callers drive it, on the GPU,
against the CPU oracle.

* bench/run_raw_encoder.py:79-100's sequence -- prepare_mlp_chunks,
  register_weights, ``E.gelu = rt.gelu``, ``E.npu_softmax_stack =
  rt.softmax_stack``, ``encoder(..., attn_fn=rt.attn_chain, mlp_fn=rt.mlp,
  fold_bias=True, npu_softmax=True)`` -- through the graph path and the
  op-by-op path, on tiny and on 2-layer large-v3: graph == op path == the
  oracle with the same GELUs (poly4 convs, poly4 MLP);
* HipRT.mlp when its fused device path fails: the unfused device path gives
  the same bits and the failure is recorded;
* encoder() with attn_fn=None: per-head score GEMMs and a softmax on the
  device (npu_softmax True and False), and the chain-vs-host gates of
  tests/test_encoder_golden.py:118-135;
* every wxhip.rowops.<name> design entry point (rowops.py:221-330),
  gelu_row4f's out_cols band and the softmax windows included.
"""
import numpy as np
import pytest
import torch

from conftest import bits, case, cosine, report, to_dev_bf16
from oracle import bf16 as OB
from oracle import encoder as OE
from oracle import rowops as OR
from wxhip import encoder as E
from wxhip import synth

pytestmark = pytest.mark.gpu

COS_FLOOR = 0.999     # the reference's own gate, tests/test_encoder_golden.py:49


def _caller_weights(model, n_layer, chunk=0):
    W = synth.add_transposed(synth.make_weights(model, n_layer=n_layer))
    d = W["w.ln_post.weight"].shape[0]
    extra = E.prepare_mlp_chunks(W, n_layer, d, chunk)
    return W, extra, d // 64


@pytest.mark.parametrize("model,n_layer,chunk,n_mels", [("tiny", 4, 768, 80),
                                                        ("large-v3", 2, 0, 128)])
def test_reference_caller_sequence(dev, model, n_layer, chunk, n_mels, monkeypatch):
    import wxhip
    case(f"run_raw_encoder sequence {model} {n_layer} layers (graph, op by op)")
    W, extra, n_head = _caller_weights(model, n_layer, chunk)
    assert W.get("w.blocks.0.mlp.0.parts") is not None
    mel = synth.make_mel(n_mels, 3000, seed=7)
    rt = wxhip.HipRT()
    rt.register_weights([v for v in W.values() if isinstance(v, np.ndarray)] + extra)
    monkeypatch.setattr(E, "gelu", rt.gelu)
    monkeypatch.setattr(E, "npu_softmax_stack", rt.softmax_stack)
    kw = dict(npu_softmax=True, n_layer=n_layer, n_head=n_head, attn_fn=rt.attn_chain,
              mlp_fn=rt.mlp, fold_bias=True)
    prof = {}
    g = E.encoder(W, mel, rt.matmul, rt.matmul, prof=prof, **kw)
    assert prof["total"] > 0 and not rt.fallbacks
    # the graph ran with the GELUs the patched module asks for
    assert [k[2:] for k in rt._encoders] == [("poly4", "poly4")]
    rt.graph_ok = False                 # the same call, op by op
    o = E.encoder(W, mel, rt.matmul, rt.matmul, prof={}, **kw)
    ref = OE.encoder_torch(W, mel, n_layer, conv_gelu="poly4", mlp_gelu="poly4")
    c_g, c_o, c_go = cosine(g, ref), cosine(o, ref), cosine(g, o)
    report(f"caller_sequence_{model}", cosine_graph=c_g, cosine_ops=c_o, cosine_graph_vs_ops=c_go)
    assert c_g >= 0.9999 and c_o >= 0.9999 and c_go >= 0.9999, (c_g, c_o, c_go)
    assert not rt.fallbacks
    # the module's own gelu is erf: the graph then differs from the poly4 run
    monkeypatch.setattr(E, "gelu", E._OWN_GELU)
    rt.graph_ok = True
    e = E.encoder(W, mel, rt.matmul, rt.matmul, **kw)
    assert not np.array_equal(e, g)
    ref_erf = OE.encoder_torch(W, mel, n_layer, mlp_gelu="poly4")
    assert cosine(e, ref_erf) >= 0.9999


def test_hiprt_mlp_fused_failure_takes_unfused_path(dev):
    """rt.mlp's ladder: the fused device MLP (GELU in fc1's epilogue) raises
    -> the unfused device MLP (fp32 fc1 bands, the g4f row kernel, fc2). Both
    round the same fp32 fc1 values with the same poly4, so the results are
    identical; the failure is recorded once and retires the fused path
    (rawxrt.py:436-455)."""
    import wxhip
    case("HipRT.mlp forced fused failure (large-v3 layer 0, 300 rows)")
    W, extra, _ = _caller_weights("large-v3", 1)
    p = "w.blocks.0."
    parts, w2t = W[p + "mlp.0.parts"], W[p + "mlp.2.weight_T"]
    h = np.random.default_rng(3).normal(0, 1, (300, 1280)).astype(np.float32)
    rt = wxhip.HipRT()
    rt.register_weights(extra + [w2t])
    fused = rt.mlp(h, parts, w2t)
    assert rt.mlp_ok and not rt.fallbacks

    def boom(*a, **k):
        raise RuntimeError("injected: fused MLP unavailable")

    rt._mlp_dev = boom
    unfused = rt.mlp(h, parts, w2t)
    assert not rt.mlp_ok and len(rt.fallbacks) == 1 and "injected" in rt.fallbacks[0]
    np.testing.assert_array_equal(unfused, fused)
    # and against the oracle: fc2(poly4_g4f(fc1(h) + b1)) on bf16 operands, fp64 sums
    f1 = OB.rb(h).astype(np.float64) @ OB.rb(W[p + "mlp.0.weight_T"]).astype(np.float64) \
        + W[p + "mlp.0.bias"]
    f = OB.to_f32(OR.gelu_poly4(f1.astype(np.float32), mode="rne", f32_input=True))
    want = f.astype(np.float64) @ OB.rb(w2t).astype(np.float64)
    assert cosine(fused, want) >= 0.99999
    # GELU_F32_OP = "erf" routes both paths through the erf GELU instead
    rt2 = wxhip.HipRT()
    rt2.GELU_F32_OP = "erf"
    rt2.GELU_OP = "erf"
    a = rt2.mlp(h, parts, w2t)
    rt2._mlp_dev = boom
    b = rt2.mlp(h, parts, w2t)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("npu_softmax", [True, False])
def test_encoder_attn_fn_none_op_path(dev, npu_softmax, monkeypatch):
    """attn_fn=None: the reference's per-head path (npu_whisper_encoder.py:
    486-508): scores by attn_mm, then npu_softmax_stack (npu_softmax) or the
    per-head softmax, then P.V by attn_mm -- here each on the device."""
    import wxhip
    case(f"encoder attn_fn=None op path, npu_softmax={npu_softmax}")
    W = synth.add_transposed(synth.make_weights("tiny", n_layer=2))
    mel = synth.make_mel(80, 1000, seed=9)
    rt = wxhip.HipRT()
    rt.register_weights([v for v in W.values() if isinstance(v, np.ndarray)])
    monkeypatch.setattr(E, "npu_softmax_stack", rt.softmax_stack)
    rt.graph_ok = False
    calls0 = rt.calls
    out = E.encoder(W, mel, rt.matmul, rt.matmul, n_layer=2, n_head=6, npu_softmax=npu_softmax)
    # per layer: q, k, v, 6 score GEMMs, 6 P.V GEMMs, out, fc1, fc2; + 2 convs
    assert rt.calls - calls0 == 2 + 2 * (3 + 12 + 3)
    c = cosine(out, OE.encoder_torch(W, mel, 2))
    report(f"attn_none_npu_softmax_{npu_softmax}", cosine=c)
    assert c >= 0.9999, c


def test_chain_vs_host_gates(dev, monkeypatch):
    """tests/test_encoder_golden.py:118-135 on the tiny encoder: the chained
    encoder (attn_fn=rt.attn_chain) and the host-routed one (no attn_fn,
    npu_softmax=True, E.npu_softmax_stack = rt.softmax_stack) both pass the
    accuracy floor, agree with each other structurally, and the chain is no
    less accurate than the host path (within 5e-4)."""
    import wxhip
    case("chain vs host gates (tiny, 4 layers)")
    W = synth.add_transposed(synth.make_weights("tiny"))
    mel = synth.make_mel(80, 3000, seed=0)
    ref = OE.encoder_torch(W, mel)
    rt = wxhip.HipRT()
    rt.register_weights([v for v in W.values() if isinstance(v, np.ndarray)])
    monkeypatch.setattr(E, "npu_softmax_stack", rt.softmax_stack)
    chain = E.encoder(W, mel, rt.matmul, rt.matmul, prof={}, attn_fn=rt.attn_chain,
                      n_layer=4, n_head=6)
    assert rt.chain_ok and not rt.fallbacks
    rt.graph_ok = False                  # the host-routed call runs op by op
    host = E.encoder(W, mel, rt.matmul, rt.matmul, prof={}, npu_softmax=True, n_layer=4, n_head=6)
    c_chain, c_host, c_ch = cosine(chain, ref), cosine(host, ref), cosine(chain, host)
    report("chain_vs_host", cosine_chain=c_chain, cosine_host=c_host, cosine_chain_vs_host=c_ch)
    assert c_host >= COS_FLOOR and c_ch >= COS_FLOOR
    assert c_chain >= c_host - 5e-4
    assert min(c_chain, c_host) >= 0.9999


# ------------------------------------------------------------------ rowops surface

def _ulps(got_bits, want):
    return OB.ulp_diff(got_bits, OB.round_rne(np.asarray(want, np.float64).astype(np.float32)))


def test_rowops_design_entry_points(dev):
    """wxhip.rowops keeps the reference's design functions (rowops.py:221-330):
    same names and keywords, device tensors in and out, c_out returned."""
    from wxhip import rowops as R
    case("rowops.<name> design entry points")
    rng = np.random.default_rng(21)
    rows, cols = 48, 1536
    x = OB.rb(rng.normal(0, 3, (rows, cols)).astype(np.float32))
    xd = to_dev_bf16(x, dev)

    def out(c=cols):
        return torch.full((rows, c), 7.0, dtype=torch.bfloat16, device=dev.device)

    y = R.layer_norm(xd, out(), rows=rows, cols=cols)
    assert _ulps(bits(y), OR.layer_norm(x)).max() <= 1
    for fn in (R.softmax_row, R.softmax_row2, R.softmax_row3, R.softmax_row4):
        assert _ulps(bits(fn(xd, out(), rows=rows, cols=cols)), OR.softmax(x)).max() <= 1
    for fn in (R.softmax_row3_win, R.softmax_row4_win, R.softmax_row4r_win):
        y = bits(fn(xd, out(), rows=rows, cols=cols, valid=1504))
        assert _ulps(y[:, :1504], OR.softmax(x, valid=1504)).max() <= 1
        assert (OB.to_f32(y[:, 1504:]) == 7.0).all()     # past the window: untouched
    np.testing.assert_array_equal(bits(R.gelu_row4(xd, out(), rows=rows, cols=cols)),
                                  OR.gelu_poly4(x, mode="trunc"))
    np.testing.assert_array_equal(bits(R.gelu_row4_rne(xd, out(), rows=rows, cols=cols)),
                                  OR.gelu_poly4(x, mode="rne"))
    # g4f: an fp32 accumulator in, bf16 out as a column band of a wider buffer
    xf = rng.normal(0, 3, (rows, 512)).astype(np.float32)
    want = OR.gelu_poly4(xf, mode="rne", f32_input=True)
    wide = torch.zeros(rows, 2048, dtype=torch.bfloat16, device=dev.device)
    xfd = torch.from_numpy(xf).to(dev.device)
    assert R.gelu_row4f(xfd, wide[:, 1024:1536], rows=rows, cols=512, out_cols=2048) is not None
    got = bits(wide)
    np.testing.assert_array_equal(got[:, 1024:1536], want)
    assert (got[:, :1024] == 0).all() and (got[:, 1536:] == 0).all()
    full = torch.zeros(rows, 2048, dtype=torch.bfloat16, device=dev.device)
    R.gelu_row4f(xfd, full, rows=rows, cols=512, out_cols=2048)   # the first band
    np.testing.assert_array_equal(bits(full)[:, :512], want)
    assert (bits(full)[:, 512:] == 0).all()
    plain = out(512)
    np.testing.assert_array_equal(bits(R.gelu_row4f(xfd, plain, rows=rows, cols=512)), want)
    with pytest.raises(ValueError):
        R.gelu_row4f(xfd, torch.zeros(rows, 256, dtype=torch.bfloat16, device=dev.device),
                     rows=rows, cols=512, out_cols=256)
    for fn in (R.gelu_row, R.gelu_row2, R.gelu_row3):
        with pytest.raises(NotImplementedError):
            fn(xd, out(), rows=rows, cols=cols)

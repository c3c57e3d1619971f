"""The Whisper audio encoder restated on the CPU, twice.

encoder_torch   torch fp32 with nn.functional ops (conv1d, layer_norm, gelu,
                linear). This is the oracle the GPU encoder is gated against
                (cosine), and the timed CPU baseline. It stands in for the
                reference's oracle, openai-whisper's ``model.encoder`` run in
                torch fp32 (tools/dump_ref.py:60-69), which is not installed
                here and cannot be fetched.
encoder_numpy   fp32 numpy, following src/npu_whisper_encoder.py:436-541 step
                for step (im2col conv, numpy LayerNorm, A&S erf GELU, per-head
                softmax). Used to pin encoder_torch: two restatements written
                from different primitives must agree.

Semantics both follow (npu_whisper_encoder.py:436-541):
  x = gelu(conv1(mel) + b1); x = gelu(conv2_stride2(x) + b2)      [ctx, d]
  x = x + positional_embedding[:ctx]         (sliced for ctx < 1500, :456-458)
  per block: h = LN(x); q = h Wq^T + bq; k = h Wk^T (no bias); v = h Wv^T + bv
             per head: softmax((q_h * hd^-1/4)(k_h * hd^-1/4)^T) v_h
             x = x + o Wo^T + bo; h = LN(x); x = x + gelu(h W1^T + b1) W2^T + b2
  x = LN(x, ln_post)                          eps 1e-5; n_head = d // 64
Weights are the ``"w." + state_dict`` keys of tools/dump_ref.py:72-76.
"""
import numpy as np

from . import rowops as R


def geometry(W):
    """n_layer and n_head read off the weights (npu_whisper_encoder.py:568-573)."""
    n_layer = 1 + max(int(k.split(".")[2]) for k in W if k.startswith("w.blocks."))
    d = W["w.ln_post.weight"].shape[0]
    return n_layer, d // 64


def _gelu_torch(kind):
    """The GELU applied at a conv or MLP point: "erf" is torch's exact GELU
    (npu_whisper_encoder.py:284-287); "poly4" is the reference's poly4 GELU
    on an fp32 input (g4f: rounded to bf16 RNE, then evaluated with RNE,
    gelu_row4f.cc:58-84), i.e. what its callers get from ``E.gelu = rt.gelu``
    (GELU_OP g4r on the fp32 array, rawxrt.py:546-565) and from the device
    MLP's g4f (rawxrt.py:457); the result is a bf16 value."""
    import torch
    import torch.nn.functional as F
    from . import bf16 as B
    if kind == "erf":
        return F.gelu
    if kind != "poly4":
        raise ValueError(f"unknown GELU {kind!r}")

    def poly4(x):
        bits = R.gelu_poly4(x.numpy(), mode="rne", f32_input=True)
        return torch.from_numpy(B.to_f32(bits).reshape(x.shape))
    return poly4


def encoder_torch(W, mel, n_layer=None, n_head=None, conv_gelu="erf", mlp_gelu="erf"):
    """mel fp32 [n_mels, T] or [B, n_mels, T] -> fp32 [ctx, d] or [B, ctx, d].
    conv_gelu / mlp_gelu: "erf" (default) or "poly4" (see _gelu_torch)."""
    import torch
    import torch.nn.functional as F
    gc, gm = _gelu_torch(conv_gelu), _gelu_torch(mlp_gelu)

    nl, nh = geometry(W)
    n_layer = n_layer or nl
    n_head = n_head or nh
    t = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
         for k, v in W.items() if isinstance(v, np.ndarray)}
    x = torch.from_numpy(np.ascontiguousarray(mel, dtype=np.float32))
    squeeze = x.dim() == 2
    if squeeze:
        x = x[None]
    with torch.no_grad():
        x = gc(F.conv1d(x, t["w.conv1.weight"], t["w.conv1.bias"], padding=1))
        x = gc(F.conv1d(x, t["w.conv2.weight"], t["w.conv2.bias"], stride=2, padding=1))
        x = x.permute(0, 2, 1)
        Bn, ctx, d = x.shape
        x = x + t["w.positional_embedding"][:ctx]
        hd = d // n_head
        scale = hd ** -0.25
        for L in range(n_layer):
            p = f"w.blocks.{L}."
            h = F.layer_norm(x, (d,), t[p + "attn_ln.weight"], t[p + "attn_ln.bias"], 1e-5)
            q = F.linear(h, t[p + "attn.query.weight"], t[p + "attn.query.bias"])
            k = F.linear(h, t[p + "attn.key.weight"])
            v = F.linear(h, t[p + "attn.value.weight"], t[p + "attn.value.bias"])
            q = q.view(Bn, ctx, n_head, hd).permute(0, 2, 1, 3) * scale
            k = k.view(Bn, ctx, n_head, hd).permute(0, 2, 3, 1) * scale
            v = v.view(Bn, ctx, n_head, hd).permute(0, 2, 1, 3)
            w = torch.softmax(q @ k, dim=-1)
            o = (w @ v).permute(0, 2, 1, 3).reshape(Bn, ctx, d)
            x = x + F.linear(o, t[p + "attn.out.weight"], t[p + "attn.out.bias"])
            h = F.layer_norm(x, (d,), t[p + "mlp_ln.weight"], t[p + "mlp_ln.bias"], 1e-5)
            f = gm(F.linear(h, t[p + "mlp.0.weight"], t[p + "mlp.0.bias"]))
            x = x + F.linear(f, t[p + "mlp.2.weight"], t[p + "mlp.2.bias"])
        x = F.layer_norm(x, (d,), t["w.ln_post.weight"], t["w.ln_post.bias"], 1e-5)
    out = x.numpy().astype(np.float32)
    return out[0] if squeeze else out


# ----------------------------------------------------------------- numpy twin

def im2col(x, kernel, stride, pad):
    """x (C, T) -> (T_out, C*kernel); column c*kernel + j pairs with conv weight
    element (c, j) (npu_whisper_encoder.py:422-431)."""
    C, T = x.shape
    xp = np.zeros((C, T + 2 * pad), dtype=x.dtype)
    xp[:, pad:pad + T] = x
    T_out = (T + 2 * pad - kernel) // stride + 1
    cols = np.empty((T_out, C * kernel), dtype=x.dtype)
    for j in range(kernel):
        cols[:, j::kernel] = xp[:, j:j + (T_out - 1) * stride + 1:stride].T
    return cols


def _ln32(x, w, b, eps=1e-5):
    mu = x.mean(axis=-1, keepdims=True)
    v = x.var(axis=-1, keepdims=True)
    return ((x - mu) / np.sqrt(v + eps) * w + b).astype(np.float32)


def _softmax32(x):
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=-1, keepdims=True)


def encoder_numpy(W, mel, n_layer=None, n_head=None):
    """fp32 numpy restatement of npu_whisper_encoder.py:436-541 (one sample)."""
    nl, nh = geometry(W)
    n_layer = n_layer or nl
    n_head = n_head or nh
    g = R.gelu_erf_as_f32
    f32 = np.float32
    c1w = W["w.conv1.weight"].astype(f32)
    O, C, KS = c1w.shape
    x = im2col(mel.astype(f32), KS, 1, 1) @ c1w.reshape(O, C * KS).T + W["w.conv1.bias"]
    x = g(x)
    c2w = W["w.conv2.weight"].astype(f32)
    O2, C2, KS2 = c2w.shape
    x = im2col(np.ascontiguousarray(x.T), KS2, 2, 1) @ c2w.reshape(O2, C2 * KS2).T \
        + W["w.conv2.bias"]
    x = g(x)
    x = (x + W["w.positional_embedding"][:x.shape[0]]).astype(f32)
    ctx, d = x.shape
    hd = d // n_head
    scale = f32(hd ** -0.25)
    for L in range(n_layer):
        p = f"w.blocks.{L}."
        h = _ln32(x, W[p + "attn_ln.weight"], W[p + "attn_ln.bias"])
        q = h @ W[p + "attn.query.weight"].T + W[p + "attn.query.bias"]
        k = h @ W[p + "attn.key.weight"].T
        v = h @ W[p + "attn.value.weight"].T + W[p + "attn.value.bias"]
        o = np.empty_like(q)
        for hh in range(n_head):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = (q[:, sl] * scale) @ (k[:, sl].T * scale)
            o[:, sl] = _softmax32(s) @ v[:, sl]
        x = (x + o @ W[p + "attn.out.weight"].T + W[p + "attn.out.bias"]).astype(f32)
        h = _ln32(x, W[p + "mlp_ln.weight"], W[p + "mlp_ln.bias"])
        f = g((h @ W[p + "mlp.0.weight"].T + W[p + "mlp.0.bias"]).astype(f32))
        x = (x + f @ W[p + "mlp.2.weight"].T + W[p + "mlp.2.bias"]).astype(f32)
    return _ln32(x, W["w.ln_post.weight"], W["w.ln_post.bias"])

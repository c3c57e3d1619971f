"""int8 quantised matmul and encoder restated on the CPU (test oracle only).

Restates the reference's quantised matmul, q_matmul_factory in
bench/probe_int8_decode.py:48-74:
  sa = max|A_row| / 127 per token (:58-59; rows of zeros get 1)
  sw = max|B_col| / 127 per output channel ("perchan", :62-63) or one
       max|B| / 127 for the tensor ("pertensor", :60-61); zeros get 1
  qa = rint(A / sa), qb = rint(B / sw) as int8 (:65-66; numpy rint: round
       half to even), all in float32
  r  = (qa @ qb exact, then float32) * sa * sw, then + bias (:67-73)
and the encoder the probe runs with it: encoder(W, mel, q_matmul,
np_matmul, fold_bias=False) (:143-145), i.e. every conv, projection and
MLP GEMM of npu_whisper_encoder.py:436-541 quantised (290 GEMMs at
large-v3), attention in fp32. The integer product is formed in float64,
which is exact for int8 operands at these K (|sum| < 2^53).

encoder_int8 uses torch's exact erf GELU and fp32 LayerNorm like
oracle.encoder.encoder_torch (the probe's numpy encoder uses the A&S erf,
within 1.5e-7 of it).
"""
import numpy as np


def quantize_rows(x):
    """Per-row (per-token) int8: -> (q int8, scale float32 [rows])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = (np.abs(x).max(axis=1) / np.float32(127.0)).astype(np.float32)
    s[s == 0] = 1.0
    q = np.rint(x / s[:, None]).astype(np.int8)
    return q, s


def quantize_cols(B, per_tensor=False):
    """weight_T B [K, N] per output channel (column) or per tensor:
    -> (q int8 [K, N], scale float32 [N])."""
    B = np.ascontiguousarray(B, dtype=np.float32)
    if per_tensor:
        s = np.full(B.shape[1], np.abs(B).max() / np.float32(127.0), np.float32)
    else:
        s = (np.abs(B).max(axis=0) / np.float32(127.0)).astype(np.float32)
    s[s == 0] = 1.0
    q = np.rint(B / s[None, :]).astype(np.int8)
    return q, s


def int_matmul(qa, qb):
    """Exact integer product of int8 matrices, as float64 (torch if present,
    for speed; numpy otherwise)."""
    try:
        import torch
        return (torch.from_numpy(qa.astype(np.float64)) @
                torch.from_numpy(qb.astype(np.float64))).numpy()
    except ImportError:  # pragma: no cover
        return qa.astype(np.float64) @ qb.astype(np.float64)


def q_matmul(A, B, bias=None, mode="perchan"):
    """The reference's q_matmul(A, B, bias) for mode perchan / pertensor / fp32."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    if mode == "fp32":
        r = A @ B
        return r if bias is None else r + bias
    qa, sa = quantize_rows(A)
    qb, sw = quantize_cols(B, per_tensor=(mode == "pertensor"))
    r = int_matmul(qa, qb).astype(np.float32)
    r = r * sa[:, None] * sw[None, :]
    return r if bias is None else (r + bias).astype(np.float32)


def _im2col(x, stride):
    """x (C, T) -> (T_out, 3 C), column c*3 + j = x[c, stride t - 1 + j]
    (npu_whisper_encoder.py:422-431, kernel 3, padding 1)."""
    C, T = x.shape
    xp = np.zeros((C, T + 2), np.float32)
    xp[:, 1:T + 1] = x
    T_out = (T + 2 - 3) // stride + 1
    cols = np.empty((T_out, C * 3), np.float32)
    for j in range(3):
        cols[:, j::3] = xp[:, j:j + (T_out - 1) * stride + 1:stride].T
    return cols


def encoder_int8(W, mel, mode="perchan", n_layer=None, n_head=None):
    """One sample: mel fp32 [n_mels, T] -> fp32 [ctx, d], every GEMM through
    q_matmul(mode) (bias added after, fold_bias=False)."""
    import torch
    import torch.nn.functional as F
    from .encoder import geometry

    nl, nh = geometry(W)
    n_layer = n_layer or nl
    n_head = n_head or nh
    f32 = np.float32
    mm = lambda A, B, b=None: q_matmul(A, B, b, mode)  # noqa: E731
    gelu = lambda x: F.gelu(torch.from_numpy(np.ascontiguousarray(x, f32))).numpy()  # noqa: E731

    def ln(x, w, b):
        return F.layer_norm(torch.from_numpy(np.ascontiguousarray(x, f32)), (x.shape[-1],),
                            torch.from_numpy(w.astype(f32)), torch.from_numpy(b.astype(f32)),
                            1e-5).numpy()

    c1 = W["w.conv1.weight"].astype(f32)
    O, C, _ = c1.shape
    x = gelu(mm(_im2col(np.asarray(mel, f32), 1), c1.reshape(O, C * 3).T) + W["w.conv1.bias"])
    c2 = W["w.conv2.weight"].astype(f32)
    O2, C2, _ = c2.shape
    x = gelu(mm(_im2col(np.ascontiguousarray(x.T), 2), c2.reshape(O2, C2 * 3).T)
             + W["w.conv2.bias"])
    x = (x + W["w.positional_embedding"][:x.shape[0]]).astype(f32)
    ctx, d = x.shape
    hd = d // n_head
    scale = hd ** -0.25
    for L in range(n_layer):
        p = f"w.blocks.{L}."
        h = ln(x, W[p + "attn_ln.weight"], W[p + "attn_ln.bias"])
        q = mm(h, W[p + "attn.query.weight"].T) + W[p + "attn.query.bias"]
        k = mm(h, W[p + "attn.key.weight"].T)
        v = mm(h, W[p + "attn.value.weight"].T) + W[p + "attn.value.bias"]
        qt = torch.from_numpy(np.ascontiguousarray(q, f32)).view(ctx, n_head, hd).permute(1, 0, 2)
        kt = torch.from_numpy(np.ascontiguousarray(k, f32)).view(ctx, n_head, hd).permute(1, 2, 0)
        vt = torch.from_numpy(np.ascontiguousarray(v, f32)).view(ctx, n_head, hd).permute(1, 0, 2)
        w = torch.softmax((qt * scale) @ (kt * scale).contiguous(), dim=-1)
        o = (w @ vt).permute(1, 0, 2).reshape(ctx, d).numpy()
        x = (x + mm(o, W[p + "attn.out.weight"].T) + W[p + "attn.out.bias"]).astype(f32)
        h = ln(x, W[p + "mlp_ln.weight"], W[p + "mlp_ln.bias"])
        f = gelu(mm(h, W[p + "mlp.0.weight"].T) + W[p + "mlp.0.bias"])
        x = (x + mm(f, W[p + "mlp.2.weight"].T) + W[p + "mlp.2.bias"]).astype(f32)
    return ln(x, W["w.ln_post.weight"], W["w.ln_post.bias"])

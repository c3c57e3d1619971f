"""Drop-in for the reference's model module src/npu_whisper_encoder.py.

``encoder(W, mel, mm, attn_mm, n_layer=4, n_head=6, prof=None, fused_gelu=False,
npu_softmax=False, attn_fn=None, mlp_fn=None, fold_bias=True)`` keeps the
signature of npu_whisper_encoder.py:436-541. The plugs must be a HipRT's
(``rt.matmul``, ``rt.attn_chain``, ``rt.mlp``) -- there is no CPU
backend, so a plug from anywhere else raises TypeError. Two device paths:

* the whole forward as one hipGraph over device-resident weights
  (``HipRT.encoder_forward`` -> libwxhip wxh_encoder_forward), taken while
  ``rt.graph_ok``/``chain_ok``/``mlp_ok`` hold and the plugs are rt's own;
* op by op, following the reference's dataflow line for line (conv GEMMs,
  per-layer LN -> q/k/v GEMMs -> attn_fn -> out GEMM -> LN -> MLP), each op a
  libwxhip launch, residual adds on the returned fp32 arrays as the
  reference does (npu_whisper_encoder.py:512-527). This path serves custom
  plugs and the fallback contract: when a stage fails, its flag is cleared,
  ``rt.fallbacks`` records why, and the next device path runs.

GELU: conv GELUs are the exact erf GELU (the reference's numpy ``gelu``,
:284-300). The MLP GELU is the exact erf GELU unless the device MLP plug is
used (``mlp_fn=rt.mlp``), which follows ``HipRT.GELU_F32_OP`` -- default
"g4f", the reference's poly4 (rawxrt.py:457), or "erf".

The module-level helpers keep the reference's names; ``layer_norm``,
``gelu`` and ``softmax`` run on the GPU (numpy in, numpy out).
"""
import time

import numpy as np

from . import _lib as L

CPU_PROF = {}
NEG = -30000.0          # the reference's bf16-safe -inf for padded softmax columns
MAX_GEMM_N = 4096       # fc1 chunking threshold of prepare_mlp_chunks (:358-406)
_ZERO_BIAS = {}
_DEV = None


def _dev():
    global _DEV
    if _DEV is None:
        from .device import Device
        _DEV = Device(0)
    return _DEV


def _timed(name, fn, *a, **kw):
    t0 = time.perf_counter()
    r = fn(*a, **kw)
    CPU_PROF[name] = CPU_PROF.get(name, 0.0) + (time.perf_counter() - t0)
    return r


# ---------------------------------------------------------------- device ops

def layer_norm(x, w, b, eps=1e-5):
    """(x - mean)/sqrt(var + eps) * w + b over the last axis, on the GPU, fp32
    in and out (npu_whisper_encoder.py:278-281)."""
    import torch
    d = _dev()
    a = np.ascontiguousarray(x, dtype=np.float32)
    t = torch.from_numpy(a.reshape(-1, a.shape[-1])).to(d.device)
    g = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32)).to(d.device)
    bb = torch.from_numpy(np.ascontiguousarray(b, dtype=np.float32)).to(d.device)
    y = d.layer_norm(t, g, bb, eps=eps, out_dtype=torch.float32)
    return y.cpu().numpy().reshape(a.shape)


def gelu(x):
    """Exact erf GELU on the GPU, fp32 in, bf16-rounded values out as fp32
    (npu_whisper_encoder.py:284-300 computes the same function in numpy)."""
    import torch
    d = _dev()
    a = np.ascontiguousarray(x, dtype=np.float32)
    t = torch.from_numpy(a.reshape(1, -1)).to(d.device)
    return d.gelu(t, L.WXH_GELU_ERF).float().cpu().numpy().reshape(a.shape)


def softmax(x):
    """Row softmax over the last axis on the GPU (npu_whisper_encoder.py:416-419)."""
    import torch
    d = _dev()
    a = np.ascontiguousarray(x, dtype=np.float32)
    t = torch.from_numpy(a.reshape(-1, a.shape[-1])).to(d.device)
    return d.softmax_rows(d.to_bf16(t)).float().cpu().numpy().reshape(a.shape)


def npu_softmax_stack(mats):
    """All heads' softmax in one launch (npu_whisper_encoder.py:341-357)."""
    mats = list(mats)
    L0, L1 = mats[0].shape
    out = softmax(np.stack(mats).reshape(-1, L1)).reshape(len(mats), L0, L1)
    return [out[i] for i in range(len(mats))]


# ---------------------------------------------------------------- data helpers

def im2col(x, kernel, stride, pad):
    """x (C, T) -> (T_out, C*kernel), column c*kernel + j pairs with conv weight
    element (c, j) (npu_whisper_encoder.py:422-431). Pure data movement."""
    C, T = x.shape
    xp = np.zeros((C, T + 2 * pad), dtype=x.dtype)
    xp[:, pad:pad + T] = x
    T_out = (T + 2 * pad - kernel) // stride + 1
    cols = np.empty((T_out, C * kernel), dtype=x.dtype)
    for j in range(kernel):
        cols[:, j::kernel] = xp[:, j:j + (T_out - 1) * stride + 1:stride].T
    return cols


def zero_bias(d):
    """A stable all-zero bias row for the bias-less key projection
    (npu_whisper_encoder.py:308-315)."""
    b = _ZERO_BIAS.get(d)
    if b is None:
        b = _ZERO_BIAS[d] = np.zeros(d, dtype=np.float32)
    return b


def prepare_mlp_chunks(W, n_layer, d, chunk=0):
    """Split every fc1 weight wider than MAX_GEMM_N into column chunks
    ``W[p + "mlp.0.parts"] = [(W1_T chunk, b1 chunk), ...]``, in place, as
    npu_whisper_encoder.py:361-406 does; returns the new arrays so the caller
    can register them. The GEMM here has no width limit; the chunks exist so
    the reference's callers (mlp_fn) see the structure they expect."""
    made = []
    for Li in range(n_layer):
        p = f"w.blocks.{Li}."
        W1, b1 = W[p + "mlp.0.weight_T"], W[p + "mlp.0.bias"]
        N = W1.shape[1]
        if chunk:
            width = chunk
        elif N <= MAX_GEMM_N:
            continue
        elif N % d == 0:
            width = d
        else:
            width = N // ((N + MAX_GEMM_N - 1) // MAX_GEMM_N)
        if N <= width:
            continue
        parts = []
        for j in range(0, N, width):
            wc = np.ascontiguousarray(W1[:, j:j + width])
            bc = np.ascontiguousarray(b1[j:j + width])
            parts.append((wc, bc))
            made += [wc, bc]
        W[p + "mlp.0.parts"] = parts
    return made


# ---------------------------------------------------------------- the encoder

def _runtime_of(fn):
    from .hiprt import HipRT
    # a HipRT's matmul, or a plug that carries its HipRT (wxhip.int8.q_matmul_factory)
    rt = getattr(fn, "__self__", None)
    if not isinstance(rt, HipRT):
        rt = getattr(fn, "rt", None)
    if not isinstance(rt, HipRT):
        raise TypeError("encoder(): mm must be a HipRT's matmul (the encoder runs "
                        "on the GPU only; there is no numpy backend)")
    return rt


def _graph_eligible(rt, mm, attn_mm, attn_fn, mlp_fn, fused_gelu):
    own = (mm == rt.matmul and attn_mm == rt.matmul
           and attn_fn in (None, rt.attn_chain) and mlp_fn in (None, rt.mlp))
    patched = any(k in vars(rt) for k in ("_attn_chain_dev", "_mlp_dev", "encoder_forward"))
    return (own and not patched and not fused_gelu and rt.graph_ok and rt.chain_ok
            and rt.mlp_ok)


def encoder(W, mel, mm, attn_mm, n_layer=4, n_head=6, prof=None,
            fused_gelu=False, npu_softmax=False, attn_fn=None,
            mlp_fn=None, fold_bias=True):
    """mel fp32 (n_mels, 2*ctx) -> features fp32 (ctx, d). See the module doc."""
    t_all = time.perf_counter()
    rt = _runtime_of(mm)
    d = W["w.conv1.weight"].shape[0]
    if d != n_head * 64:
        raise ValueError(f"n_head={n_head} does not match d_model={d} (n_head = d/64)")
    out = None
    if _graph_eligible(rt, mm, attn_mm, attn_fn, mlp_fn, fused_gelu):
        mlp_gelu = "erf"
        if mlp_fn is not None and W.get("w.blocks.0.mlp.0.parts") is not None:
            mlp_gelu = "poly4" if rt.GELU_F32_OP == "g4f" else "erf"
        try:
            out = rt.encoder_forward(W, mel, n_layer=n_layer, mlp_gelu=mlp_gelu)
        except Exception as exc:
            rt.graph_ok = False
            msg = f"encoder graph -> op-by-op path: {type(exc).__name__}: {exc}"
            rt.fallbacks.append(msg)
            print(f"[hiprt] {msg}", flush=True)
    if out is None:
        out = _encoder_ops(W, mel, mm, attn_mm, n_layer, n_head, npu_softmax,
                           attn_fn, mlp_fn, fold_bias)
    if prof is not None:
        prof["total"] = time.perf_counter() - t_all
    return out


def _encoder_ops(W, mel, mm, attn_mm, n_layer, n_head, npu_softmax, attn_fn,
                 mlp_fn, fold_bias):
    """The reference's dataflow (npu_whisper_encoder.py:440-539), op by op."""
    g = globals()["gelu"]           # monkeypatchable, as E.gelu = rt.gelu
    c1w = W["w.conv1.weight"]
    O, Cc, KS = c1w.shape
    A = _timed("im2col", im2col, np.asarray(mel, np.float32), KS, 1, 1)
    x = mm(A, np.ascontiguousarray(c1w.reshape(O, Cc * KS).T)) + W["w.conv1.bias"]
    x = _timed("gelu", g, x)
    c2w = W["w.conv2.weight"]
    O2, C2, KS2 = c2w.shape
    A = _timed("im2col", im2col, np.ascontiguousarray(x.T), KS2, 2, 1)
    x = mm(A, np.ascontiguousarray(c2w.reshape(O2, C2 * KS2).T)) + W["w.conv2.bias"]
    x = _timed("gelu", g, x)
    x = x + W["w.positional_embedding"][:x.shape[0]]
    ctx, d = x.shape
    hd = d // n_head
    scale = hd ** -0.25

    def wT(key):
        got = W.get(key + "_T")
        if got is None:
            got = W[key + "_T"] = np.ascontiguousarray(W[key].T)
        return got

    for Li in range(n_layer):
        p = f"w.blocks.{Li}."
        h = _timed("layernorm", layer_norm, x, W[p + "attn_ln.weight"], W[p + "attn_ln.bias"])
        ak = f"L{Li}.attn_ln"
        q = mm(h, wT(p + "attn.query.weight"), akey=ak, bias=W[p + "attn.query.bias"])
        k = mm(h, wT(p + "attn.key.weight"), akey=ak, bias=zero_bias(d))
        v = mm(h, wT(p + "attn.value.weight"), akey=ak, bias=W[p + "attn.value.bias"])
        if attn_fn is not None:
            o = _timed("attn_chain", attn_fn, q, k, v, n_head, scale)
        else:
            o = np.empty_like(q)
            wgts = []
            for hh in range(n_head):
                sl = slice(hh * hd, (hh + 1) * hd)
                qh = np.ascontiguousarray(q[:, sl] * scale)
                kh = np.ascontiguousarray(k[:, sl].T) * scale
                wgts.append(attn_mm(qh, kh))
            wgts = npu_softmax_stack(wgts)
            for hh in range(n_head):
                sl = slice(hh * hd, (hh + 1) * hd)
                o[:, sl] = attn_mm(wgts[hh], np.ascontiguousarray(v[:, sl]))
        x = x + mm(o, wT(p + "attn.out.weight"), bias=W[p + "attn.out.bias"])
        h = _timed("layernorm", layer_norm, x, W[p + "mlp_ln.weight"], W[p + "mlp_ln.bias"])
        parts = W.get(p + "mlp.0.parts")
        if parts is not None and mlp_fn is not None:
            x = x + _timed("mlp_dev", mlp_fn, h, parts, wT(p + "mlp.2.weight"),
                           f"L{Li}.mlp_ln") + W[p + "mlp.2.bias"]
            continue
        if parts is not None:
            ak = f"L{Li}.mlp_ln"
            f = _timed("gelu", g, np.concatenate(
                [mm(h, wc, akey=ak) + bc for wc, bc in parts], axis=1))
        else:
            f = _timed("gelu", g, mm(h, wT(p + "mlp.0.weight"), bias=W[p + "mlp.0.bias"]))
        x = x + mm(f, wT(p + "mlp.2.weight"), bias=W[p + "mlp.2.bias"])
    return layer_norm(x, W["w.ln_post.weight"], W["w.ln_post.bias"])

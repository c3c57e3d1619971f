"""Drop-in for the reference's model module src/npu_whisper_encoder.py.

``encoder(W, mel, mm, attn_mm, n_layer=4, n_head=6, prof=None, fused_gelu=False,
npu_softmax=False, attn_fn=None, mlp_fn=None, fold_bias=True)`` keeps the
signature and the result of npu_whisper_encoder.py:436-541. The plugs must
belong to a HipRT (``rt.matmul``, ``rt.attn_chain``, ``rt.mlp``): there is no
CPU backend, so a plug from anywhere else raises TypeError.

Two device paths compute the same function:

* **graph**: the whole forward as one hipGraph over device-resident weights
  (``HipRT.encoder_forward`` -> wxh_encoder_forward). Taken when every plug is
  rt's own, rt's flags (``graph_ok``, ``chain_ok``, ``mlp_ok``) hold, and the
  module's ``gelu`` is either its own or ``rt.gelu`` with a GELU the graph
  builds (see ``_plan``).
* **op by op**: each step of the reference's dataflow as its own libwxhip
  launch (``_OpByOp``), host fp32 arrays between steps, residual adds on the
  host. It serves custom plugs, a patched ``gelu`` the graph cannot express,
  and the fallback contract: a failing stage clears its flag, records why in
  ``rt.fallbacks`` and the next device path runs.

GELU. The module's ``gelu`` is the exact erf GELU (the reference's numpy
``gelu``, :284-300, computes the same function with A&S's erf). Callers may
replace it, as the reference's do with ``E.gelu = rt.gelu``
(bench/run_raw_encoder.py:82-83; serve/npu_stt_server.py:203); the
replacement then applies to both conv GELUs and to the host-side MLP GELU,
exactly as in the reference. The device MLP plug (``mlp_fn=rt.mlp`` with fc1
chunks) uses ``HipRT.GELU_F32_OP`` instead (default "g4f", the reference's
poly4, rawxrt.py:457). ``fused_gelu=True`` (the reference's fc1 GEMM with the
GELU inside the core, :93-107) is the fc1 GEMM with the erf-GELU epilogue.

The module-level helpers keep the reference's names; ``layer_norm``,
``gelu`` and ``softmax`` run on the GPU (numpy in, numpy out).
"""
import functools
import time

import numpy as np

from . import _lib as L

CPU_PROF = {}
NEG = -30000.0          # the reference's bf16-safe -inf for padded softmax columns
MAX_GEMM_N = 4096       # fc1 chunking threshold of prepare_mlp_chunks (:358-406)
_DEV = None


def _dev():
    global _DEV
    if _DEV is None:
        from .device import Device
        _DEV = Device(0)
    return _DEV


def _timed(name, fn, *a, **kw):
    t0 = time.perf_counter()
    try:
        return fn(*a, **kw)
    finally:
        CPU_PROF[name] = CPU_PROF.get(name, 0.0) + time.perf_counter() - t0


# ---------------------------------------------------------------- device ops

def _to_dev(a, dtype=np.float32):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).to(_dev().device)


def layer_norm(x, w, b, eps=1e-5):
    """(x - mean)/sqrt(var + eps) * w + b over the last axis, on the GPU, fp32
    in and out (npu_whisper_encoder.py:278-281)."""
    import torch
    shape = np.shape(x)
    t = _to_dev(x).reshape(-1, shape[-1])
    y = _dev().layer_norm(t, _to_dev(w), _to_dev(b), eps=eps, out_dtype=torch.float32)
    return y.cpu().numpy().reshape(shape)


def gelu(x):
    """Exact erf GELU on the GPU, fp32 in, bf16-rounded values out as fp32
    (npu_whisper_encoder.py:284-300 computes the same function in numpy)."""
    shape = np.shape(x)
    y = _dev().gelu(_to_dev(x).reshape(1, -1), L.WXH_GELU_ERF)
    return y.float().cpu().numpy().reshape(shape)


_OWN_GELU = gelu


def softmax(x):
    """Row softmax over the last axis on the GPU (npu_whisper_encoder.py:416-419)."""
    shape = np.shape(x)
    d = _dev()
    p = d.softmax_rows(d.to_bf16(_to_dev(x).reshape(-1, shape[-1])))
    return p.float().cpu().numpy().reshape(shape)


def npu_softmax_stack(mats):
    """Every head's row softmax in one launch (npu_whisper_encoder.py:341-357)."""
    mats = [np.asarray(m, np.float32) for m in mats]
    flat = softmax(np.concatenate(mats, axis=0))
    bounds = np.cumsum([0] + [m.shape[0] for m in mats])
    return [flat[a:b] for a, b in zip(bounds[:-1], bounds[1:])]


# ---------------------------------------------------------------- data helpers

def im2col(x, kernel, stride, pad):
    """x (C, T) -> (T_out, C*kernel) with column c*kernel + j holding
    x[c, t*stride + j - pad] (zero outside [0, T)), so that the product with
    conv_weight.reshape(O, C*kernel).T is the conv1d (the layout of
    npu_whisper_encoder.py:422-431). Pure data movement."""
    xp = np.pad(x, ((0, 0), (pad, pad)))
    win = np.lib.stride_tricks.sliding_window_view(xp, kernel, axis=1)[:, ::stride]
    # win: (C, T_out, kernel) -> (T_out, C, kernel), flattened over (C, kernel)
    return np.ascontiguousarray(win.transpose(1, 0, 2)).reshape(win.shape[1], -1)


@functools.lru_cache(maxsize=None)
def zero_bias(d):
    """The all-zero bias of the bias-less key projection. One array per
    width, the same object on every call (npu_whisper_encoder.py:308-315
    relies on that identity so the weight cache keys stay stable); it is
    read-only, since every caller shares it."""
    z = np.zeros(d, dtype=np.float32)
    z.setflags(write=False)
    return z


def _fc1_chunk_width(n_out, d, chunk):
    """Column width the reference splits an fc1 of n_out outputs into, or
    None when it stays whole (npu_whisper_encoder.py:383-396)."""
    if chunk:
        width = chunk
    elif n_out <= MAX_GEMM_N:
        return None
    elif n_out % d == 0:
        width = d
    else:
        pieces = -(-n_out // MAX_GEMM_N)
        width = n_out // pieces
    return width if n_out > width else None


def prepare_mlp_chunks(W, n_layer, d, chunk=0):
    """Split every fc1 weight wider than MAX_GEMM_N (or than `chunk`, when
    given) into column chunks, in place: ``W[p + "mlp.0.parts"]`` becomes a
    list of (W1_T columns, b1 entries) pairs covering the outputs left to
    right. Returns the new arrays (each chunk's weight, then its bias) so the
    caller can register them. Same rule and result as
    npu_whisper_encoder.py:364-406; the GEMM here has no width limit, so the
    chunks only keep the structure the reference's MLP plug expects."""
    created = []
    for layer in range(n_layer):
        prefix = f"w.blocks.{layer}."
        w1t, b1 = W[prefix + "mlp.0.weight_T"], W[prefix + "mlp.0.bias"]
        width = _fc1_chunk_width(w1t.shape[1], d, chunk)
        if width is None:
            continue
        starts = range(0, w1t.shape[1], width)
        parts = [(w1t[:, s:s + width].copy(), b1[s:s + width].copy()) for s in starts]
        W[prefix + "mlp.0.parts"] = parts
        created.extend(a for pair in parts for a in pair)
    return created


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


def _gelu_kind(rt, g):
    """The GELU a module-level ``gelu`` computes, as the graph names it
    ("erf" or "poly4"), or None when the graph cannot run it."""
    from .hiprt import HipRT
    if g is _OWN_GELU:
        return "erf"
    if getattr(g, "__self__", None) is rt and getattr(g, "__func__", None) is HipRT.gelu:
        # rt.gelu: rt.GELU_OP on the fp32 input; g4r and g4f both round the
        # input to bf16 (RNE) and evaluate poly4 with RNE, as the graph's
        # poly4 epilogues do; the truncating g4 has no graph form
        return {"g4r": "poly4", "g4f": "poly4", "erf": "erf"}.get(rt.GELU_OP)
    return None


def _plan(rt, W, mm, attn_mm, attn_fn, mlp_fn, fused_gelu):
    """(conv_gelu, mlp_gelu) of the graph forward when it computes what the
    reference would for these arguments, else None (run op by op)."""
    own_plugs = (mm == rt.matmul and attn_mm == rt.matmul
                 and attn_fn in (None, rt.attn_chain) and mlp_fn in (None, rt.mlp))
    overridden = {"_attn_chain_dev", "_mlp_dev", "encoder_forward"} & set(vars(rt))
    if not own_plugs or overridden or not (rt.graph_ok and rt.chain_ok and rt.mlp_ok):
        return None
    conv = _gelu_kind(rt, globals()["gelu"])
    if conv is None:
        return None
    if fused_gelu:
        mlp = "erf"
    elif mlp_fn is not None and W.get("w.blocks.0.mlp.0.parts") is not None:
        mlp = {"g4f": "poly4", "erf": "erf"}.get(rt.GELU_F32_OP)
    else:
        mlp = conv      # the reference applies the module's gelu to fc1's output
    return None if mlp is None else (conv, mlp)


def encoder(W, mel, mm, attn_mm, n_layer=4, n_head=6, prof=None,
            fused_gelu=False, npu_softmax=False, attn_fn=None,
            mlp_fn=None, fold_bias=True):
    """mel fp32 (n_mels, 2*ctx) -> features fp32 (ctx, d). See the module doc."""
    t_start = time.perf_counter()
    rt = _runtime_of(mm)
    d = W["w.conv1.weight"].shape[0]
    if d != n_head * 64:
        raise ValueError(f"n_head={n_head} does not match d_model={d} (n_head = d/64)")
    feats = None
    plan = _plan(rt, W, mm, attn_mm, attn_fn, mlp_fn, fused_gelu)
    if plan is not None:
        try:
            feats = rt.encoder_forward(W, mel, n_layer=n_layer, mlp_gelu=plan[1],
                                       conv_gelu=plan[0])
        except Exception as exc:
            rt._retire("graph_ok", "whole-encoder hipGraph", "op-by-op launches", exc)
    if feats is None:
        run = _OpByOp(W, rt, mm, attn_mm, n_head, fold_bias, globals()["gelu"])
        feats = run(np.asarray(mel, np.float32), n_layer, npu_softmax, attn_fn, mlp_fn,
                    fused_gelu)
    if prof is not None:
        prof["total"] = time.perf_counter() - t_start
    return feats


class _OpByOp:
    """The reference's encoder dataflow (npu_whisper_encoder.py:440-539) as
    one device launch per step: conv GEMMs with the module's gelu, then per
    block LN -> q/k/v GEMMs -> attention (the plug, or per-head score GEMMs,
    a softmax and P.V GEMMs) -> out GEMM and residual -> LN -> MLP and
    residual; ln_post last. Bias placement follows ``fold_bias`` as the
    reference does (folded: the GEMM adds it; else added on the host)."""

    def __init__(self, W, rt, mm, attn_mm, n_head, fold_bias, act):
        self.W, self.rt, self.mm, self.attn_mm = W, rt, mm, attn_mm
        self.n_head, self.fold, self.act = n_head, fold_bias, act

    def wt(self, name):
        """``name + "_T"`` (in, out), derived once, as :563-566 do."""
        key = name + "_T"
        if key not in self.W:
            self.W[key] = np.ascontiguousarray(self.W[name].T)
        return self.W[key]

    def conv(self, x_ct, name, stride):
        w = self.W[f"w.{name}.weight"]
        out_ch, in_ch, taps = w.shape
        cols = _timed("im2col", im2col, x_ct, taps, stride, 1)
        y = self.mm(cols, np.ascontiguousarray(w.reshape(out_ch, in_ch * taps).T))
        return _timed("gelu", self.act, y + self.W[f"w.{name}.bias"])

    def linear(self, x, name, akey=None, bias=None):
        """x . W_T (+ bias): handed to the GEMM when folding, added here
        otherwise. bias=False means no bias term at all."""
        wt = self.wt(f"{name}.weight")
        if bias is False:
            return self.mm(x, wt, akey=akey)
        if self.fold:
            return self.mm(x, wt, akey=akey, bias=bias)
        return self.mm(x, wt, akey=akey) + bias

    def heads(self, q, k, v, npu_softmax):
        """Per head: scores (q_h s)(k_h s)^T by attn_mm, softmax over all
        heads at once (npu_softmax) or head by head, then P_h v_h."""
        d = q.shape[1]
        hd = d // self.n_head
        s = hd ** -0.25
        cols = [slice(h * hd, (h + 1) * hd) for h in range(self.n_head)]
        scores = [self.attn_mm(np.ascontiguousarray(q[:, c] * s),
                               np.ascontiguousarray(k[:, c].T) * s) for c in cols]
        if npu_softmax:
            probs = npu_softmax_stack(scores)
        else:
            probs = [_timed("softmax", softmax, sc) for sc in scores]
        return np.concatenate([self.attn_mm(p, np.ascontiguousarray(v[:, c]))
                               for p, c in zip(probs, cols)], axis=1)

    def block(self, x, layer, npu_softmax, attn_fn, mlp_fn, fused_gelu):
        W, p = self.W, f"w.blocks.{layer}."
        d = x.shape[1]
        h = _timed("layernorm", layer_norm, x, W[p + "attn_ln.weight"], W[p + "attn_ln.bias"])
        ak = f"L{layer}.attn_ln"
        q = self.linear(h, p + "attn.query", ak, W[p + "attn.query.bias"])
        k = self.linear(h, p + "attn.key", ak, zero_bias(d) if self.fold else False)
        v = self.linear(h, p + "attn.value", ak, W[p + "attn.value.bias"])
        if attn_fn is not None:
            o = _timed("attn_chain", attn_fn, q, k, v, self.n_head, (d // self.n_head) ** -0.25)
        else:
            o = self.heads(q, k, v, npu_softmax)
        x = x + self.linear(o, p + "attn.out", None, W[p + "attn.out.bias"])

        h = _timed("layernorm", layer_norm, x, W[p + "mlp_ln.weight"], W[p + "mlp_ln.bias"])
        parts = W.get(p + "mlp.0.parts")
        b2 = W[p + "mlp.2.bias"]
        if fused_gelu:
            f = self.rt.matmul_gelu(h, self.wt(p + "mlp.0.weight"), W[p + "mlp.0.bias"])
        elif parts is not None and mlp_fn is not None:
            y = _timed("mlp_dev", mlp_fn, h, parts, self.wt(p + "mlp.2.weight"),
                       f"L{layer}.mlp_ln")
            return x + y + b2
        elif parts is not None:
            ak = f"L{layer}.mlp_ln"
            fc1 = np.hstack([self.mm(h, wc, akey=ak) + bc for wc, bc in parts])
            f = _timed("gelu", self.act, fc1)
        else:
            fc1 = self.mm(h, self.wt(p + "mlp.0.weight")) + W[p + "mlp.0.bias"]
            f = _timed("gelu", self.act, fc1)
        return x + self.mm(f, self.wt(p + "mlp.2.weight")) + b2

    def __call__(self, mel, n_layer, npu_softmax, attn_fn, mlp_fn, fused_gelu):
        W = self.W
        x = self.conv(mel, "conv1", 1)
        x = self.conv(np.ascontiguousarray(x.T), "conv2", 2)
        x = x + W["w.positional_embedding"][:x.shape[0]]
        for layer in range(n_layer):
            x = self.block(x, layer, npu_softmax, attn_fn, mlp_fn, fused_gelu)
        return layer_norm(x, W["w.ln_post.weight"], W["w.ln_post.bias"])

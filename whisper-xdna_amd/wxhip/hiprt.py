"""HipRT: a drop-in for the reference's raw-XRT backend ``rawxrt.RawRT``.

Same method names, arguments and fallback contract as src/rawxrt.py, with the
device work done by libwxhip.so's gfx950 kernels instead of AIE overlays:

  matmul / mm_start / mm_finish   rawxrt.py:926-996   -> wxh_gemm_bf16
  register_weights                rawxrt.py:307-316   -> device bf16 cache
  attn_chain / _attn_chain_dev    rawxrt.py:813-891   -> wxh_attention (fused)
  _attn_host                      rawxrt.py:893-918   -> per-head GEMM + softmax + GEMM
  mlp / _mlp_dev                  rawxrt.py:436-544   -> fc1 GEMM(+GELU epilogue) -> fc2 GEMM
  gelu                            rawxrt.py:546-565   -> wxh_gelu (GELU_OP, default g4r)
  softmax_stack                   rawxrt.py:569-585   -> wxh_softmax_rows
  rowop                           rawxrt.py:384-400   -> the op-code table of compile_rowop.py:12-19

Inputs and outputs are host numpy fp32 arrays as in the reference (bf16
buffers as uint16 bit arrays); everything between upload and download runs on
the GPU. There is no CPU compute path: when a device stage raises, the runtime
clears the stage's flag, records the reason in ``fallbacks`` and takes the
next DEVICE path, exactly as the reference steps fused -> chain -> host-routed
(rawxrt.py:822-838). If the last device path fails too, the error propagates.

Differences kept on purpose (numerics only improve):
* the bias is added in fp32 in the GEMM epilogue; the reference folds it into
  the GEMM as a bf16-rounded row of B (rawxrt.py:352-371);
* q and k are not pre-scaled by hd^-1/4 in bf16; the attention kernel applies
  scale^2 to the fp32 scores (attn_mmul.cc:22-24 does the same);
* rowop() returns a fresh array, not a view aliasing device memory that the
  next launch overwrites (rawxrt.py:335-339).
"""
import os
import time

import numpy as np

from . import _lib as L
from . import rowops as R
from .device import Device

PROF = {}


def _t(name, dt):
    PROF[name] = PROF.get(name, 0.0) + dt


def _torch():
    import torch
    return torch


def _pad8(k):
    return (k + 7) // 8 * 8


class HipRT:
    # ONE GELU op for rt.gelu, as the reference keeps one overlay
    # (rawxrt.py:409-434); g4r = poly4 with RNE.
    GELU_OP = os.environ.get("GELU_OP", "g4r")
    # the device MLP's fp32-input GELU (rawxrt.py:457); "erf" selects the
    # exact GELU instead of the reference's g4f poly4
    GELU_F32_OP = os.environ.get("GELU_F32_OP", "g4f")
    SM_OP = os.environ.get("SM_OP", "s3")

    def __init__(self, device=0, max_ctx=6):
        self.dev = Device(device)
        self.max_ctx = max_ctx
        self._live = {}        # no hw_contexts exist here; kept for callers that count them
        self._known = {}       # id(weight array) -> key
        self._keep = []
        self._wdev = {}        # key -> device bf16 [N, K]
        self._bdev = {}        # id(bias) -> device fp32
        self._encoders = {}    # (id(W), n_layer, mlp_gelu) -> HipEncoder
        self.calls = 0
        self.ctx_creates = 0
        self.evictions = 0
        self.graph_ok = True   # whole-forward hipGraph (wxhip.encoder)
        self.chain_ok = True
        self.fused_ok = True
        self.mlp_ok = True
        self.softmax_ok = True
        self.fallbacks = []

    # -- weights -------------------------------------------------------------
    def register_weights(self, arrays):
        """Name arrays that never change so their device copy is made once
        (keyed by id(), references held for the runtime's lifetime, as
        rawxrt.py:307-316)."""
        for a in arrays:
            if id(a) not in self._known:
                self._known[id(a)] = f"w{len(self._keep)}"
                self._keep.append(a)

    def _weight_dev(self, B, bkey=None):
        """Host fp32 B [K, N] (a *.weight_T) -> device bf16 [N, K]."""
        torch = _torch()
        key = bkey if bkey is not None else self._known.get(id(B))
        if key is not None and key in self._wdev:
            return self._wdev[key]
        t0 = time.perf_counter()
        src = torch.from_numpy(np.ascontiguousarray(B, dtype=np.float32)).to(self.dev.device)
        K, N = src.shape
        # the GEMM wants K % 8 == 0: zero-pad K (A is padded the same way)
        w = torch.zeros(N, _pad8(K), dtype=torch.bfloat16, device=self.dev.device)
        self.dev.to_bf16(src, transpose=True, out=w[:, :K])
        if key is not None:
            self._wdev[key] = w
        _t("upload_B", time.perf_counter() - t0)
        return w

    def _bias_dev(self, bias):
        torch = _torch()
        if bias is None:
            return None
        got = self._bdev.get(id(bias))
        if got is not None and got[0] is bias:
            return got[1]
        d = torch.from_numpy(np.ascontiguousarray(bias, dtype=np.float32)).to(self.dev.device)
        if id(bias) in self._known:
            self._bdev[id(bias)] = (bias, d)
        return d

    def _act_dev(self, A):
        """Host fp32 activation -> device bf16 (RNE on the device)."""
        torch = _torch()
        t0 = time.perf_counter()
        src = torch.from_numpy(np.ascontiguousarray(A, dtype=np.float32)).to(self.dev.device)
        M, K = src.shape
        if K % 8:
            a = torch.zeros(M, _pad8(K), dtype=torch.bfloat16, device=self.dev.device)
            self.dev.to_bf16(src, out=a[:, :K])
        else:
            a = self.dev.to_bf16(src)
        _t("upload_A", time.perf_counter() - t0)
        return a

    # -- GEMM ------------------------------------------------------------------
    def mm_start(self, A, B, akey=None, bkey=None, bias=None, cbo=None):
        """Upload operands and launch C = A.B (+bias); returns a handle for
        mm_finish. Launches are stream-ordered, so several may be in flight."""
        M, K = A.shape
        K2, N = B.shape
        if K != K2:
            raise ValueError(f"matmul: A {A.shape} and B {B.shape} disagree on K")
        a = self._act_dev(A)
        w = self._weight_dev(B, bkey)
        c = self.dev.gemm(a, w, self._bias_dev(bias), L.WXH_EPI_F32, out=cbo)
        self.calls += 1
        return (c, time.perf_counter())

    def mm_finish(self, h):
        c, t_sub = h
        t0 = time.perf_counter()
        out = c.cpu().numpy()
        _t("run+download", time.perf_counter() - t0)
        return out

    def matmul(self, A, B, akey=None, bkey=None, bias=None):
        """A (M,K) f32 @ B (K,N) f32 [+ bias] -> (M,N) f32; bf16 in, fp32 acc."""
        return self.mm_finish(self.mm_start(A, B, akey=akey, bkey=bkey, bias=bias))

    # -- element-wise ----------------------------------------------------------
    def rowop(self, op, buf_bf16, rows, cols):
        """Run row op `op` (compile_rowop.py:12-19 codes) over a (rows, cols)
        bf16 buffer (uint16 bits, numpy or torch); returns uint16 numpy."""
        torch = _torch()
        x = R.as_device_bf16(self.dev, buf_bf16, rows, cols)
        t0 = time.perf_counter()
        y = R.run_op(self.dev, op, x)
        out = R.bits_to_numpy(y)
        _t(f"{op}_run", time.perf_counter() - t0)
        del torch
        return out

    def gelu(self, x):
        """GELU over any shaped fp32 array via self.GELU_OP, returned as fp32
        (rawxrt.py:546-565; one op for every shape, no tiling needed)."""
        torch = _torch()
        flat = np.ascontiguousarray(x, dtype=np.float32).reshape(1, -1)
        src = torch.from_numpy(flat).to(self.dev.device)
        variant = R.GELU_VARIANT[self.GELU_OP]
        xin = src if self.GELU_OP in ("erf", "g4f") else self.dev.to_bf16(src)
        y = self.dev.gelu(xin, variant)
        return y.float().cpu().numpy().reshape(np.shape(x))

    def softmax_stack(self, mats):
        """Row softmax of every (L0, L1) head matrix in one launch."""
        torch = _torch()
        nh = len(mats)
        L0, L1 = mats[0].shape
        big = torch.from_numpy(np.ascontiguousarray(np.stack(mats), dtype=np.float32)
                               .reshape(nh * L0, L1)).to(self.dev.device)
        p = self.dev.softmax_rows(self.dev.to_bf16(big))
        f = p.float().cpu().numpy()
        return [f[i * L0:(i + 1) * L0] for i in range(nh)]

    # -- attention -------------------------------------------------------------
    def attn_chain(self, q, k, v, nh, scale):
        """o = concat_h softmax((q_h s)(k_h s)^T) v_h for s = scale (the
        reference's hd^-1/4). Fused kernel first, then the unfused device
        chain; each failure is recorded and retires only its own path."""
        if self.chain_ok:
            try:
                return self._attn_chain_dev(q, k, v, nh, scale)
            except Exception as exc:
                self.chain_ok = False
                msg = f"attention chain -> host path: {type(exc).__name__}: {exc}"
                self.fallbacks.append(msg)
                print(f"[hiprt] {msg}", flush=True)
        return self._attn_host(q, k, v, nh, scale)

    def attn_fused(self, q, k, v, nh, scale):
        return self._attn_chain_dev(q, k, v, nh, scale)

    def _attn_chain_dev(self, q, k, v, nh, scale):
        torch = _torch()
        ctx, d = q.shape
        if d != nh * 64:
            raise ValueError(f"attention: d={d} is not n_head*64 (n_head={nh})")
        t0 = time.perf_counter()
        dev = self.dev.device
        qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
                      for a in (q, k, v))
        Q, K, Vt = self.dev.pack_qkv(qt, kt, vt, 1, ctx, nh)
        o = self.dev.attention(Q, K, Vt, 1, nh, ctx, float(scale) ** 2,
                               out_dtype=torch.float32)
        out = o.cpu().numpy()
        _t("attn_chain", time.perf_counter() - t0)
        self.calls += 1
        return out

    def _attn_host(self, q, k, v, nh, scale):
        """Per-head scores through the GEMM, one softmax launch for all heads,
        then P.V through the GEMM (rawxrt.py:893-918), all on the device."""
        ctx, d = q.shape
        hd = d // nh
        o = np.empty((ctx, d), np.float32)
        wg = []
        for h in range(nh):
            sl = slice(h * hd, (h + 1) * hd)
            qh = np.ascontiguousarray(q[:, sl] * scale)
            kh = np.ascontiguousarray(k[:, sl].T) * scale
            wg.append(self.matmul(qh, kh))
        wg = self.softmax_stack(wg)
        for h in range(nh):
            sl = slice(h * hd, (h + 1) * hd)
            o[:, sl] = self.matmul(wg[h], np.ascontiguousarray(v[:, sl]))
        return o

    # -- MLP ---------------------------------------------------------------------
    def mlp(self, h, parts, B, akey=None, bkey=None):
        """fc2(GELU(fc1(h))) without fc2's bias (the caller adds b2,
        npu_whisper_encoder.py:525-527). `parts` are fc1 column chunks
        [(W1_T chunk, b1 chunk), ...] (prepare_mlp_chunks)."""
        if self.mlp_ok:
            try:
                return self._mlp_dev(h, parts, B, akey, bkey)
            except Exception as exc:
                self.mlp_ok = False
                msg = f"device mlp -> host path: {type(exc).__name__}: {exc}"
                self.fallbacks.append(msg)
                print(f"[hiprt] {msg}", flush=True)
        f = self.gelu(np.concatenate(
            [self.matmul(h, wc, akey=akey) + bc for wc, bc in parts], axis=1))
        return self.matmul(f, B, bkey=bkey)

    def _mlp_dev(self, h, parts, B, akey=None, bkey=None):
        """fc1 chunks with the GELU fused into their epilogue write bf16 column
        bands of fc2's A operand; fc2 runs from it; one download."""
        torch = _torch()
        t0 = time.perf_counter()
        a = self._act_dev(h)
        M = a.shape[0]
        width = sum(wc.shape[1] for wc, _ in parts)
        f = torch.empty(M, width, dtype=torch.bfloat16, device=self.dev.device)
        epi = {"g4f": L.WXH_EPI_BF16_GELU_POLY4, "erf": L.WXH_EPI_BF16_GELU_ERF}[self.GELU_F32_OP]
        col = 0
        for wc, bc in parts:
            n = wc.shape[1]
            self.dev.gemm(a, self._weight_dev(wc), self._bias_dev(bc), epi, out=f[:, col:col + n])
            col += n
        w2 = self._weight_dev(B, bkey)
        c = self.dev.gemm(f, w2, None, L.WXH_EPI_F32)
        out = c.cpu().numpy()
        self.calls += 1 + len(parts)
        _t("mlp_dev", time.perf_counter() - t0)
        return out

    # -- the whole encoder on the device ------------------------------------------
    def encoder_forward(self, W, mel, n_layer=None, mlp_gelu="erf"):
        """mel [n_mels, T] or [B, n_mels, T] fp32 -> features, one hipGraph.
        Weights are uploaded on first use per weight dict and stay resident."""
        from .native import HipEncoder
        key = (id(W), n_layer, mlp_gelu)
        enc = self._encoders.get(key)
        if enc is None:
            enc = HipEncoder(self.dev, W, n_layer=n_layer, mlp_gelu=mlp_gelu)
            self._encoders[key] = enc
            self._keep.append(W)
        t0 = time.perf_counter()
        out = enc.forward_numpy(mel)
        _t("encoder_graph", time.perf_counter() - t0)
        return out


RawRT = HipRT

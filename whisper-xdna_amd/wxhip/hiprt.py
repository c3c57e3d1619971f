"""HipRT: a drop-in for the reference's raw-XRT backend ``rawxrt.RawRT``.

Same method names, arguments and fallback contract as src/rawxrt.py, with the
device work done by libwxhip.so's gfx950 kernels instead of AIE overlays:

  matmul / mm_start / mm_finish   rawxrt.py:926-996   -> wxh_gemm_bf16
  register_weights                rawxrt.py:307-316   -> device bf16 cache
  attn_chain / _attn_chain_dev    rawxrt.py:813-891   -> wxh_attention (fused)
  _attn_host                      rawxrt.py:893-918   -> score GEMMs, one softmax, P.V GEMMs
  mlp / _mlp_dev                  rawxrt.py:436-544   -> fc1 GEMM(+GELU epilogue) -> fc2 GEMM
  gelu                            rawxrt.py:546-565   -> wxh_gelu (GELU_OP, default g4r)
  softmax_stack                   rawxrt.py:569-585   -> wxh_softmax_rows
  rowop                           rawxrt.py:384-400   -> the op-code table of compile_rowop.py:12-19

Inputs and outputs are host numpy fp32 arrays as in the reference (bf16
buffers as uint16 bit arrays); everything between upload and download runs on
the GPU. There is no CPU compute path. Where the reference steps down a ladder
of implementations when one raises (fused -> chain -> host-routed,
rawxrt.py:822-838; device MLP -> host MLP, :444-455), every rung here is a
device path: the failing rung's flag is cleared, a line naming the stage and
the error is appended to ``fallbacks`` (and printed), and the next rung runs.
The last rung's error propagates.

Numerics that differ from the reference on purpose (each is closer to the
fp32 definition):
* the bias is added in fp32 by the GEMM epilogue; the reference folds it into
  the GEMM as a bf16-rounded row of B (rawxrt.py:352-371);
* attn_chain passes q and k to the fused kernel unscaled and applies the
  product of the two hd^-1/4 factors once to the fp32 scores, where the
  reference rounds q*hd^-1/4 and k*hd^-1/4 to bf16 first;
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

    # deadline of every blocking wait on the device (ms), as the reference
    # bounds each run with NPU_RUN_TIMEOUT_MS (rawxrt.py:51-53, 319-324);
    # passing it raises WxhError (WXH_ERR_TIMEOUT), which trips the fallback
    RUN_TIMEOUT_MS = int(os.environ.get("NPU_RUN_TIMEOUT_MS", "10000"))

    def __init__(self, device=0, max_ctx=6):
        self.dev = Device(device)
        self.dev.set_timeout(self.RUN_TIMEOUT_MS)
        self.max_ctx = max_ctx
        self._live = {}        # no hw_contexts exist here; kept for callers that count them
        self._known = {}       # id(weight array) -> key
        self._keep = []
        self._wdev = {}        # key -> device bf16 [N, K]
        self._bdev = {}        # id(bias) -> device fp32
        self._encoders = {}    # (id(W), n_layer, mlp_gelu, conv_gelu) -> HipEncoder
        self.calls = 0
        self.ctx_creates = 0
        self.evictions = 0
        self.graph_ok = True   # whole-forward hipGraph (wxhip.encoder)
        self.chain_ok = True
        self.fused_ok = True
        self.mlp_ok = True
        self.softmax_ok = True
        self.fallbacks = []

    # -- the fallback contract -------------------------------------------------
    def _retire(self, flag, stage, successor, exc):
        """Stage `stage` raised: clear its flag so later calls skip it, and
        record (and print) which path takes over and why."""
        setattr(self, flag, False)
        note = f"{stage} failed ({type(exc).__name__}: {exc}); {successor} takes over"
        self.fallbacks.append(note)
        print(f"[hiprt] {note}", flush=True)

    def _ladder(self, rungs, *args):
        """Run the first enabled rung of (flag, stage, fn) ... ; a rung that
        raises is retired and the next one runs. The last rung has no flag."""
        for i, (flag, stage, fn) in enumerate(rungs):
            last = i == len(rungs) - 1
            if not last and not getattr(self, flag):
                continue
            if last:
                return fn(*args)
            try:
                return fn(*args)
            except Exception as exc:
                self._retire(flag, stage, rungs[i + 1][1], exc)
        raise AssertionError("unreachable")

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
        d = self._f32_dev(bias)
        if id(bias) in self._known:
            self._bdev[id(bias)] = (bias, d)
        return d

    def _f32_dev(self, a):
        """Host array -> device fp32 (a read-only array, e.g. zero_bias, is
        copied first: torch does not wrap read-only memory)."""
        torch = _torch()
        return torch.from_numpy(np.require(a, np.float32, ["C", "W"])).to(self.dev.device)

    def _act_dev(self, A):
        """Host fp32 activation -> device bf16 (RNE on the device)."""
        torch = _torch()
        t0 = time.perf_counter()
        src = self._f32_dev(A)
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

    def matmul_gelu(self, A, B, bias, akey=None, bkey=None):
        """gelu(A @ B + bias) with the GELU inside the GEMM's epilogue: the
        reference's fused fc1 (npu_matmul_gelu, npu_whisper_encoder.py:93-107),
        here with the exact erf GELU; bf16 values returned as fp32."""
        a = self._act_dev(A)
        c = self.dev.gemm(a, self._weight_dev(B, bkey), self._bias_dev(bias),
                          L.WXH_EPI_BF16_GELU_ERF)
        self.calls += 1
        return c.float().cpu().numpy()

    # -- element-wise ----------------------------------------------------------
    def rowop(self, op, buf_bf16, rows, cols):
        """Run row op `op` (compile_rowop.py:12-19 codes) over a (rows, cols)
        bf16 buffer (uint16 bits, numpy or torch); returns uint16 numpy."""
        x = R.as_device_bf16(self.dev, buf_bf16, rows, cols)
        t0 = time.perf_counter()
        out = R.bits_to_numpy(R.run_op(self.dev, op, x))
        _t(f"{op}_run", time.perf_counter() - t0)
        return out

    def _gelu_dev(self, x, out=None):
        """self.GELU_OP over a 2-D fp32 device tensor -> bf16: g4r/g4f round
        the input to bf16 (RNE) inside the kernel; g4 takes bf16 input."""
        variant = R.GELU_VARIANT[self.GELU_OP]
        xin = self.dev.to_bf16(x) if self.GELU_OP == "g4" else x
        return self.dev.gelu(xin, variant, out=out)

    def gelu(self, x):
        """GELU over any shaped fp32 array via self.GELU_OP, returned as fp32
        (rawxrt.py:546-565; one op for every shape, no tiling needed)."""
        y = self._gelu_dev(self._f32_dev(np.reshape(x, (1, -1))))
        return y.float().cpu().numpy().reshape(np.shape(x))

    def softmax_stack(self, mats):
        """Row softmax of every (L0, L1) head matrix in one launch."""
        nh = len(mats)
        L0, L1 = mats[0].shape
        big = self._f32_dev(np.reshape(np.stack(mats), (nh * L0, L1)))
        f = self.dev.softmax_rows(self.dev.to_bf16(big)).float().cpu().numpy()
        return list(f.reshape(nh, L0, L1))

    # -- attention -------------------------------------------------------------
    def attn_chain(self, q, k, v, nh, scale):
        """o = concat_h softmax((q_h s)(k_h s)^T) v_h for s = scale (the
        reference's hd^-1/4): the fused kernel, else the unfused device path."""
        return self._ladder([("chain_ok", "fused attention kernel", self._attn_chain_dev),
                             (None, "per-head score GEMMs + row softmax", self._attn_host)],
                            q, k, v, nh, scale)

    def attn_fused(self, q, k, v, nh, scale):
        return self._attn_chain_dev(q, k, v, nh, scale)

    def _attn_chain_dev(self, q, k, v, nh, scale):
        torch = _torch()
        ctx, d = q.shape
        if d != nh * 64:
            raise ValueError(f"attention: d={d} is not n_head*64 (n_head={nh})")
        t0 = time.perf_counter()
        Q, K, Vt = self.dev.pack_qkv(self._f32_dev(q), self._f32_dev(k), self._f32_dev(v),
                                     1, ctx, nh)
        o = self.dev.attention(Q, K, Vt, 1, nh, ctx, float(scale) ** 2,
                               out_dtype=torch.float32)
        out = o.cpu().numpy()
        _t("attn_chain", time.perf_counter() - t0)
        self.calls += 1
        return out

    def _attn_host(self, q, k, v, nh, scale):
        """The unfused attention of rawxrt.py:893-918, device-resident: per
        head, the scores (q_h s)(k_h s)^T from the GEMM (k_h s rows are the
        [N, K] weight operand as they stand), rounded to bf16 by its epilogue
        straight into that head's band of one [nh * ctx, ctx] buffer; one
        row-softmax launch over every head (the reference's softmax_stack);
        then P_h v_h from the GEMM into that head's columns of O. One upload
        of q, k, v and one download of O."""
        torch = _torch()
        ctx, d = q.shape
        hd = d // nh
        dv = self.dev.device
        kp = _pad8(ctx)          # P is the A operand of P.V: K = ctx, padded to 8
        scores = torch.zeros(nh * ctx, kp, dtype=torch.bfloat16, device=dv)
        # q and k scaled on the host in fp32, as the reference stages them
        qs = self.dev.to_bf16(self._f32_dev(q * np.float32(scale)))
        ks = self.dev.to_bf16(self._f32_dev(k * np.float32(scale)))
        vt = torch.zeros(d, kp, dtype=torch.bfloat16, device=dv)
        self.dev.to_bf16(self._f32_dev(v), transpose=True, out=vt[:, :ctx])
        for h in range(nh):
            c = slice(h * hd, (h + 1) * hd)
            self.dev.gemm(qs[:, c], ks[:, c], None, L.WXH_EPI_BF16,
                          out=scores[h * ctx:(h + 1) * ctx, :ctx])
        # P's pad columns stay zero: they are K entries of the P.V GEMM
        probs = self.dev.softmax_rows(scores, valid=ctx, out=torch.zeros_like(scores))
        o = torch.empty(ctx, d, dtype=torch.float32, device=dv)
        for h in range(nh):
            c = slice(h * hd, (h + 1) * hd)
            self.dev.gemm(probs[h * ctx:(h + 1) * ctx], vt[c], None, L.WXH_EPI_F32,
                          out=o[:, c])
        self.calls += 2 * nh
        return o.cpu().numpy()

    # -- MLP ---------------------------------------------------------------------
    def mlp(self, h, parts, B, akey=None, bkey=None):
        """fc2(GELU(fc1(h))) without fc2's bias (the caller adds b2,
        npu_whisper_encoder.py:525-527). `parts` are fc1 column chunks
        [(W1_T chunk, b1 chunk), ...] (prepare_mlp_chunks)."""
        return self._ladder([("mlp_ok", "fused device MLP", self._mlp_dev),
                             (None, "unfused device MLP (fc1, GELU row kernel, fc2)",
                              self._mlp_unfused)],
                            h, parts, B, akey, bkey)

    def _fc1_bands(self, a, parts, epi, dtype):
        """Every fc1 chunk's GEMM writes its own column band of one [M, width]
        buffer; returns the buffer."""
        torch = _torch()
        width = sum(wc.shape[1] for wc, _ in parts)
        f = torch.empty(a.shape[0], width, dtype=dtype, device=self.dev.device)
        edges = np.cumsum([0] + [wc.shape[1] for wc, _ in parts])
        for (wc, bc), c0, c1 in zip(parts, edges[:-1], edges[1:]):
            self.dev.gemm(a, self._weight_dev(wc), self._bias_dev(bc), epi, out=f[:, c0:c1])
        self.calls += len(parts)
        return f

    def _mlp_dev(self, h, parts, B, akey=None, bkey=None):
        """fc1 chunks with the GELU (GELU_F32_OP) in their epilogue write bf16
        column bands of fc2's A operand; fc2 runs from it; one download."""
        torch = _torch()
        t0 = time.perf_counter()
        epi = {"g4f": L.WXH_EPI_BF16_GELU_POLY4, "erf": L.WXH_EPI_BF16_GELU_ERF}[self.GELU_F32_OP]
        f = self._fc1_bands(self._act_dev(h), parts, epi, torch.bfloat16)
        c = self.dev.gemm(f, self._weight_dev(B, bkey), None, L.WXH_EPI_F32)
        self.calls += 1
        out = c.cpu().numpy()
        _t("mlp_dev", time.perf_counter() - t0)
        return out

    def _mlp_unfused(self, h, parts, B, akey=None, bkey=None):
        """The reference's host-side MLP order (fc1 chunks + bias in fp32, then
        rt.gelu's GELU_OP, then fc2; rawxrt.py:453-455), every step on the
        device: fp32 fc1 bands, the GELU row kernel into bf16, fc2."""
        torch = _torch()
        f32 = self._fc1_bands(self._act_dev(h), parts, L.WXH_EPI_F32, torch.float32)
        c = self.dev.gemm(self._gelu_dev(f32), self._weight_dev(B, bkey), None, L.WXH_EPI_F32)
        self.calls += 1
        return c.cpu().numpy()

    # -- the whole encoder on the device ------------------------------------------
    def encoder_forward(self, W, mel, n_layer=None, mlp_gelu="erf", conv_gelu="erf"):
        """mel [n_mels, T] or [B, n_mels, T] fp32 -> features, one hipGraph.
        Weights are uploaded on first use per weight dict and stay resident."""
        from .native import HipEncoder
        key = (id(W), n_layer, mlp_gelu, conv_gelu)
        enc = self._encoders.get(key)
        if enc is None:
            enc = HipEncoder(self.dev, W, n_layer=n_layer, mlp_gelu=mlp_gelu,
                             conv_gelu=conv_gelu)
            self._encoders[key] = enc
            self._keep.append(W)
        t0 = time.perf_counter()
        out = enc.forward_numpy(mel)
        _t("encoder_graph", time.perf_counter() - t0)
        return out


RawRT = HipRT

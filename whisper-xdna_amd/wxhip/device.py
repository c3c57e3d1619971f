"""Device-tensor front end of libwxhip.so.

`Device` owns one wxh_ctx and exposes every op on torch tensors that already
live on the GPU (torch is the device-memory and stream plumbing here; the
compute is the library's HIP kernels). Every op is launched on torch's current
stream for the device, so it is ordered with the caller's torch work.
Shapes, dtypes and contiguity are checked here before any launch; the library
checks them again.
"""
import ctypes as C

from . import _lib as L


def _torch():
    import torch
    return torch


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _ld(t):
    """Row stride of a 2-D tensor; a single row's stride is meaningless (numpy
    and torch may report 0), so it is taken as the row length."""
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


class Device:
    """One libwxhip context on GPU `index` (gfx950 only)."""

    def __init__(self, index=0):
        torch = _torch()
        if not torch.cuda.is_available():
            raise L.WxhLibraryError("no GPU visible to torch; libwxhip needs a gfx950 device")
        self.lib = L.load()
        self.index = index
        self.device = torch.device("cuda", index)
        h = C.c_void_p()
        L.call("wxh_create", index, C.byref(h))
        self._h = h

    # -- plumbing ----------------------------------------------------------
    @property
    def handle(self):
        return self._h

    def stream(self):
        return C.c_void_p(_torch().cuda.current_stream(self.device).cuda_stream)

    def synchronize(self):
        _torch().cuda.synchronize(self.device)

    def set_fail_inject(self, mask):
        L.call("wxh_set_fail_inject", self._h, mask)

    def set_timeout(self, ms):
        """Deadline of the library's own blocking waits (0: none); see
        wxh_set_timeout."""
        L.call("wxh_set_timeout", self._h, int(ms))

    def set_tuning(self, what, value):
        """A tuning switch (WXH_TUNE_*; 0 = automatic); see wxh_set_tuning."""
        L.call("wxh_set_tuning", self._h, int(what), int(value))

    def wait(self):
        """wxh_synchronize: the context's stream, under its deadline."""
        L.call("wxh_synchronize", self._h)

    def close(self):
        if getattr(self, "_h", None):
            self.lib.wxh_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, t, dtype, name, dims=None):
        torch = _torch()
        if t.device != self.device:
            raise ValueError(f"{name} must be on {self.device}, got {t.device}")
        if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
            raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
        if dims is not None and t.dim() != dims:
            raise ValueError(f"{name} must be {dims}-D, got shape {tuple(t.shape)}")
        if t.dim() >= 1 and t.stride(-1) != 1:
            raise ValueError(f"{name} must have unit stride in its last dimension")
        del torch

    @staticmethod
    def _dt(t):
        torch = _torch()
        return L.WXH_F32 if t.dtype == torch.float32 else L.WXH_BF16

    # -- row ops -------------------------------------------------------------
    def layer_norm(self, x, gamma=None, beta=None, eps=1e-5, out_dtype=None,
                   resid=None, sum_out=None, out=None):
        """LN over the last axis of a 2-D x (bf16 or fp32); see wxh_layernorm."""
        torch = _torch()
        self._check(x, (torch.bfloat16, torch.float32), "x", 2)
        rows, cols = x.shape
        out_dtype = out_dtype or torch.bfloat16
        y = out if out is not None else torch.empty(rows, cols, dtype=out_dtype, device=self.device)
        self._check(y, (torch.bfloat16, torch.float32), "out", 2)
        for n, t in (("gamma", gamma), ("beta", beta)):
            if t is not None:
                self._check(t, torch.float32, n, 1)
                if t.numel() != cols:
                    raise ValueError(f"{n} must have {cols} elements")
        if resid is not None:
            self._check(resid, torch.float32, "resid", 2)
        if sum_out is not None:
            self._check(sum_out, torch.float32, "sum_out", 2)
        L.call("wxh_layernorm", self._h, _ptr(x), self._dt(x), _ld(x),
               _ptr(resid), _ld(resid) if resid is not None else 0,
               _ptr(sum_out), _ld(sum_out) if sum_out is not None else 0,
               _ptr(gamma), _ptr(beta), eps, _ptr(y), self._dt(y), _ld(y),
               rows, cols, self.stream())
        return y

    def gelu(self, x, variant=L.WXH_GELU_ERF, out=None):
        """Element-wise GELU of a 2-D x (bf16 or fp32) -> bf16."""
        torch = _torch()
        self._check(x, (torch.bfloat16, torch.float32), "x", 2)
        rows, cols = x.shape
        y = out if out is not None else torch.empty(rows, cols, dtype=torch.bfloat16, device=self.device)
        self._check(y, torch.bfloat16, "out", 2)
        if tuple(y.shape[:1]) != (rows,) or y.shape[1] < cols:
            raise ValueError("out must have the rows of x and at least its columns")
        L.call("wxh_gelu", self._h, _ptr(x), self._dt(x), _ld(x), _ptr(y),
               _ld(y), rows, cols, variant, self.stream())
        return y

    def log_mel(self, audio, n_mels=80, out=None):
        """Whisper log-mel features of 16 kHz fp32 audio on the device:
        [n_samples] -> [n_mels, n_samples // 160], or [B, n_samples] ->
        [B, n_mels, n_samples // 160] (floor at each clip's maximum - 8)."""
        torch = _torch()
        squeeze = audio.dim() == 1
        a = (audio[None] if squeeze else audio)
        self._check(a, torch.float32, "audio", 2)
        a = a.contiguous()
        B, n = a.shape
        y = out if out is not None else torch.empty(B, n_mels, n // 160, dtype=torch.float32,
                                                    device=self.device)
        if tuple(y.shape) != (B, n_mels, n // 160) or y.dtype != torch.float32 or not y.is_contiguous():
            raise ValueError(f"out must be contiguous fp32 [{B}, {n_mels}, {n // 160}]")
        L.call("wxh_log_mel", self._h, _ptr(a), B, n, n_mels, _ptr(y), self.stream())
        return y[0] if squeeze else y

    def softmax_rows(self, x, valid=None, out=None):
        """Row softmax of bf16 x over its first `valid` columns -> bf16."""
        torch = _torch()
        self._check(x, torch.bfloat16, "x", 2)
        rows, cols = x.shape
        valid = cols if valid is None else valid
        if not 0 < valid <= cols:
            raise ValueError(f"valid={valid} outside (0, {cols}]")
        y = out if out is not None else torch.empty_like(x)
        self._check(y, torch.bfloat16, "out", 2)
        L.call("wxh_softmax_rows", self._h, _ptr(x), _ld(x), _ptr(y),
               _ld(y), rows, valid, self.stream())
        return y

    def to_bf16(self, x, transpose=False, out=None):
        """fp32 2-D -> bf16 (RNE), optionally transposed."""
        torch = _torch()
        self._check(x, torch.float32, "x", 2)
        rows, cols = x.shape
        shape = (cols, rows) if transpose else (rows, cols)
        y = out if out is not None else torch.empty(shape, dtype=torch.bfloat16, device=self.device)
        L.call("wxh_convert_f32_bf16", self._h, _ptr(x), _ld(x), _ptr(y),
               _ld(y), rows, cols, int(transpose), self.stream())
        return y

    # -- GEMM ------------------------------------------------------------------
    def gemm(self, A, W, bias=None, epilogue=L.WXH_EPI_F32, out=None):
        """A [M,K] bf16 . W [N,K]^T bf16 (+bias fp32) with a WXH_EPI_* epilogue.
        For WXH_EPI_RESID_F32, `out` is the fp32 residual updated in place."""
        torch = _torch()
        self._check(A, torch.bfloat16, "A", 2)
        self._check(W, torch.bfloat16, "W", 2)
        M, K = A.shape
        N, K2 = W.shape
        if K != K2:
            raise ValueError(f"A {tuple(A.shape)} and W {tuple(W.shape)} disagree on K")
        if bias is not None:
            self._check(bias, torch.float32, "bias", 1)
            if bias.numel() != N:
                raise ValueError("bias must have N elements")
        odt = torch.float32 if epilogue in (L.WXH_EPI_F32, L.WXH_EPI_RESID_F32) else torch.bfloat16
        if out is None:
            if epilogue == L.WXH_EPI_RESID_F32:
                raise ValueError("the residual epilogue needs out= (the fp32 residual)")
            out = torch.empty(M, N, dtype=odt, device=self.device)
        self._check(out, odt, "out", 2)
        if tuple(out.shape) != (M, N):
            raise ValueError(f"out must be {(M, N)}")
        L.call("wxh_gemm_bf16", self._h, M, N, K, _ptr(A), _ld(A), _ptr(W),
               _ld(W), _ptr(bias), _ptr(out), _ld(out), epilogue, self.stream())
        return out

    # -- int8 ------------------------------------------------------------------
    def quantize_rows(self, x, cols_pad=None, per_tensor=False, out=None, scale=None):
        """Symmetric int8 quantisation of a 2-D x (fp32 or bf16), per row
        (scale [rows]) or per tensor (scale [1]); see wxh_quantize_rows.
        Returns (q int8 [rows, cols_pad], scale fp32)."""
        torch = _torch()
        self._check(x, (torch.float32, torch.bfloat16), "x", 2)
        rows, cols = x.shape
        cols_pad = cols if cols_pad is None else int(cols_pad)
        if out is None:
            out = torch.empty(rows, cols_pad, dtype=torch.int8, device=self.device)
        self._check(out, torch.int8, "out", 2)
        if tuple(out.shape) != (rows, cols_pad):
            raise ValueError(f"out must be {(rows, cols_pad)}")
        n = 1 if per_tensor else rows
        if scale is None:
            scale = torch.empty(n, dtype=torch.float32, device=self.device)
        self._check(scale, torch.float32, "scale", 1)
        if scale.numel() < n:
            raise ValueError(f"scale needs {n} elements")
        L.call("wxh_quantize_rows", self._h, _ptr(x), self._dt(x), _ld(x), rows, cols,
               _ptr(out), _ld(out), cols_pad, _ptr(scale), int(bool(per_tensor)),
               self.stream())
        return out, scale

    def gemm_i8(self, A, a_scale, W, w_scale, bias=None, epilogue=L.WXH_EPI_F32, out=None):
        """int8 A [M,K] (row scales) . int8 W [N,K]^T (column scales) (+bias)
        with a WXH_EPI_* epilogue; see wxh_gemm_i8."""
        torch = _torch()
        self._check(A, torch.int8, "A", 2)
        self._check(W, torch.int8, "W", 2)
        M, K = A.shape
        N, K2 = W.shape
        if K != K2:
            raise ValueError(f"A {tuple(A.shape)} and W {tuple(W.shape)} disagree on K")
        self._check(a_scale, torch.float32, "a_scale", 1)
        self._check(w_scale, torch.float32, "w_scale", 1)
        if a_scale.numel() < M or w_scale.numel() < N:
            raise ValueError("a_scale needs M and w_scale N elements")
        if bias is not None:
            self._check(bias, torch.float32, "bias", 1)
            if bias.numel() != N:
                raise ValueError("bias must have N elements")
        f32 = (L.WXH_EPI_F32, L.WXH_EPI_RESID_F32, L.WXH_EPI_F32_GELU_ERF)
        odt = torch.float32 if epilogue in f32 else torch.bfloat16
        if out is None:
            if epilogue == L.WXH_EPI_RESID_F32:
                raise ValueError("the residual epilogue needs out= (the fp32 residual)")
            out = torch.empty(M, N, dtype=odt, device=self.device)
        self._check(out, odt, "out", 2)
        if tuple(out.shape) != (M, N):
            raise ValueError(f"out must be {(M, N)}")
        L.call("wxh_gemm_i8", self._h, M, N, K, _ptr(A), _ld(A), _ptr(a_scale), _ptr(W),
               _ld(W), _ptr(w_scale), _ptr(bias), _ptr(out), _ld(out), epilogue, self.stream())
        return out

    # -- attention -------------------------------------------------------------
    def padded_len(self, T):
        return self.lib.wxh_attention_padded_len(T)

    def attn_buffers(self, batch, n_head, T):
        """Zeroed Q, K [B*nh, Tp, 64] and Vt [B*nh, 64, Tp] bf16 buffers."""
        torch = _torch()
        Tp = self.padded_len(T)
        z = dict(dtype=torch.bfloat16, device=self.device)
        return (torch.zeros(batch * n_head, Tp, 64, **z), torch.zeros(batch * n_head, Tp, 64, **z),
                torch.zeros(batch * n_head, 64, Tp, **z))

    def pack_qkv(self, q, k, v, batch, T, n_head, bufs=None):
        """fp32 rows [B*T, nh*64] -> (Q, K, Vt) attention operand layouts."""
        torch = _torch()
        for n, t in (("q", q), ("k", k), ("v", v)):
            self._check(t, torch.float32, n, 2)
            if tuple(t.shape) != (batch * T, n_head * 64):
                raise ValueError(f"{n} must be {(batch * T, n_head * 64)}")
        if not (_ld(q) == _ld(k) == _ld(v)):
            raise ValueError("q, k, v must share a row stride")
        Q, K, Vt = bufs if bufs is not None else self.attn_buffers(batch, n_head, T)
        L.call("wxh_pack_qkv", self._h, _ptr(q), _ptr(k), _ptr(v), _ld(q), batch, T,
               n_head, _ptr(Q), _ptr(K), _ptr(Vt), self.stream())
        return Q, K, Vt

    def attention(self, Q, K, Vt, batch, n_head, T, scale, out_dtype=None, out=None):
        """softmax(scale Q K^T) V -> [B*T, nh*64] (bf16 or fp32)."""
        torch = _torch()
        Tp = self.padded_len(T)
        for n, t, shp in (("Q", Q, (batch * n_head, Tp, 64)), ("K", K, (batch * n_head, Tp, 64)),
                          ("Vt", Vt, (batch * n_head, 64, Tp))):
            self._check(t, torch.bfloat16, n, 3)
            if tuple(t.shape) != shp or not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous {shp}, got {tuple(t.shape)}")
        out_dtype = out_dtype or torch.bfloat16
        o = out if out is not None else torch.empty(batch * T, n_head * 64, dtype=out_dtype,
                                                    device=self.device)
        L.call("wxh_attention", self._h, _ptr(Q), _ptr(K), _ptr(Vt), batch, n_head, T,
               float(scale), _ptr(o), self._dt(o), _ld(o), self.stream())
        return o

"""The reference's int8 quantised matmul, on the GPU.

bench/probe_int8_decode.py:48-74 defines ``q_matmul_factory(mode)``, a
matmul plug ``q_matmul(A, B, bias=None, **kw)`` for the encoder entry point
(A [M, K] activations, B [K, N] the weight_T, fp32 numpy):

* ``perchan``: per-token scales on A, per-column (output channel) scales on B;
* ``pertensor``: per-token scales on A, one scale for B;
* ``fp32``: no quantisation (the control).

The probe runs ``encoder(W, mel, q_matmul_factory(mode), np_matmul,
fold_bias=False)`` (:143-145); ``wxhip.encoder.encoder`` takes the plug the
same way. Here both operands go to the device and are quantised by
``wxh_quantize_rows`` (scale = max|x| / 127, q = rint(x / scale), K
zero-padded to a multiple of 128); ``wxh_gemm_i8`` forms the exact int32
products, converts, scales by the row and column scales and adds the bias,
all in fp32, in the reference's order. ``fp32`` runs the library's
unquantised GEMM (``HipRT.matmul``: bf16 operands, fp32 accumulation; the
device has no fp32 GEMM). B's quantisation is kept per array (by identity,
the array held alive), as ``HipRT.register_weights`` keeps device weights.

For a whole encoder on the device use ``HipEncoder(dev, W, int8=True)``,
which runs the same quantisation inside one graph.
"""
import numpy as np

from . import _lib as L

MODES = ("fp32", "perchan", "pertensor")


def _pad128(k):
    return (k + 127) // 128 * 128


def q_matmul_factory(mode, rt=None):
    """-> q_matmul(A, B, bias=None, **kw) on the GPU of `rt` (a HipRT; one is
    created on device 0 when omitted)."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}")
    from .hiprt import HipRT
    rt = rt if rt is not None else HipRT()
    state = {"w": {}}
    stats = {"n": 0}

    def q_matmul(A, B, bias=None, **kw):
        import torch
        rt_ = rt
        if mode == "fp32":
            return rt_.matmul(A, B, bias=bias)
        dev = rt_.dev
        A = np.ascontiguousarray(A, np.float32)
        M, K = A.shape
        K2, N = np.shape(B)
        if K != K2:
            raise ValueError(f"q_matmul: A {A.shape} and B {np.shape(B)} disagree on K")
        if K % 8:
            raise ValueError(f"q_matmul: K={K} must be a multiple of 8")
        Kp = _pad128(K)
        ent = state["w"].get(id(B))
        if ent is None or ent[0] is not B:
            w = torch.from_numpy(np.ascontiguousarray(B, np.float32)).to(dev.device)
            w = w.t().contiguous()  # (N, K): the GEMM's weight layout
            wq, sw = dev.quantize_rows(w, cols_pad=Kp, per_tensor=(mode == "pertensor"))
            if mode == "pertensor":
                sw = sw.expand(N).contiguous()
            ent = (B, wq, sw)
            state["w"][id(B)] = ent
        _, wq, sw = ent
        a = torch.from_numpy(A).to(dev.device)
        aq, sa = dev.quantize_rows(a, cols_pad=Kp)
        b = None
        if bias is not None:
            b = torch.from_numpy(np.ascontiguousarray(bias, np.float32).reshape(-1)).to(dev.device)
        c = dev.gemm_i8(aq, sa, wq, sw, b, L.WXH_EPI_F32)
        stats["n"] += 1
        return c.cpu().numpy()

    q_matmul.stats = stats
    q_matmul.rt = rt  # the encoder entry point runs its other ops on this HipRT
    return q_matmul


__all__ = ["MODES", "q_matmul_factory"]

#!/usr/bin/env python3
"""Kernel driver for hardware-counter collection.

    python3 whisper-xdna_amd/wxhip/probe.py KERNEL [--reps N] [--batch B]

Runs one encoder kernel of the large-v3-shaped encoder (d 1280, 20 heads,
ctx 1500, batch B, default 16) N times on seeded synthetic operands through
the C ABI, preceded by N plain device copies of 512 MiB (torch's copy
kernel). Under `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`, the
copies' counter readings against their known byte count give the scale
factor that turns the kernel's readings into HBM bytes per launch.

KERNEL is one of
  fc1        A [B*1500, 1280] . W1 [5120, 1280]^T + b1, erf-GELU, bf16 out
  fc2        A [B*1500, 5120] . W2 [1280, 5120]^T + b2 into the fp32 residual
  qkv        A [B*1500, 1280] . Wqkv [3840, 1280]^T split into Q, K, Vt
  out_proj   A [B*1500, 1280] . Wo [1280, 1280]^T + bo into the fp32 residual
  attention  softmax(Q K^T / 8) V over B*20 heads of 1500 keys
  rowops     the row kernels on the standalone rowops shapes, N launches each
             on one buffer pair per kernel: LayerNorm [1500, 1280] bf16 and
             [24000, 1280] fp32 -> bf16, erf-GELU and poly4-GELU (g4r)
             [1500, 5120] bf16, softmax [30000, 1500] bf16
"""
import argparse
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

D, NH, CTX, FF = 1280, 20, 1500, 5120
COPY_BYTES = 512 << 20


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("kernel", choices=["fc1", "fc2", "qkv", "out_proj", "attention", "rowops"])
    ap.add_argument("--reps", type=int, default=4)
    ap.add_argument("--batch", type=int, default=16)
    args = ap.parse_args()

    import torch
    import wxhip
    from wxhip import _lib as L

    dev = wxhip.Device(0)
    g = torch.Generator(device=dev.device).manual_seed(0)
    M = args.batch * CTX

    def normal(shape, std, dtype=torch.bfloat16):
        return (torch.randn(shape, generator=g, device=dev.device) * std).to(dtype)

    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev.device).normal_(generator=g)
    dst = torch.empty_like(src)
    run = None
    if args.kernel in ("fc1", "fc2", "qkv", "out_proj"):
        K, N = {"fc1": (D, FF), "fc2": (FF, D), "qkv": (D, 3 * D), "out_proj": (D, D)}[args.kernel]
        A, W, b = normal((M, K), 1.0), normal((N, K), 0.02), normal((N,), 0.02, torch.float32)
        if args.kernel == "fc1":
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev.device)
            run = lambda: dev.gemm(A, W, b, L.WXH_EPI_BF16_GELU_ERF, out=out)
        elif args.kernel == "qkv":
            # the fused QKV epilogue exists only inside the encoder graph; the
            # C ABI's bf16 epilogue runs the same main loop over the same shape
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev.device)
            run = lambda: dev.gemm(A, W, b, L.WXH_EPI_BF16, out=out)
        else:
            x = normal((M, N), 1.0, torch.float32)
            run = lambda: dev.gemm(A, W, b, L.WXH_EPI_RESID_F32, out=x)
    elif args.kernel == "rowops":
        def rowop_runs():
            cases = []
            x = normal((1500, 1280), 2.0)
            gm = 1 + normal((1280,), 0.1, torch.float32)
            bt = normal((1280,), 0.1, torch.float32)
            y = torch.empty_like(x)
            cases.append(("layernorm 1500x1280 bf16", lambda: dev.layer_norm(x, gm, bt, out=y)))
            xf = normal((24000, 1280), 2.0, torch.float32)
            yf = torch.empty(24000, 1280, dtype=torch.bfloat16, device=dev.device)
            cases.append(("layernorm 24000x1280 f32->bf16",
                          lambda: dev.layer_norm(xf, gm, bt, out=yf)))
            xg = normal((1500, 5120), 3.0)
            yg = torch.empty_like(xg)
            cases.append(("gelu erf 1500x5120", lambda: dev.gelu(xg, L.WXH_GELU_ERF, out=yg)))
            cases.append(("gelu poly4 1500x5120",
                          lambda: dev.gelu(xg, L.WXH_GELU_POLY4_RNE, out=yg)))
            xs = normal((30000, 1500), 4.0)
            ys = torch.empty_like(xs)
            cases.append(("softmax 30000x1500", lambda: dev.softmax_rows(xs, out=ys)))
            return cases

        cases = rowop_runs()

        def run():
            for name, fn in cases:
                fn()
    else:
        Q, Kt, Vt = dev.attn_buffers(args.batch, NH, CTX)
        for t in (Q, Kt, Vt):
            t.copy_(normal(t.shape, 1.0))
        run = lambda: dev.attention(Q, Kt, Vt, args.batch, NH, CTX, 64 ** -0.5)

    for i in range(args.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[probe] copy {COPY_BYTES} bytes x {args.reps}", flush=True)
    for i in range(args.reps):
        run()
    dev.synchronize()
    what = "rowops shapes" if args.kernel == "rowops" else f"batch {args.batch}"
    print(f"[probe] {args.kernel} {what} x {args.reps}", flush=True)


if __name__ == "__main__":
    main()

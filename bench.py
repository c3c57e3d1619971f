#!/usr/bin/env python3
"""Benchmark of the Whisper-encoder hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
                    [--no-rowops] [--no-int8] [--workload l16|l1|l16s]
    python bench.py --probe KERNEL [--reps N] [--batch B]   (counter runs)

A step is one encoder forward (mel -> features) of the workload over inputs
already resident in HBM, replayed as the captured hipGraph. Default workload:
the large-v3-shaped encoder (32 layers, d 1280, 20 heads, ctx 1500) on a
batch of 16 synthetic log-mels [16, 128, 3000]; `value` is mel-frames/s.
The same run also reports the batch-1 latency (large-v3, ctx 1500; the median
of >= 20 single replays timed with HIP events), the
encoder's fraction of the bf16 MFMA peak, per-stage device times (HIP events
on the stream the kernels run on), the roofline of the dominant kernel, the
row kernels' HBM throughput over rotating buffers larger than the 256 MB
Infinity Cache, the same encoder with int8 GEMMs (`int8`: the reference's
per-token / per-channel quantised matmul; an extra line, not `value`), and
the CPU baseline (the torch fp32 oracle on this host's cores, on a bounded
sample).

Prints ONE JSON line.

--probe KERNEL runs one kernel of the large-v3-shaped encoder (batch B,
default 16) N times on seeded operands through the C ABI, after N plain
512 MiB device copies, and prints no JSON: it is the program the rocprofv3
counter runs in profiles/ profile. The copies' FETCH_SIZE / WRITE_SIZE
against their known byte count give the factor that turns the kernel's
readings into bytes. KERNEL: fc1 (erf-GELU epilogue, bf16 out), fc2 and
out_proj (fp32 residual epilogue), qkv (the QKV main loop with a plain bf16
epilogue), attention (softmax(Q K^T / 8) V over B*20 heads of 1500 keys),
rowops (LayerNorm [1500,1280] bf16 and [24000,1280] fp32 -> bf16, erf- and
poly4-GELU [1500,5120], softmax [30000,1500], each N times), encoder (graph
replays of the whole 32-layer forward at batch B: every kernel as the
encoder launches it, split-K included).
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT / "whisper-xdna_amd"), str(ROOT)]

METRIC = "large-v3 encoder ms @ctx=1500 bs=1; mel-frames/s bs=16; % bf16 MFMA peak"
PEAK_BF16 = 2.5e15      # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12       # MI355X HBM3E, B/s
PEAK_FP64_TF = 78.6     # MI355X fp64, TFLOP/s
PEAK_I8 = 5.0e15        # MI355X dense int8 MFMA, OP/s
# HBM-side bytes per launch of the kernels that can be the dominant stage,
# measured with `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` over
# `bench.py --probe KERNEL` at the batch-16 shape, each counter scaled by
# what it reads for a 512 MiB device copy (FETCH_SIZE x 2.000, WRITE_SIZE
# x 1.000); the summaries, with their commands, are in profiles/.
TRAFFIC_BYTES = {
    "fc1": (8.125e8, "profiles/gemm_fc1_l16_traffic.md"),
    "attention": (2.504e8, "profiles/attention_l16_traffic.md"),
}
LARGE = dict(n_mels=128, d=1280, n_head=20, n_layer=32, n_ctx=1500)
WORKLOADS = {
    "l16": dict(batch=16, n_frames=3000,
                name="whisper-large-v3-shaped encoder, batch 16, ctx 1500, 32 layers, bf16/fp32-acc"),
    "l1": dict(batch=1, n_frames=3000,
               name="whisper-large-v3-shaped encoder, batch 1, ctx 1500, 32 layers, bf16/fp32-acc"),
    "l16s": dict(batch=16, n_frames=1024,
                 name="whisper-large-v3-shaped encoder, batch 16, ctx 512, 32 layers, bf16/fp32-acc"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def stage_flops(g, batch, n_frames):
    """Algorithmic FLOPs per stage of one forward (2*M*N*K per GEMM,
    4*ctx^2*d per layer for attention; unpadded shapes)."""
    d, nm, nl = g["d"], g["n_mels"], g["n_layer"]
    ctx = (n_frames - 1) // 2 + 1
    M = batch * ctx
    return {
        "conv1": 2 * batch * n_frames * d * 3 * nm,
        "conv2": 2 * M * d * 3 * d,
        "qkv": nl * 2 * M * 3 * d * d,
        "attention": nl * 4 * batch * ctx * ctx * d,
        "out_proj": nl * 2 * M * d * d,
        "fc1": nl * 2 * M * 4 * d * d,
        "fc2": nl * 2 * M * 4 * d * d,
    }


def stage_launches(g):
    nl = g["n_layer"]
    return {"conv1": 1, "conv2": 1, "qkv": nl, "attention": nl, "out_proj": nl,
            "fc1": nl, "fc2": nl, "layernorm": 2 * nl, "ln_post": 1, "prep": 1}


def time_forward(enc, mel, steps, warmup, host=None):
    """Wall time per forward over `steps` graph replays (synchronised on
    both sides). With `host` (a dict), also the host CPU time (user + system
    of every thread of the process, the quantity bench/run_raw_encoder.py:
    113-118 reports from os.times, here from time.process_time for its finer
    resolution) that issuing them took, per forward: the host's whole share
    of the forward, since the replays run on the GPU."""
    import torch
    for _ in range(warmup):
        enc.forward(mel)
    torch.cuda.synchronize()
    c0 = time.process_time()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = enc.forward(mel)
    c1 = time.process_time()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    if host is not None:
        host["host_cpu_ms_per_step"] = round((c1 - c0) / steps * 1e3, 3)
    return dt, out


def latency_median(enc, mel, n, warmup):
    """Median device time of `n` single forwards (graph replays), each
    bracketed by HIP events on the stream the library launches on (torch's
    current stream), after `warmup` untimed ones."""
    import numpy as np
    import torch
    for _ in range(warmup):
        enc.forward(mel)
    torch.cuda.synchronize()
    evs = []
    for _ in range(n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        enc.forward(mel)
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in evs])) / 1e3


PROBE_KERNELS = ("fc1", "fc2", "qkv", "out_proj", "attention", "rowops", "encoder")


def probe(kernel, reps, batch):
    """One kernel at its large-v3 shape, `reps` times, after `reps` plain
    512 MiB device copies (the counters' scale reference); see the module
    doc. Prints a line per phase."""
    import torch
    import wxhip
    from wxhip import _lib as L
    D, NH, CTX, FF = 1280, 20, 1500, 5120
    copy_bytes = 512 << 20
    dev = wxhip.Device(0)
    g = torch.Generator(device=dev.device).manual_seed(0)
    M = batch * CTX

    def normal(shape, std, dtype=torch.bfloat16):
        return (torch.randn(shape, generator=g, device=dev.device) * std).to(dtype)

    src = torch.empty(copy_bytes // 2, dtype=torch.bfloat16, device=dev.device).normal_(generator=g)
    dst = torch.empty_like(src)
    if kernel in ("fc1", "fc2", "qkv", "out_proj"):
        K, N = {"fc1": (D, FF), "fc2": (FF, D), "qkv": (D, 3 * D), "out_proj": (D, D)}[kernel]
        A, W, b = normal((M, K), 1.0), normal((N, K), 0.02), normal((N,), 0.02, torch.float32)
        if kernel in ("fc1", "qkv"):
            # the fused QKV epilogue exists only inside the encoder graph; the
            # C ABI's bf16 epilogue runs the same main loop over the same shape
            out = torch.empty(M, N, dtype=torch.bfloat16, device=dev.device)
            epi = L.WXH_EPI_BF16_GELU_ERF if kernel == "fc1" else L.WXH_EPI_BF16
            cases = [(kernel, lambda: dev.gemm(A, W, b, epi, out=out))]
        else:
            x = normal((M, N), 1.0, torch.float32)
            cases = [(kernel, lambda: dev.gemm(A, W, b, L.WXH_EPI_RESID_F32, out=x))]
    elif kernel == "encoder":
        from wxhip import synth
        enc = wxhip.HipEncoder(dev, synth.make_weights("large-v3"))
        mel = torch.from_numpy(synth.make_mel_batch(batch, 128, 3000)).to(dev.device)
        enc.forward(mel)            # graph captured outside the counted phase
        cases = [("encoder forward (graph replay)", lambda: enc.forward(mel))]
    elif kernel == "attention":
        Q, Kt, Vt = dev.attn_buffers(batch, NH, CTX)
        for t in (Q, Kt, Vt):
            t.copy_(normal(t.shape, 1.0))
        cases = [(kernel, lambda: dev.attention(Q, Kt, Vt, batch, NH, CTX, 64 ** -0.5))]
    else:
        x = normal((1500, 1280), 2.0)
        gm = 1 + normal((1280,), 0.1, torch.float32)
        bt = normal((1280,), 0.1, torch.float32)
        y = torch.empty_like(x)
        xf = normal((24000, 1280), 2.0, torch.float32)
        yf = torch.empty(24000, 1280, dtype=torch.bfloat16, device=dev.device)
        xg = normal((1500, 5120), 3.0)
        yg = torch.empty_like(xg)
        xs = normal((30000, 1500), 4.0)
        ys = torch.empty_like(xs)
        cases = [("layernorm 1500x1280 bf16", lambda: dev.layer_norm(x, gm, bt, out=y)),
                 ("layernorm 24000x1280 f32->bf16", lambda: dev.layer_norm(xf, gm, bt, out=yf)),
                 ("gelu erf 1500x5120", lambda: dev.gelu(xg, L.WXH_GELU_ERF, out=yg)),
                 ("gelu poly4 1500x5120", lambda: dev.gelu(xg, L.WXH_GELU_POLY4_RNE, out=yg)),
                 ("softmax 30000x1500", lambda: dev.softmax_rows(xs, out=ys))]
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[probe] copy {copy_bytes} bytes x {reps}", flush=True)
    for name, fn in cases:
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        print(f"[probe] {name} (batch {batch}) x {reps}", flush=True)


def rowop_bandwidth(dev):
    """Row kernels over rotating buffer sets > 256 MB, captured in a graph so
    launch gaps do not count; returns GB/s per kernel (algorithmic bytes =
    one read + one write of every element). Beside each, `copy_frac`: the
    kernel's rate over that of a plain device copy (torch's copy or
    conversion kernel) moving the same bytes per element under the same
    protocol, the practical ceiling at that size."""
    import torch
    from wxhip import _lib as L
    out = {}
    specs = [
        ("layernorm_1500x1280_bf16", (1500, 1280), 80),
        # the encoder's own LayerNorm: fp32 residual in, bf16 out, batch 16
        ("layernorm_24000x1280_f32_to_bf16", (24000, 1280), 4),
        ("gelu_erf_1500x5120_bf16", (1500, 5120), 24),
        ("gelu_poly4_1500x5120_bf16", (1500, 5120), 24),
        ("softmax_30000x1500_bf16", (30000, 1500), 4),
    ]
    for name, shape, nset in specs:
        xdt = torch.float32 if "f32_to" in name else torch.bfloat16
        xs = [torch.randn(shape, device=dev.device).to(xdt) for _ in range(nset)]
        ys = [torch.empty(shape, dtype=torch.bfloat16, device=dev.device) for _ in range(nset)]
        g = torch.ones(shape[1], device=dev.device)
        b = torch.zeros(shape[1], device=dev.device)

        def run(i):
            if name.startswith("layernorm"):
                dev.layer_norm(xs[i], g, b, out=ys[i])
            elif name.startswith("gelu_erf"):
                dev.gelu(xs[i], L.WXH_GELU_ERF, out=ys[i])
            elif name.startswith("gelu_poly4"):
                dev.gelu(xs[i], L.WXH_GELU_POLY4_RNE, out=ys[i])
            else:
                dev.softmax_rows(xs[i], out=ys[i])

        def graphed_seconds(fn):
            """Seconds per launch of fn(i) over the rotating set, graph-replayed."""
            for i in range(nset):
                fn(i)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(nset):
                    fn(i)
            graph.replay()
            torch.cuda.synchronize()
            reps = 5
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / 1e3 / (reps * nset)

        per = graphed_seconds(run)
        # the same bytes moved by a plain copy (fp32 -> bf16: the conversion)
        per_copy = graphed_seconds(lambda i: ys[i].copy_(xs[i]))
        nbytes = (xs[0].element_size() + 2) * shape[0] * shape[1]
        gbs = nbytes / per / 1e9
        out[name] = {"us": round(per * 1e6, 2), "GB/s": round(gbs, 1),
                     "hbm_frac": round(gbs * 1e9 / PEAK_HBM, 3),
                     "copy_us": round(per_copy * 1e6, 2),
                     "copy_frac": round(per_copy / per, 3),
                     "working_set_MB": round(nset * nbytes / 1e6)}
        del xs, ys
        torch.cuda.empty_cache()
    return out


def frontend_rate(dev, batch, n_mels):
    """GPU log-mel front end (wxh_log_mel) over `batch` synthetic 30 s clips:
    device time per launch (HIP events over 20 launches). Work: a 201-bin
    real DFT of 3000 frames of 400 samples per clip, in fp64 (199 paired
    terms x 2 FMA per bin, the algorithmic count of a direct real DFT; the
    Goertzel recurrence the kernel runs takes 1.5x that), plus the filterbank."""
    import torch
    g = torch.Generator(device=dev.device).manual_seed(0)
    audio = torch.randn(batch, 480000, generator=g, device=dev.device) * 0.1
    out = torch.empty(batch, n_mels, 3000, dtype=torch.float32, device=dev.device)
    for _ in range(3):
        dev.log_mel(audio, n_mels, out=out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        dev.log_mel(audio, n_mels, out=out)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / 20
    flop = batch * 3000 * (201 * 199 * 4 + 2 * 2 * 201)
    return {"batch": batch, "n_mels": n_mels, "us": round(us, 1),
            "us_per_clip": round(us / batch, 2), "clips_per_s": round(batch / us * 1e6, 1),
            "fp64_tflops": round(flop / us / 1e6, 2),
            "fp64_frac": round(flop / us / 1e6 / PEAK_FP64_TF, 4)}


def cpu_rowops():
    """The oracle's row ops on the host, on the standalone rowops shapes
    (numpy, one core): LayerNorm [1500, 1280] and softmax [30000, 1500] in
    float64, erf-GELU [1500, 5120] as the reference's own fp32 A&S 7.1.26
    evaluation (npu_whisper_encoder.py:284-300). Median of 3; the softmax is
    timed once on its first 3000 rows (a tenth of the shape, about half a
    second), so its "ms" is for that sample. GB/s over the same algorithmic
    bytes as the GPU row-kernel figures (bf16 in and out)."""
    import numpy as np
    from oracle import rowops as OR
    from wxhip import synth
    x = synth.rowop_inputs(seed=0)
    cases = [("layernorm_1500x1280", lambda: OR.layer_norm(x["ln_x"], x["ln_gamma"], x["ln_beta"]),
              x["ln_x"].size, 3),
             ("gelu_erf_1500x5120", lambda: OR.gelu_erf_as_f32(x["gelu_x"]), x["gelu_x"].size, 3),
             ("softmax_30000x1500", lambda: OR.softmax(x["sm_x"][:3000]), 3000 * 1500, 1)]
    out = {}
    for name, fn, n, reps in cases:
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        t = float(np.median(ts))
        out[name] = {"ms": round(t * 1e3, 2), "GB/s": round(4 * n / t / 1e9, 2)}
    out["cores"] = 1
    out["sample"] = "softmax: rows 0..2999 of [30000, 1500]; the others whole"
    return out


def cpu_baseline(W, n_mels):
    """torch fp32 oracle on this host's cores: one warmup and three timed
    forwards of one large-v3 sample (3000 mel frames, seed 0: item 0 of the
    measured batch), with one thread per core this process may run on (its
    CPU affinity; the host's total core count is reported beside it).
    Returns the figures and the oracle's features for that sample."""
    import numpy as np
    import torch
    from oracle import encoder as OE
    from wxhip import synth
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(max(1, usable or 1))
    mel = synth.make_mel(n_mels, 3000, seed=0)
    ref = OE.encoder_torch(W, mel)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        OE.encoder_torch(W, mel)
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    # the front end on the CPU: the oracle's numpy log-mel of one 30 s clip
    from oracle import audio as OA
    clip = np.random.default_rng(0).normal(0, 0.1, 480000).astype(np.float32)
    OA.log_mel_spectrogram(clip, n_mels)
    t0 = time.perf_counter()
    for _ in range(3):
        OA.log_mel_spectrogram(clip, n_mels)
    fe_ms = (time.perf_counter() - t0) / 3 * 1e3
    return {"value": round(3000 / t, 1), "unit": "mel-frames/s",
            "frontend_log_mel_ms_per_clip": round(fe_ms, 2),
            "rowops": cpu_rowops(),
            "cores": torch.get_num_threads(), "host_cores": os.cpu_count(),
            "affinity_cores": usable, "kind": "port",
            "sample": "1 of the 16 large-v3 mels (3000 frames, batch 1), torch fp32 "
                      "encoder restatement, median of 3 after 1 warmup, one thread "
                      "per core of the process's CPU affinity",
            "ms_per_forward": round(t * 1e3, 1)}, ref


def stage_roofline(enc, mel):
    """Per-stage device times of one workload (mean of 3 un-graphed
    profile forwards, HIP events on the library stream) and the roofline of
    its dominant GEMM / attention kernel: algorithmic FLOP per launch over
    its average launch time, against the bf16 dense peak."""
    import numpy as np
    B, _, T = mel.shape
    profs = [enc.profile(mel) for _ in range(3)]
    stages = {k: float(np.mean([p[k] for p in profs])) for k in profs[0]}
    flops = stage_flops(LARGE, B, T)
    launches = stage_launches(LARGE)
    per = {}
    for k, ms in stages.items():
        e = {"ms": round(ms, 3), "us_per_launch": round(ms * 1e3 / launches[k], 2)}
        if k in flops and ms > 0:
            e["mfma_frac"] = round(flops[k] / (ms / 1e3) / PEAK_BF16, 4)
        per[k] = e
    dom = max((k for k in flops), key=lambda k: stages[k])
    s_launch = stages[dom] / 1e3 / launches[dom]
    f_launch = flops[dom] / launches[dom]
    return {"bound": "mfma", "kernel": dom, "achieved": round(f_launch / s_launch / 1e12, 1),
            "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
            "frac": round(f_launch / s_launch / PEAK_BF16, 4), "flop_per_launch": f_launch,
            "avg_launch_us": round(s_launch * 1e6, 2), "batch": int(B), "stages": per}


def int8_line(enc, mel, args, B, T):
    """The same encoder with the int8 GEMM path (per-token activation and
    per-output-channel weight scales, the reference's quantised matmul of
    bench/probe_int8_decode.py:48-74; attention stays bf16): forward time,
    batch-1 latency, per-stage times and the int8 MFMA rate of the GEMMs
    (against MI355X's dense int8 peak, 5.0 POP/s). The out_proj and fc2
    stages include the quantisation of their A operand (the fp32 attention
    output, the fp32 GELU(fc1)); LayerNorm quantises its own output."""
    import numpy as np
    import torch
    from wxhip import synth
    enc.set_int8(True)
    dt, out = time_forward(enc, mel, args.steps, args.warmup)
    assert torch.isfinite(out).all().item()
    profs = [enc.profile(mel) for _ in range(3)]
    stages = {k: float(np.mean([p[k] for p in profs])) for k in profs[0]}
    flops = stage_flops(LARGE, B, T)
    r = {"ms_per_step": round(dt * 1e3, 3), "value": round(B * T / dt, 1),
         "unit": "mel-frames/s", "stages_ms": {k: round(v, 3) for k, v in stages.items()}}
    for k in ("qkv", "out_proj", "fc1", "fc2"):
        if stages.get(k, 0) > 0:
            r[f"{k}_tops"] = round(flops[k] / (stages[k] / 1e3) / 1e12, 1)
            r[f"{k}_i8_frac"] = round(flops[k] / (stages[k] / 1e3) / PEAK_I8, 4)
    if not args.no_latency and T == 3000:
        r["latency_bs1_ms"] = round(
            latency_median(enc, mel[:1].contiguous(), max(args.steps, 20), args.warmup) * 1e3, 3)
    enc.set_int8(False)
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="l16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-rowops", action="store_true")
    ap.add_argument("--no-latency", action="store_true")
    ap.add_argument("--no-int8", action="store_true")
    ap.add_argument("--probe", choices=PROBE_KERNELS, default=None)
    ap.add_argument("--reps", type=int, default=4)
    ap.add_argument("--batch", type=int, default=16)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path "
              "(the encoder would shard as independent batch items, one group per GPU "
              "with replicated weights and no collective; that is not built)",
              file=sys.stderr)
        sys.exit(2)
    if args.probe:
        probe(args.probe, args.reps, args.batch)
        return

    import numpy as np
    import torch
    import wxhip
    from wxhip import synth

    wl = WORKLOADS[args.workload]
    B, T = wl["batch"], wl["n_frames"]
    log(f"weights: large-v3 shape, seed 0 ...")
    t0 = time.perf_counter()
    W = synth.make_weights("large-v3")
    log(f"  {time.perf_counter() - t0:.1f} s")
    dev = wxhip.Device(0)
    # int8 copies of the GEMM weights are made during the upload, for the
    # int8 line below; the measured forward is the bf16 path
    enc = wxhip.HipEncoder(dev, W, int8=not args.no_int8)
    enc.set_int8(False)
    log("weights uploaded")
    mel = torch.from_numpy(synth.make_mel_batch(B, 128, T)).to(dev.device)

    host = {}
    dt, out = time_forward(enc, mel, args.steps, args.warmup, host)
    assert torch.isfinite(out).all().item()
    out0 = out[0].float().cpu().numpy()  # item 0 of the timed forward
    frames = B * T
    log(f"{args.workload}: {dt * 1e3:.2f} ms/forward, {frames / dt:.0f} mel-frames/s")

    # per-stage device time of the same workload (HIP events, library stream)
    profs = [enc.profile(mel) for _ in range(3)]
    stages = {k: float(np.mean([p[k] for p in profs])) for k in profs[0]}
    flops = stage_flops(LARGE, B, T)
    launches = stage_launches(LARGE)
    kern = {}
    for k, ms in stages.items():
        e = {"ms": round(ms, 3), "launches": launches[k]}
        if k in flops and ms > 0:
            tf = flops[k] / (ms / 1e3)
            e.update(tflops=round(tf / 1e12, 1), mfma_frac=round(tf / PEAK_BF16, 4))
        kern[k] = e
    dom = max((k for k in flops), key=lambda k: stages[k])
    per_launch_s = stages[dom] / 1e3 / launches[dom]
    flop_per_launch = flops[dom] / launches[dom]
    achieved = flop_per_launch / per_launch_s / 1e12
    total_flops = sum(flops.values())

    res = {
        "metric": METRIC,
        "value": round(frames / dt, 1),
        "unit": "mel-frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded random-init large-v3-shaped weights N(0,0.02), "
                "log-mels N(-0.3,0.5) clipped to [-1,1.5], seeds 0..15",
        "config": {"workload": wl["name"], "batch": B, "n_frames": T,
                   "ctx": (T - 1) // 2 + 1, "d_model": 1280, "n_head": 20, "n_layer": 32},
        "encoder_tflops": round(total_flops / dt / 1e12, 1),
        "encoder_mfma_frac": round(total_flops / dt / PEAK_BF16, 4),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_BF16, 4),
                     "traffic": TRAFFIC_BYTES[dom][0] if dom in TRAFFIC_BYTES else None,
                     "traffic_source": TRAFFIC_BYTES[dom][1] if dom in TRAFFIC_BYTES else None,
                     "flop_per_launch": flop_per_launch,
                     "avg_launch_us": round(per_launch_s * 1e6, 2)},
        "stages": kern,
        **host,
    }

    if not args.no_latency and args.workload != "l1":
        mel1 = mel[:1].contiguous() if T == 3000 else torch.from_numpy(
            synth.make_mel(128, 3000, 0)[None]).to(dev.device)
        dt1m, _ = time_forward(enc, mel1, max(args.steps, 20), args.warmup)
        dt1 = latency_median(enc, mel1, max(args.steps, 20), 2)
        res["latency_bs1_ms"] = round(dt1 * 1e3, 3)
        res["latency_bs1_ms_mean_back_to_back"] = round(dt1m * 1e3, 3)
        f1 = sum(stage_flops(LARGE, 1, 3000).values())
        res["latency_bs1_mfma_frac"] = round(f1 / dt1 / PEAK_BF16, 4)
        res["roofline_bs1"] = stage_roofline(enc, mel1)
        log(f"l1 latency: {dt1 * 1e3:.2f} ms; {res['roofline_bs1']}")
    elif args.workload == "l1":
        res["latency_bs1_ms"] = round(latency_median(enc, mel, max(args.steps, 20), 2) * 1e3, 3)
        res["latency_bs1_ms_mean_back_to_back"] = round(dt * 1e3, 3)
        res["roofline_bs1"] = stage_roofline(enc, mel)

    if not args.no_int8:
        res["int8"] = int8_line(enc, mel, args, B, T)
        log(f"int8: {res['int8']}")

    res["frontend"] = frontend_rate(dev, B, 128)
    log(f"frontend: {res['frontend']}")
    if not args.no_rowops:
        res["rowops"] = rowop_bandwidth(dev)
        log(f"rowops: {res['rowops']}")

    del enc
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log("cpu baseline (torch fp32, one large-v3 sample) ...")
        res["cpu_baseline"], ref0 = cpu_baseline(W, 128)
        log(f"  {res['cpu_baseline']}")
        if T == 3000:
            # parity of the measured run: its item 0 against the oracle
            a = out0.astype(np.float64).ravel()
            b = np.asarray(ref0, np.float64).ravel()
            res["cosine_item0_vs_oracle"] = round(
                float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b))), 7)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

"""Write the committed golden fixtures (run from the repo root):

    python tests/golden/make_golden.py

poly4_all_bf16.npz            poly4 GELU (g4r RNE and g4 truncation) of every
                              finite bf16 value, from the oracle restatement
                              of kernels/gelu_poly4_eval.inc:27-65 (already
                              cross-checked against oracle/poly4.c)
encoder_tiny_2layer_ctx50.npz tiny-shaped 2-layer encoder, seed-0 weights,
                              mel [80, 100] from seed 0, through the torch
                              fp32 oracle

The fixtures are produced by the oracle in oracle/ (the reference's Python
is not run), so they pin the oracle against regressions and give the GPU tests
a CPU-free expected answer.
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "whisper-xdna_amd")]

from oracle import bf16 as OB  # noqa: E402
from oracle import encoder as OE  # noqa: E402
from oracle import rowops as OR  # noqa: E402
from wxhip import synth  # noqa: E402

HERE = Path(__file__).resolve().parent


def main():
    allv = OB.to_f32(np.arange(65536, dtype=np.uint16))
    finite = allv[np.isfinite(allv)]
    with np.errstate(all="ignore"):
        np.savez_compressed(HERE / "poly4_all_bf16.npz", x_bits=OB.round_rne(finite),
                            rne=OR.gelu_poly4(finite, "rne"), trunc=OR.gelu_poly4(finite, "trunc"))
    W = synth.make_weights("tiny", n_layer=2)
    mel = synth.make_mel(80, 100, seed=0)
    np.savez_compressed(HERE / "encoder_tiny_2layer_ctx50.npz", mel=mel,
                        out=OE.encoder_torch(W, mel))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()

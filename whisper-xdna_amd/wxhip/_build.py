"""Build libwxhip.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m wxhip._build          (from whisper-xdna_amd/)

The library lands next to this file (wxhip/libwxhip.so) so it travels with the
source tree; objects go to whisper-xdna_amd/_build/. Every HIP translation unit
is compiled for gfx950 only, with packed-fp32 instruction selection disabled.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "libwxhip.so"
SOURCES = ["gemm_t256.hip", "gemm_t128.hip", "gemm_t128w8.hip", "gemm_t12864.hip", "gemm.hip",
           "rowops.hip", "attention.hip", "audio.hip", "quant.hip", "capi.cpp"]
ARCH = "gfx950"
# Per-file code generation options. The attention kernel feeds every MFMA
# result straight into VALU work (softmax, rescaling), and the GEMM
# epilogues read every accumulator once; with the accumulators in VGPRs
# (MFMA "VGPR form", supported since gfx90a) neither needs
# v_accvgpr_read/write copies (about 190 VALU slots per 64-key attention
# block).
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
FILE_FLAGS = {"attention.hip": _VGPR_MFMA, "gemm.hip": _VGPR_MFMA, "gemm_t256.hip": _VGPR_MFMA,
              "gemm_t128.hip": _VGPR_MFMA, "gemm_t128w8.hip": _VGPR_MFMA,
              "gemm_t12864.hip": _VGPR_MFMA}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build libwxhip.so)")


def _flags():
    # code object v5: loadable by both the ROCm 7.2 runtime and the 7.0
    # runtime that the torch wheel bundles (whichever the process loaded first)
    return ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
            "-mcode-object-version=5",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
            f"-I{CSRC}", f"-I{ROOT.parent / 'include'}"]


def _compile(src):
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc(), "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)] + _flags() + \
        FILE_FLAGS.get(src, [])
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    noise = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l]
    return obj, "\n".join(noise)


def build(verbose=True):
    """Compile every source and link libwxhip.so. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for obj, warn in results:
        if warn.strip() and verbose:
            print(warn, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}",
           "-mcode-object-version=5", "-o", str(tmp)] + \
          [str(o) for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()

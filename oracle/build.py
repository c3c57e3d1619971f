"""Build the oracle's C restatements (test infrastructure only).

    python -m oracle.build        (from the repo root)

Compiles oracle/poly4.c to oracle/_build/libpoly4_oracle.so with gcc. The
reference's own kernels cannot be built here: they are AIE2 C++ that needs
aie_api/aie.hpp, the peano/llvm-aie toolchain and MLIR-AIE's
lut_based_ops.cpp, none of which exist in this image -- so there is no
oracle/_ref build.
"""
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build"
LIB = OUT / "libpoly4_oracle.so"


def build():
    OUT.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
           str(HERE / "poly4.c"), "-o", str(LIB)]
    subprocess.run(cmd, check=True)
    return LIB


def load():
    import ctypes
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    lib.poly4_gelu.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long,
                               ctypes.c_int, ctypes.c_int]
    lib.poly4_gelu.restype = None
    return lib


def poly4_gelu_c(x, mode="rne", f32_input=False):
    """numpy fp32 array -> uint16 bf16 bits through the C restatement."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    load().poly4_gelu(x.ctypes.data, y.ctypes.data, x.size, 0 if mode == "rne" else 1,
                      int(bool(f32_input)))
    return y


if __name__ == "__main__":
    print(build())

"""ctypes binding of libwxhip.so (declarations mirror include/wxhip.h).

The library is loaded after torch, so the process holds a single HIP runtime
(torch's bundled libamdhip64.so.7, which the library then binds to by
SONAME) and device pointers / streams from torch tensors are valid here.
There is no fallback: if the library is missing or the device is not gfx950,
loading raises ``WxhLibraryError``.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libwxhip.so")

WXH_OK, WXH_ERR_INVALID, WXH_ERR_HIP, WXH_ERR_INJECTED = 0, 1, 2, 3
WXH_ERR_UNSUPPORTED, WXH_ERR_STATE, WXH_ERR_TIMEOUT = 4, 5, 6
WXH_BF16, WXH_F32, WXH_I8 = 0, 1, 2
WXH_GELU_ERF, WXH_GELU_POLY4_RNE, WXH_GELU_POLY4_TRUNC = 0, 1, 2
WXH_EPI_F32, WXH_EPI_BF16, WXH_EPI_BF16_GELU_ERF = 0, 1, 2
WXH_EPI_BF16_GELU_POLY4, WXH_EPI_RESID_F32, WXH_EPI_F32_GELU_ERF = 3, 4, 5
WXH_FAIL_GEMM, WXH_FAIL_ATTN, WXH_FAIL_ROWOP, WXH_FAIL_ENCODER = 1, 2, 4, 8
WXH_FAIL_FRONTEND = 16
WXH_TUNE_GEMM_SPLITK, WXH_TUNE_ATTN_KEYSPLIT = 0, 1

ERROR_NAMES = {1: "invalid argument", 2: "HIP error", 3: "injected failure",
               4: "unsupported", 5: "bad state", 6: "deadline passed"}


class WxhLibraryError(RuntimeError):
    """libwxhip.so is missing or cannot run on this machine."""


class WxhError(RuntimeError):
    """A libwxhip.so entry point returned a non-zero status."""

    def __init__(self, code, fn, msg):
        super().__init__(f"{fn}: {ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


class EncoderDims(C.Structure):
    _fields_ = [("n_mels", C.c_int), ("d_model", C.c_int), ("n_head", C.c_int),
                ("n_layer", C.c_int), ("n_ctx", C.c_int), ("mlp_gelu", C.c_int),
                ("conv_gelu", C.c_int)]


P, I, I64, F, U32 = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_uint32
PP = C.POINTER(C.c_void_p)

# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "wxh_version": [],
    "wxh_last_error": [],
    "wxh_create": [I, PP],
    "wxh_destroy": [P],
    "wxh_set_fail_inject": [P, U32],
    "wxh_get_stream": [P, PP],
    "wxh_synchronize": [P],
    "wxh_set_timeout": [P, I],
    "wxh_set_tuning": [P, I, I],
    "wxh_log_mel": [P, P, I, I, I, P, P],
    "wxh_log_mel_noalloc": [P, P, I, I, I, P, P],
    "wxh_mel_filterbank": [I, P],
    "wxh_layernorm": [P, P, I, I64, P, I64, P, I64, P, P, F, P, I, I64, I, I, P],
    "wxh_gelu": [P, P, I, I64, P, I64, I, I, I, P],
    "wxh_softmax_rows": [P, P, I64, P, I64, I, I, P],
    "wxh_convert_f32_bf16": [P, P, I64, P, I64, I, I, I, P],
    "wxh_gemm_bf16": [P, I, I, I, P, I64, P, I64, P, P, I64, I, P],
    "wxh_quantize_rows": [P, P, I, I64, I, I, P, I64, I, P, I, P],
    "wxh_gemm_i8": [P, I, I, I, P, I64, P, P, I64, P, P, P, I64, I, P],
    "wxh_attention_padded_len": [I],
    "wxh_pack_qkv": [P, P, P, P, I64, I, I, I, P, P, P, P],
    "wxh_attention": [P, P, P, P, I, I, I, F, P, I, I64, P],
    "wxh_encoder_create": [P, C.POINTER(EncoderDims), PP],
    "wxh_encoder_destroy": [P],
    "wxh_encoder_set_weight": [P, C.c_char_p, P, C.POINTER(C.c_int64), I],
    "wxh_encoder_ready": [P],
    "wxh_encoder_forward": [P, P, I, I, P, P],
    "wxh_encoder_forward_host": [P, P, I, I, P],
    "wxh_encoder_set_graph": [P, I],
    "wxh_encoder_enable_int8": [P],
    "wxh_encoder_set_int8": [P, I],
    "wxh_encoder_profile": [P, P, I, I, P, C.POINTER(C.c_float), I],
}
_RESTYPE = {"wxh_version": C.c_char_p, "wxh_last_error": C.c_char_p}

_lib = None


def exported_symbols():
    """Names every declaration in include/wxhip.h maps to (for export checks)."""
    return sorted(SIGNATURES)


def load(require_torch=True):
    """Load libwxhip.so once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if require_torch:
        import torch  # noqa: F401  -- one HIP runtime per process (see above)
    if not LIB_PATH.exists():
        raise WxhLibraryError(
            f"{LIB_PATH} is not built; run `python -m wxhip._build` in "
            f"whisper-xdna_amd/ (or __graft_entry__.build())")
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int)
    _lib = lib
    return lib


def check(code, fn):
    if code != WXH_OK:
        msg = load().wxh_last_error().decode(errors="replace")
        raise WxhError(code, fn, msg)


def call(name, *args):
    """Call entry point `name` and raise WxhError on a non-zero status."""
    check(getattr(load(), name)(*args), name)

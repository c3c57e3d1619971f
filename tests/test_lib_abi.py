"""CPU checks of the C ABI and the host-side logic (no GPU, no kernel launches).

* libwxhip.so loads and exports every function include/wxhip.h declares, and
  the Python binding declares exactly that set;
* entry points fail cleanly (status + message, no crash) on bad handles and
  when no GPU is present;
* host logic: synthetic generators, the rowop op-code table, the MLP chunking,
  and bench.py's one-GPU guard.
"""
import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from wxhip import _lib as L
from wxhip import encoder as E
from wxhip import rowops as R
from wxhip import synth

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wxhip.h"


@pytest.fixture(scope="module")
def lib():
    if not L.LIB_PATH.exists():
        from wxhip import _build
        _build.build(verbose=False)
    return L.load(require_torch=False)


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wxh_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == L.exported_symbols()


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(L.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (wxh_\w+)", out))
    missing = set(header_functions()) - exported
    assert not missing, missing
    for name in header_functions():
        assert getattr(lib, name) is not None


def test_version_and_clean_errors_without_device(lib):
    assert lib.wxh_version().startswith(b"wxhip")
    # null handles: error status and a message, never a crash
    assert lib.wxh_synchronize(None) == L.WXH_ERR_INVALID
    assert b"null" in lib.wxh_last_error()
    rc = lib.wxh_gemm_bf16(None, 1, 1, 8, None, 8, None, 8, None, None, 1, 0, None)
    assert rc == L.WXH_ERR_INVALID
    assert lib.wxh_attention_padded_len(1500) == 1536
    assert lib.wxh_attention_padded_len(512) == 512
    assert lib.wxh_attention_padded_len(1) == 64


def test_create_fails_cleanly_without_gpu(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = lib.wxh_create(0, C.byref(h))
    assert rc != L.WXH_OK and lib.wxh_last_error()


def test_synth_weights_deterministic_and_shaped():
    a = synth.make_weights("tiny", n_layer=2)
    b = synth.make_weights("tiny", n_layer=2)
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])
    assert a["w.conv1.weight"].shape == (384, 80, 3)
    assert a["w.blocks.1.mlp.0.weight"].shape == (1536, 384)
    assert "w.blocks.0.attn.key.bias" not in a
    assert (a["w.blocks.0.attn_ln.weight"] == 1).all() and (a["w.ln_post.bias"] == 0).all()
    s = a["w.blocks.1.attn.query.weight"]
    assert abs(s.std() - 0.02) < 1e-3 and abs(s.mean()) < 1e-3
    from wxhip.native import weight_names
    assert {"w." + n for n in weight_names(2)} == set(a.keys())


def test_synth_mel_and_rowop_inputs():
    m = synth.make_mel(128, 3000, seed=0)
    assert m.shape == (128, 3000) and m.dtype == np.float32
    assert m.min() >= -1.0 and m.max() <= 1.5 and abs(m.mean() - (-0.28)) < 0.05
    bm = synth.make_mel_batch(3, 80, 100)
    np.testing.assert_array_equal(bm[2], synth.make_mel(80, 100, seed=2))
    r = synth.rowop_inputs()
    assert r["ln_x"].shape == (1500, 1280) and r["sm_x"].shape == (30000, 1500)


def test_rowop_table_covers_reference_codes():
    # compile_rowop.py:12-19
    ref_codes = {"ln", "sm", "s2", "s3", "s3w", "s4", "s4w", "gl", "g2", "g3", "g4",
                 "g4f", "g4r", "s4rw"}
    assert set(R.OPS) == ref_codes


def test_prepare_mlp_chunks_like_reference():
    W = synth.add_transposed(synth.make_weights({"n_mels": 8, "d": 1280, "n_head": 20,
                                                 "n_layer": 1, "n_ctx": 16}))
    made = E.prepare_mlp_chunks(W, 1, 1280)
    parts = W["w.blocks.0.mlp.0.parts"]
    assert len(parts) == 4 and all(p[0].shape == (1280, 1280) for p in parts)
    assert len(made) == 8
    np.testing.assert_array_equal(np.concatenate([p[0] for p in parts], 1),
                                  W["w.blocks.0.mlp.0.weight_T"])
    T = synth.add_transposed(synth.make_weights("tiny", n_layer=1))
    assert E.prepare_mlp_chunks(T, 1, 384) == [] and "w.blocks.0.mlp.0.parts" not in T


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in (r.stdout + r.stderr)

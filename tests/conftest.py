import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "whisper-xdna_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run on the MI355X box)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs (large-v3 depth)")


@pytest.fixture(scope="session")
def dev():
    """The libwxhip Device on GPU 0. Skips only when no GPU is visible at all;
    on a GPU machine a missing or broken library is an error, not a skip."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import wxhip
    d = wxhip.Device(0)
    yield d
    torch.cuda.synchronize()


def bits(t):
    """bf16 torch tensor -> uint16 numpy bits."""
    import numpy as np
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def to_dev_bf16(x, dev):
    """fp32 numpy -> bf16 device tensor (RNE, via torch's cast, which is RNE)."""
    import torch
    return torch.from_numpy(x).to(dev.device).to(torch.bfloat16)


def cosine(a, b):
    import numpy as np
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float((a * b).sum() / (np.linalg.norm(a) * np.linalg.norm(b)))


def case(msg):
    """Name the case before a GPU step, flushed, so a crash log shows it."""
    print(f"[case] {msg}", flush=True)


def report(name, **values):
    """Append one JSON line of measured values to $WXH_REPORT when it is set
    (the GPU runs collect cosines and error levels this way)."""
    import json
    path = os.environ.get("WXH_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"case": name, **values}) + "\n")

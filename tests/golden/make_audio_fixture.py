"""Write tests/golden/jfk_3s.npy: 3 s (48000 samples) of the reference's own
test input tests/data/jfk.wav (16 kHz mono 16-bit PCM, public domain), as
int16, starting at 1.0 s. Data only: the log-mel tests decode it with the
reference's conversion (/ 32768) and compare the GPU front end with the
oracle on real speech. Run from the repository root:

    python tests/golden/make_audio_fixture.py /root/reference/tests/data/jfk.wav
"""
import sys
import wave
from pathlib import Path

import numpy as np

src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/data/jfk.wav"
with wave.open(src, "rb") as w:
    assert w.getnchannels() == 1 and w.getsampwidth() == 2 and w.getframerate() == 16000
    pcm = np.frombuffer(w.readframes(w.getnframes()), dtype="<i2")
clip = np.ascontiguousarray(pcm[16000:16000 + 48000])
out = Path(__file__).with_name("jfk_3s.npy")
np.save(out, clip)
print(out, clip.shape, clip.dtype, int(np.abs(clip).max()))

"""The long-recording policy of the reference's server (audio_ctx ladder,
30 s windows, half-second tail rule), restated in wxhip.windows: host logic
on the CPU here, the batched GPU path in tests/test_gpu_audio.py."""
import pytest

from wxhip import windows as WN


def test_ctx_for_rounds_up_onto_the_ladder():
    # serve/npu_stt_server.py:228-236: never less context than asked for
    assert [WN.ctx_for(r) for r in (1, 512, 513, 1000, 1024, 1025, 1499, 1500, 9999)] == \
        [512, 512, 768, 1024, 1024, 1280, 1500, 1500, 1500]
    assert WN.ctx_for(None) == WN.ctx_for(0) == 1500          # absent: the full context
    assert WN.ctx_for(700, ladder=[1024, 512]) == 1024        # unsorted ladders are sorted
    with pytest.raises(ValueError):
        WN.ctx_for(5, ladder=[])


def test_split_windows_tail_rule_and_cap():
    N, SR = WN.N_SAMPLES, WN.SAMPLE_RATE
    assert WN.split_windows(0) == [(0, 0)]                    # empty input: one silent window
    assert WN.split_windows(N) == [(0, N)]
    assert WN.split_windows(N + SR // 2 - 1) == [(0, N)]      # sub-half-second tail dropped
    assert WN.split_windows(N + SR // 2) == [(0, N), (N, SR // 2)]
    assert WN.split_windows(2 * N + 5 * SR) == [(0, N), (N, N), (2 * N, 5 * SR)]
    assert WN.split_windows(5 * N, max_windows=2) == [(0, N), (N, N)]

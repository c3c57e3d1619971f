"""CPU oracle for the Whisper-encoder hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``wxhip``) imports
this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and there only as the
reference answer a result is compared with (or as the timed CPU baseline),
never as something a product path calls.

Modules
-------
bf16      fp32 <-> bf16 bit conversions (round-to-nearest-even and truncation)
rowops    the row-wise definitions: LayerNorm, erf-GELU, poly4-GELU, softmax
encoder   the encoder restated twice: torch fp32 (nn ops) and numpy (im2col)
audio     whisper's log-mel front end (numpy float64 STFT, Slaney filterbank)
int8      the reference's int8 quantised matmul (per-token / per-channel or
          per-tensor scales) and the encoder run with it
poly4.c   an independent C restatement of the poly4 GELU, built by ``build.py``

Every function cites the reference file:line it restates. How each function
is pinned (golden vectors, closed forms, library routines, invariants) is
listed in the tests under ``tests/test_oracle_*.py``; a function with no such
check would be marked "parity unpinned" here -- there is none at present.
"""

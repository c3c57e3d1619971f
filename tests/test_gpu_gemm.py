"""GPU parity of the MFMA GEMM (wxh_gemm_bf16) against an fp64 matmul of the
same bf16-rounded operands (the textbook oracle for a bf16 x bf16 -> fp32
GEMM; RawRT.matmul's contract, rawxrt.py:926-996).

Tolerance: fp32 accumulation of K products can differ from the exact sum by
at most ~K * 2^-24 * sum|a_k w_k|; the gate is 2e-4 * (|A| |W|^T), far below
any indexing or layout error (those are O(1) relative).
"""
import numpy as np
import pytest
import torch

from conftest import bits, case, cosine
from oracle import bf16 as OB
from oracle import rowops as OR
from wxhip import _lib as L

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = OB.rb(rng.normal(0, 1, (M, K)).astype(np.float32))
    W = OB.rb(rng.normal(0, 0.05, (N, K)).astype(np.float32))
    b = rng.normal(0, 0.1, N).astype(np.float32)
    return A, W, b


def _exact(A, W, b=None):
    r = A.astype(np.float64) @ W.astype(np.float64).T
    if b is not None:
        r += b
    return r, np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T


def _dev(x, dev, bf16=True):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev.device)
    return t.to(torch.bfloat16) if bf16 else t


SHAPES = [
    (128, 128, 64),      # one tile
    (1500, 1280, 1280),  # out-proj at batch 1 (M tail: 1500 = 11*128 + 92)
    (1500, 3840, 1280),  # fused QKV
    (300, 384, 240),     # conv1 of tiny: K = 3*80 is not a multiple of 64
    (77, 200, 40),       # ragged everything
    (1, 64, 8),          # smallest
    (1500, 1280, 5120),  # fc2
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_f32_bias(dev, M, N, K):
    case(f"gemm f32+bias M={M} N={N} K={K}")
    A, W, b = _operands(M, N, K, seed=M + N + K)
    C = dev.gemm(_dev(A, dev), _dev(W, dev), _dev(b, dev, False), L.WXH_EPI_F32)
    got = C.cpu().numpy()
    ref, mag = _exact(A, W, b)
    err = np.abs(got - ref)
    bad = err > 2e-4 * mag + 1e-6
    if bad.any():
        i, j = np.argwhere(bad)[0]
        pytest.fail(f"{int(bad.sum())} elements off; first ({i},{j}) got {got[i, j]} "
                    f"want {ref[i, j]}; max err {err.max()}")


def test_gemm_structured_layout(dev):
    """One-hot rows/columns pin the fragment layout: C[m, n] = A[m, k] W[n, k]
    picks exactly one product, so a transposed or shifted fragment shows up
    as a wrong index, not as noise."""
    case("gemm one-hot layout probe")
    M = N = 256
    K = 256
    A = np.zeros((M, K), np.float32)
    W = np.zeros((N, K), np.float32)
    for m in range(M):
        A[m, m % K] = 1.0 + (m % 7)
    for n in range(N):
        W[n, (3 * n) % K] = 1.0 + (n % 5)
    C = dev.gemm(_dev(A, dev), _dev(W, dev), None, L.WXH_EPI_F32).cpu().numpy()
    np.testing.assert_array_equal(C, A @ W.T)


def test_gemm_bf16_and_gelu_epilogues(dev):
    M, N, K = 1500, 1536, 384
    case(f"gemm bf16 epilogues M={M} N={N} K={K}")
    A, W, b = _operands(M, N, K, seed=7)
    ref, mag = _exact(A, W, b)
    a, w, bb = _dev(A, dev), _dev(W, dev), _dev(b, dev, False)
    # the fp32 accumulator itself is gated against the exact sum ...
    acc = dev.gemm(a, w, bb, L.WXH_EPI_F32).cpu().numpy()
    assert (np.abs(acc - ref) <= 2e-4 * mag + 1e-6).all()
    # ... and the bf16 epilogue is exactly RNE of that same accumulator (the
    # summation order does not depend on the epilogue)
    y = bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16))
    np.testing.assert_array_equal(y, OB.round_rne(acc))
    # erf GELU epilogue against the exact GELU of the fp32 accumulator
    yg = bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16_GELU_ERF))
    assert OB.ulp_diff(yg, OB.round_rne(OR.gelu_erf(acc).astype(np.float32))).max() <= 1
    # poly4 (g4f) epilogue: bit-exact given the same fp32 accumulator
    yp = bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16_GELU_POLY4))
    np.testing.assert_array_equal(yp, OR.gelu_poly4(acc, "rne", f32_input=True))


def test_gemm_256_tiles_gelu_and_bf16(dev):
    """An fc1-sized GEMM on the 256x256 tile: 24 x 20 tiles, the last row
    tile partial (checked epilogue) and the others interior (the GELU
    epilogue stores directly, the plain bf16 one through LDS). The main loop
    is the same for every epilogue, so the fp32 accumulator is the
    reference for both; two launches in a row agree."""
    M, N, K = 6100, 5120, 1280
    case(f"gemm 256x256 gelu/bf16 M={M} N={N} K={K}")
    A, W, b = _operands(M, N, K, seed=9)
    a, w, bb = _dev(A, dev), _dev(W, dev), _dev(b, dev, False)
    acc = dev.gemm(a, w, bb, L.WXH_EPI_F32).cpu().numpy()
    rows = np.r_[np.random.default_rng(2).choice(M - 300, 40, replace=False), np.arange(M - 260, M, 13)]
    ref, mag = _exact(A[rows], W, b)
    assert (np.abs(acc[rows] - ref) <= 2e-4 * mag + 1e-6).all()
    yg = bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16_GELU_ERF))
    assert OB.ulp_diff(yg, OB.round_rne(OR.gelu_erf(acc).astype(np.float32))).max() <= 1
    np.testing.assert_array_equal(bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16_GELU_ERF)), yg)
    np.testing.assert_array_equal(bits(dev.gemm(a, w, bb, L.WXH_EPI_BF16)), OB.round_rne(acc))


def test_gemm_residual_epilogue(dev):
    M, N, K = 1500, 1280, 5120
    case(f"gemm residual M={M} N={N} K={K}")
    A, W, b = _operands(M, N, K, seed=11)
    x0 = np.random.default_rng(12).normal(0, 1, (M, N)).astype(np.float32)
    x = _dev(x0, dev, False)
    dev.gemm(_dev(A, dev), _dev(W, dev), _dev(b, dev, False), L.WXH_EPI_RESID_F32, out=x)
    ref, mag = _exact(A, W, b)
    err = np.abs(x.cpu().numpy() - (x0 + ref))
    assert (err <= 2e-4 * mag + 1e-5).all(), err.max()


def test_gemm_strided_views(dev):
    """Row strides != K / N (column bands of wider buffers)."""
    case("gemm strided views")
    A, W, b = _operands(200, 256, 128, seed=3)
    Abig = torch.zeros(200, 512, dtype=torch.bfloat16, device=dev.device)
    Abig[:, 64:192] = _dev(A, dev)
    Cbig = torch.full((200, 1024), 5.0, dtype=torch.float32, device=dev.device)
    dev.gemm(Abig[:, 64:192], _dev(W, dev), None, L.WXH_EPI_F32, out=Cbig[:, 256:512])
    ref, mag = _exact(A, W)
    got = Cbig.cpu().numpy()
    assert (np.abs(got[:, 256:512] - ref) <= 2e-4 * mag + 1e-6).all()
    assert (got[:, :256] == 5.0).all() and (got[:, 512:] == 5.0).all()


def test_gemm_rejects_bad_shapes(dev):
    a = torch.zeros(4, 12, dtype=torch.bfloat16, device=dev.device)
    w = torch.zeros(4, 12, dtype=torch.bfloat16, device=dev.device)
    with pytest.raises(L.WxhError) as ei:
        dev.gemm(a, w)
    assert ei.value.code == L.WXH_ERR_INVALID


def test_hiprt_matmul_plugin(dev):
    """RawRT.matmul's signature: fp32 host A (M,K) @ B (K,N) [+bias]."""
    import wxhip
    case("HipRT.matmul")
    rt = wxhip.HipRT()
    rng = np.random.default_rng(2)
    A = rng.normal(0, 1, (300, 384)).astype(np.float32)
    B = rng.normal(0, 0.05, (384, 640)).astype(np.float32)
    bias = rng.normal(0, 0.1, 640).astype(np.float32)
    rt.register_weights([B, bias])
    out = rt.matmul(A, B, bias=bias)
    ref = OB.rb(A).astype(np.float64) @ OB.rb(B).astype(np.float64) + bias
    assert cosine(out, ref) > 0.999999
    np.testing.assert_allclose(out, ref, rtol=1e-3, atol=1e-3)
    assert rt.calls == 1
    out2 = rt.matmul(A, B, bias=bias)
    np.testing.assert_array_equal(out, out2)


@pytest.mark.parametrize("M,N,K", [(1000, 1000, 640), (1000, 1000, 704), (1500, 1280, 1280),
                                   (1500, 3840, 1280), (1400, 3000, 640), (1500, 5120, 1280),
                                   (1000, 1000, 128), (1000, 1000, 256), (1000, 1000, 384)])
def test_gemm_narrow_tile_epilogues(dev, M, N, K):
    """The batch-1 tile shapes besides 128x128: at most 128 tiles of 128x128
    without a split run on 128x64 tiles (the out-proj shape, and one with
    partial edge tiles in both dimensions), with K-steps of 128 where K
    allows and of 64 otherwise (K = 704), and with fewer K-steps than ring
    slots (K = 128, 256: the prologue issues what exists and waits for all
    of it) or exactly as many (K = 384); 257-512 tiles that fit 256 tiles
    of 128x192 on those (the QKV shape, and one with partial tiles). The
    batch-1 shapes also take the XCD block order (the fc1 shape: 480 tiles
    of 128x128 in 2 x 4 blocks). Every epilogue against the fp64 product of
    the same bf16 operands, the bf16 ones against RNE / the GELU definitions
    of the fp32 result."""
    case(f"gemm 128x64 tiles M={M} N={N} K={K}")
    A, W, b = _operands(M, N, K, seed=M + 7 * N + K)
    Ad, Wd, bd = _dev(A, dev), _dev(W, dev), _dev(b, dev, False)
    ref, mag = _exact(A, W, b)
    acc = dev.gemm(Ad, Wd, bd, L.WXH_EPI_F32).cpu().numpy()
    assert (np.abs(acc - ref) <= 2e-4 * mag + 1e-6).all()
    np.testing.assert_array_equal(bits(dev.gemm(Ad, Wd, bd, L.WXH_EPI_BF16)), OB.round_rne(acc))
    yg = bits(dev.gemm(Ad, Wd, bd, L.WXH_EPI_BF16_GELU_ERF))
    assert OB.ulp_diff(yg, OB.round_rne(OR.gelu_erf(acc).astype(np.float32))).max() <= 1
    x0 = np.random.default_rng(M).normal(0, 1, (M, N)).astype(np.float32)
    x = dev.gemm(Ad, Wd, bd, L.WXH_EPI_RESID_F32, out=_dev(x0, dev, False)).cpu().numpy()
    np.testing.assert_array_equal(x, (x0 + acc).astype(np.float32))


@pytest.mark.parametrize("M,N,K,epi", [(4096 + 100, 4096, 3072, "resid"),
                                       (4096, 4096 + 64, 4096, "bf16"),
                                       (4200, 4096, 3072 + 64, "f32")])
def test_gemm_long_k_asymmetric_ring(dev, M, N, K, epi):
    """At least 256 tiles of 256x256 with K >= 3072 take the ring where A has
    three LDS slots and W two (the batch-16 fc2 kernel); partial edge tiles
    and a K-step count that is not a multiple of 3 included. A sample of
    rows and columns against the fp64 product of the same bf16 operands."""
    case(f"gemm asymmetric ring M={M} N={N} K={K} {epi}")
    A, W, b = _operands(M, N, K, seed=K + N)
    rows = np.r_[0:64, M // 2:M // 2 + 64, M - 64:M]
    cols = np.r_[0:64, N // 2 - 32:N // 2 + 32, N - 64:N]
    ref, mag = _exact(A[rows], W[cols], b[cols])
    Ad, Wd, bd = _dev(A, dev), _dev(W, dev), _dev(b, dev, False)
    if epi == "resid":
        x = np.random.default_rng(1).normal(0, 1, (M, N)).astype(np.float32)
        C = dev.gemm(Ad, Wd, bd, L.WXH_EPI_RESID_F32, out=_dev(x, dev, False))
        got = C.cpu().numpy()[np.ix_(rows, cols)] - x[np.ix_(rows, cols)]
        tol = 2e-4 * mag + 1e-6 + 2.0 ** -22 * np.abs(x[np.ix_(rows, cols)])
    elif epi == "bf16":
        C = dev.gemm(Ad, Wd, bd, L.WXH_EPI_BF16)
        got = OB.to_f32(bits(C))[np.ix_(rows, cols)]
        tol = 2e-4 * mag + 1e-6 + 2.0 ** -8 * np.abs(ref)   # one bf16 rounding
    else:
        C = dev.gemm(Ad, Wd, bd, L.WXH_EPI_F32)
        got = C.cpu().numpy()[np.ix_(rows, cols)]
        tol = 2e-4 * mag + 1e-6
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"{int((err > tol).sum())} off, max err {err.max()}"


def test_gemm_operand_beyond_2gib(dev):
    """A spans more than 2 GiB (900000 rows of K = 1280 bf16, 2.3 GB): each
    tile's buffer descriptor starts at that tile's first row, so the DMA
    kernel addresses the whole operand with 32-bit offsets. Rows on either
    side of the 2 GiB byte offset, and the first and last rows, against the
    fp64 product of the same bf16 operands."""
    M, N, K = 900_000, 64, 1280
    case(f"gemm A beyond 2 GiB M={M} N={N} K={K}")
    g = torch.Generator(device=dev.device).manual_seed(11)
    A = torch.empty(M, K, dtype=torch.bfloat16, device=dev.device)
    for r0 in range(0, M, 100_000):  # in slices: no 4.6 GB fp32 temporary
        r1 = min(M, r0 + 100_000)
        A[r0:r1] = torch.randn(r1 - r0, K, generator=g, device=dev.device).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g, device=dev.device) * 0.05).to(torch.bfloat16)
    C = dev.gemm(A, W, None, L.WXH_EPI_F32)
    edge = (1 << 31) // (K * 2)            # the row holding byte 2^31 of A
    rows = np.array([0, 1, 255, 256, edge - 257, edge - 1, edge, edge + 1, edge + 256,
                     M - 257, M - 1])
    idx = torch.from_numpy(rows).to(dev.device)
    Ar = A.index_select(0, idx).float().cpu().numpy()
    Wf = W.float().cpu().numpy()
    ref, mag = _exact(Ar, Wf)
    got = C.index_select(0, idx).cpu().numpy()
    assert (np.abs(got - ref) <= 2e-4 * mag + 1e-6).all()
    del A, C
    torch.cuda.empty_cache()

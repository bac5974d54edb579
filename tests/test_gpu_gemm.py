"""GPU parity of the quantizer and INT8 GEMM kernels against the CPU oracle.

Bar: quantizer bit-exact; int32 accumulators bit-exact; Plain / BiasOnly /
BiasResidual bit-exact (both sides evaluate the same roundings, fused
multiply-adds written explicitly); BiasGELU within 2e-6 relative (the device
and host tanhf differ in the last bits).  The reference's own acceptance bound
(max |INT8 - FP32 GEMM| < 0.012*sqrt(K), tests/test_int8_gemm.cu:17) is checked
on its own srand(42) inputs.  At 8192^3, where the oracle is too slow, sampled
rows are compared exactly and the whole matrix through a column checksum.
"""
import numpy as np
import pytest

from conftest import pack_i8, rng

pytestmark = pytest.mark.gpu

GPT2_KN = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def problem(M, N, K, seed):
    r = rng(seed)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    return A, W


# ------------------------------------------------------------------ quantizer
# Widths on both sides of each form's limit (one wave per row up to 1024
# columns, 256 threads with the row in registers up to 4096, two passes
# beyond), row counts not a multiple of the four rows per workgroup, and the
# batch-16 prefill sizes.
@pytest.mark.parametrize("rows,cols", [(1, 768), (16, 3072), (4, 8192), (130, 516), (3, 4), (256, 768),
                                       (5, 256), (7, 260), (9, 1024), (6, 1028), (3, 2048), (5, 4096),
                                       (3, 4100), (2048, 768), (2048, 3072)])
def test_quantize_bit_exact(ie, orc, rows, cols):
    r = rng(rows * 31 + cols)
    x = (r.standard_normal((rows, cols)) * r.uniform(1e-3, 1e3, (rows, 1))).astype(np.float32)
    x[0, : min(cols, 8)] = [127.0, -63.5, 62.5, 0.5, -0.5, 1.5, 2.5, -126.5][: min(cols, 8)]  # ties
    if rows > 2:
        x[2] = 0.0  # zero row -> scale 1
    p_gpu, s_gpu = ie.quantize(dev(x))
    p_ref, s_ref = orc.quantize(x)
    assert np.array_equal(host(s_gpu), s_ref)
    assert np.array_equal(host(p_gpu), p_ref)


def test_quantize_reference_inputs(ie, orc):
    g = orc.GlibcRand(42)
    x = g.uniform(512 * 512).reshape(512, 512)
    p_gpu, s_gpu = ie.quantize(dev(x))
    p_ref, s_ref = orc.quantize(x)
    assert np.array_equal(host(p_gpu), p_ref) and np.array_equal(host(s_gpu), s_ref)


# ------------------------------------------------------------------ int32 core
def i32_case(ie, orc, M, N, K, path, seed):
    r = rng(seed)
    A = r.integers(-128, 128, (M, K), dtype=np.int64).astype(np.int8)
    B = r.integers(-128, 128, (N, K), dtype=np.int64).astype(np.int8)
    Ap, Bp = pack_i8(A).reshape(M, K // 4), pack_i8(B).reshape(N, K // 4)
    got = host(ie.int8_gemm(dev(Ap), dev(Bp), epilogue=ie.EPI_I32, path=path))
    want = orc.gemm_i32(Ap, Bp)
    assert np.array_equal(got, want), (M, N, K, path, np.argwhere(got != want)[:5])


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("K,N", GPT2_KN)
def test_i32_gemv_exact(ie, orc, M, K, N):
    i32_case(ie, orc, M, N, K, ie.PATH_GEMV, M * 7 + N + K)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(768, 13), (768, 1001), (768, 1030), (3072, 1001), (3072, 2050)])
def test_i32_gemv_ragged_n(ie, orc, M, K, N):
    """The dot4 GEMV's row groups (4 rows per wave, one- and four-wave
    workgroups) with a partial last group and N on both sides of 1024."""
    i32_case(ie, orc, M, N, K, ie.PATH_GEMV, M * 13 + N + K)


@pytest.mark.parametrize("M", [1, 16, 17, 64, 130, 512])
@pytest.mark.parametrize("K,N", GPT2_KN)
def test_i32_mfma_exact(ie, orc, M, K, N):
    i32_case(ie, orc, M, N, K, ie.PATH_MFMA, M * 11 + N + K)


@pytest.mark.parametrize("M", [1, 3, 4, 5, 8, 9, 13, 16])
def test_i32_lm_head_shape(ie, orc, M):
    """The 768 x 50257 LM head (N % 4 == 1: a partial last 4-feature item):
    the burst GEMV for M <= 8 with one and two activation-row blocks, the
    MFMA GEMV at M = 9-16 (a partial last 16-feature group)."""
    i32_case(ie, orc, M, 50257, 768, ie.PATH_AUTO, 99 + M)


@pytest.mark.parametrize("M,N,K", [(9, 16390, 3072), (16, 16400, 3072), (12, 50257, 768), (16, 20001, 768)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_wide_n_mfma_gemv_epilogues(ie, orc, M, N, K, epi):
    """9 <= M <= 16 with a wide N: the MFMA GEMV at K = 768 (ragged last
    16-feature group), the burst GEMV's 16-row form at K = 3072 (ragged last
    4-feature item); every epilogue; int32 and Plain/Bias/Residual bit-exact,
    GELU to 2e-6."""
    A, W = problem(M, N, K, 17 * M + N + epi)
    r = rng(37 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_GEMV))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None,
                            dev(res) if epi == 3 else None, path=ie.PATH_GEMV))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N", [(2, 16390), (7, 16387)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_burst_gemv_k3072_epilogues(ie, orc, M, N, epi):
    """The burst GEMV at K = 3072 (two 4-feature items per wave), ragged N,
    every epilogue; int32 and Plain/Bias/Residual bit-exact, GELU to 2e-6."""
    K = 3072
    A, W = problem(M, N, K, 13 * M + N + epi)
    r = rng(31 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_GEMV))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None,
                            dev(res) if epi == 3 else None, path=ie.PATH_GEMV))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(5, 7, 4), (3, 9, 20), (19, 33, 36), (1, 1, 16), (129, 257, 80),
                                   (16, 100, 8192), (200, 64, 2048), (7, 3, 0)])
@pytest.mark.parametrize("path", [1, 2])
def test_i32_odd_shapes(ie, orc, M, N, K, path):
    if path == 1 and M > 16:
        pytest.skip("GEMV path takes M <= 16")
    i32_case(ie, orc, M, N, K, path, M + N + K + path)


@pytest.mark.parametrize("M,N", [(2, 8200), (7, 8200), (16, 8192), (8, 4096), (4, 28672), (5, 16400),
                                 (13, 16400), (16, 28672), (1, 8193), (2, 8194), (3, 8195), (6, 4099),
                                 (11, 1027), (16, 30), (9, 5), (4, 1)])
def test_i32_gemv_k8192_paths(ie, orc, M, N):
    """K = 8192 decode GEMV: every block count of activation rows (M 1-4, 5-8,
    9-16), one to four 4-feature items per wave (N = 28672), a partial last
    item (N % 4 != 0) and fewer items than waves (N = 1 .. 30)."""
    i32_case(ie, orc, M, N, 8192, ie.PATH_GEMV, M * 3 + N)


@pytest.mark.parametrize("M,N", [(13, 16400), (3, 8195), (6, 4099)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_k8192_gemv_epilogues(ie, orc, epi, M, N):
    K = 8192
    A, W = problem(M, N, K, 77 + epi)
    r = rng(6 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=ie.PATH_GEMV))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(16, 700, 768), (6, 13, 3072), (9, 1000, 768), (16, 768, 3072)])
@pytest.mark.parametrize("epi", [0, 1, 3])
def test_mfma_gemv_twelve_feature_workgroups(ie, orc, M, N, K, epi):
    """Small N at 5 <= M <= 16: the MFMA GEMV takes 12 features per workgroup
    when 16 would leave CUs idle and 12 fill them (columns 12-15 of each
    workgroup re-read its feature 11 and are not stored), including a
    partial last workgroup (N = 700, 13, 1000); bit-exact."""
    A, W = problem(M, N, K, 41 * M + N + K + epi)
    r = rng(77 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=ie.PATH_GEMV))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    assert np.array_equal(got, want), np.abs(got - want).max()


# ------------------------------------------------------------------ epilogues
@pytest.mark.parametrize("M,K,N,path", [(1, 768, 2304, 1), (16, 3072, 768, 1), (4, 768, 3072, 1),
                                        (64, 768, 2304, 2), (512, 3072, 768, 2), (16, 768, 768, 2)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_epilogues(ie, orc, M, K, N, path, epi):
    A, W = problem(M, N, K, M + K + N + epi)
    r = rng(5 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=path))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(100, 300, 128), (33, 65, 384), (520, 4100, 256), (1000, 2100, 768),
                                   (128, 768, 3072), (97, 700, 640), (130, 770, 2048), (1, 100, 256),
                                   (31, 33, 1024), (40, 200, 8192)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_small_grid_stream_kernel(ie, orc, M, N, K, epi):
    """Mid-size shapes (K % 128 == 0, too few 256x256 tiles for the large-tile
    kernel): while the 32x32 blocks of C fit two per CU (512 on 256 CUs) the
    kernel whose two waves split a block's K and stream it through their own
    LDS rings (one K-group each at
    100x300x128, so the second wave's range is empty; one row, 1x100x256;
    128x768x3072, 130x770x2048, 97x700x640, 33x65x384, 31x33x1024 and
    40x200x8192, 32 groups per wave, past the ring); beyond, the 64x64
    LDS tile kernel (520x4100x256, 1000x2100x768).  Ragged M and N, every
    epilogue; int32 and Plain/Bias/Residual bit-exact, GELU to 2e-6."""
    A, W = problem(M, N, K, 7 * M + N + K + epi)
    r = rng(11 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_MFMA))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(1100, 2100, 768), (2048, 2304, 768)])
@pytest.mark.parametrize("epi", [0, 2, 3, 4])
def test_prefill_sized_wide_gemm(ie, orc, M, N, K, epi):
    """A batch of prompts through the QKV / FFN-up projections: the LDS tile
    kernel with 128x64 tiles (2048x2304, two per CU, two-stage ring) and 64x64
    tiles (1100x2100, three-stage ring); ragged M and N, int32 and
    Plain/Residual bit-exact, GELU to 2e-6."""
    A, W = problem(M, N, K, 3 * M + N + epi)
    r = rng(17 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_MFMA))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(1100, 1000, 128), (1100, 1000, 384), (1200, 1100, 640),
                                   (600, 1100, 128), (600, 1000, 256), (600, 1000, 384), (700, 900, 640)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_tile_kernel_short_k_ring(ie, orc, M, N, K, epi):
    """The 64x64 LDS tile kernel's short-K rings: three stages when the grid
    takes more than one round of workgroups (1100x1000: 288 tiles, 1200x1100:
    342, on 256 CUs) and four when it fits one (600x1100: 180 tiles, 165-160),
    against K stage counts below, equal to and past the ring: one 128-byte
    stage (the prologue and the loop re-read it into the other slots), two,
    three, and five (the ring wraps); ragged M and N, the whole output, int32
    and Plain/Bias/Residual bit-exact, GELU to 2e-6."""
    A, W = problem(M, N, K, 13 * M + N + K + epi)
    r = rng(29 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_MFMA))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("M,N,K", [(2100, 2200, 2048), (2048, 768, 3072), (700, 3000, 4096)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_tile_kernel_long_k(ie, orc, M, N, K, epi):
    """The LDS tile kernel's four-stage ring (K >= 2048) with 128x64 tiles
    (2100x2200x2048) and 64x64 tiles (the FFN-down shape 2048x768x3072,
    700x3000x4096): ragged M and N, every epilogue, on rows around tile edges
    (int32 also through a full column checksum); bit-exact, GELU to 2e-6."""
    A, W = problem(M, N, K, 5 * M + N + K + epi)
    r = rng(23 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    rows = sorted({0, 1, 63, 64, 127, 128, M // 2, M - 65, M - 2, M - 1})
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32, path=ie.PATH_MFMA))
        assert np.array_equal(got[rows], orc.gemm_i32(Ap[rows], Wp))
        a8 = Ap.view(np.int8).reshape(M, K).astype(np.int64)
        w8 = Wp.view(np.int8).reshape(N, K).astype(np.int64)
        assert np.array_equal(got.astype(np.int64).sum(0), w8 @ a8.sum(0))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None,
                            dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    want = orc.gemm(Ap[rows], Wp, sA[rows], sW, epi, bias if epi else None, res[rows] if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got[rows], want, rtol=2e-6, atol=1e-7), np.abs(got[rows] - want).max()
    else:
        assert np.array_equal(got[rows], want), np.abs(got[rows] - want).max()


@pytest.mark.parametrize("path", [1, 2])
def test_residual_may_alias_output(ie, orc, path):
    import torch

    M, K, N = 8, 768, 768
    A, W = problem(M, N, K, 3)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    res = rng(4).standard_normal((M, N)).astype(np.float32)
    want = orc.gemm(Ap, Wp, sA, sW, 3, bias, res)
    C = dev(res)
    ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), 3, dev(bias), C, out=C, path=path)
    assert np.array_equal(host(C), want)


# ------------------------------------------------------------------ reference test
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (512, 512, 512), (1024, 1024, 1024),
                                   (2048, 2048, 2048), (512, 1024, 256)])
def test_reference_k14_cases(ie, orc, M, N, K):
    """tests/test_int8_gemm.cu:97-101 end to end on the GPU (quantize + GEMM)."""
    g = orc.GlibcRand(42)
    A = g.uniform(M * K).reshape(M, K)
    B = g.uniform(K * N).reshape(K, N)
    BT = np.ascontiguousarray(B.T)
    Ap, sA = ie.quantize(dev(A))
    Bp, sB = ie.quantize(dev(BT))
    C = host(ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN))
    ref = orc.gemm_f64(A, B)
    assert np.abs(C - ref).max() < 0.012 * np.sqrt(K)
    if M * N * K <= 1024 ** 3:
        Ap_o, sA_o = orc.quantize(A)
        Bp_o, sB_o = orc.quantize(BT)
        assert np.array_equal(C, orc.gemm(Ap_o, Bp_o, sA_o, sB_o, 0))


# ------------------------------------------------------------------ full size
def test_8192_cube_sampled_rows_and_checksum(ie, orc):
    import torch

    M = N = K = 8192
    gen = torch.Generator(device="cuda").manual_seed(1234)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device="cuda", generator=gen)
    B = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=gen)
    Ap, Bp = A.view(torch.int32), B.view(torch.int32)
    C = ie.int8_gemm(Ap, Bp, epilogue=ie.EPI_I32, path=ie.PATH_MFMA)
    torch.cuda.synchronize()
    # every element through a checksum: sum_m C[m, n] == (sum_m A[m, :]) . B[n, :]
    colsum = A.to(torch.int64).sum(0).cpu().numpy()
    want_cs = B.cpu().numpy().astype(np.int64) @ colsum
    assert np.array_equal(C.to(torch.int64).sum(0).cpu().numpy(), want_cs)
    rowsum = B.to(torch.int64).sum(0).cpu().numpy()
    want_rs = A.cpu().numpy().astype(np.int64) @ rowsum
    assert np.array_equal(C.to(torch.int64).sum(1).cpu().numpy(), want_rs)
    # exact rows from the oracle (first, last, and rows in the middle of tiles)
    rows = np.array([0, 1, 127, 128, 4095, 4097, 8190, 8191])
    a_rows = Ap[torch.from_numpy(rows).cuda()].cpu().numpy()
    want = orc.gemm_i32(a_rows, Bp.cpu().numpy())
    assert np.array_equal(C[torch.from_numpy(rows).cuda()].cpu().numpy(), want)


def test_headline_8192_cube_plain_as_timed(ie, orc):
    """The timed headline itself: bench.headline_inputs (N(0,1) from seed 42,
    quantized per row by the library) and bench_headline's call, Plain
    epilogue, into one C.  That is gemm_i8_256_kernel<Plain, 8 waves, buffer
    copies>: 1024 tiles walked 4 per persistent workgroup, 64 K stages.
    Checked three ways:
      * rows on both edges of every 256-row tile and columns on both edges of
        every 256-column tile, bit-exact against the oracle's Plain GEMM
        (the reference's ((float)acc * sA) * sB, 14_int8_gemm.cu:154);
      * the whole matrix bit-exact against the int32 path's accumulators
        dequantized with the same two fp32 roundings (torch, elementwise),
        the int32 matrix itself held by exact int64 row and column checksums;
      * a second launch into the same C gives the same bits."""
    import torch

    import bench

    M = N = K = 8192
    Ap, Bp, sA, sB = bench.headline_inputs(ie)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN, out=C)  # bench_headline's launch
    torch.cuda.synchronize()
    first = C.clone()
    ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN, out=C)
    torch.cuda.synchronize()
    assert torch.equal(C, first)
    del first

    edges = np.unique(np.concatenate([np.arange(0, M, 256), np.arange(255, M, 256), [4100]]))
    idx = torch.from_numpy(edges).cuda()
    Bp_h, sB_h, sA_h = Bp.cpu().numpy(), sB.cpu().numpy(), sA.cpu().numpy()
    want_rows = orc.gemm(Ap[idx].cpu().numpy(), Bp_h, sA_h[edges], sB_h, 0)
    assert np.array_equal(C[idx].cpu().numpy(), want_rows)
    want_cols = orc.gemm(Ap.cpu().numpy(), Bp_h[edges], sA_h, sB_h[edges], 0)
    assert np.array_equal(C[:, idx].cpu().numpy(), want_cols)

    acc = ie.int8_gemm(Ap, Bp, epilogue=ie.EPI_I32, path=ie.PATH_MFMA)
    torch.cuda.synchronize()
    A8 = Ap.view(torch.int8).view(M, K)
    B8 = Bp.view(torch.int8).view(N, K)
    colsum = A8.to(torch.int64).sum(0).cpu().numpy()
    rowsum = B8.to(torch.int64).sum(0).cpu().numpy()
    assert np.array_equal(acc.to(torch.int64).sum(0).cpu().numpy(), B8.cpu().numpy().astype(np.int64) @ colsum)
    assert np.array_equal(acc.to(torch.int64).sum(1).cpu().numpy(), A8.cpu().numpy().astype(np.int64) @ rowsum)
    deq = (acc.to(torch.float32) * sA[:, None]) * sB[None, :]
    assert torch.equal(C, deq)


@pytest.mark.parametrize("M,N", [(4352, 4352), (4300, 4350)])
@pytest.mark.parametrize("epi", [0, 1, 3])
def test_big_tile_persistent_odd_stages(ie, orc, epi, M, N):
    """Plain / Bias / Residual on the 256x256-tile kernel with more tiles than
    CUs (17 x 17 = 289: persistent workgroups take a second tile) and an odd
    number of 128-byte K stages (K = 640: 5), so a second tile's first stage
    lands in the other LDS slot; rows from both edges of every 256-row tile,
    bit-exact against the oracle."""
    K = 640
    A, W = problem(M, N, K, 70 + epi)
    r = rng(71)
    bias = r.standard_normal(N).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None,
                            dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    rows = sorted(set(range(0, M, 256)) | set(range(255, M, 256)) | {M - 2, M - 1})
    want = orc.gemm(Ap[rows], Wp, sA[rows], sW, epi, bias if epi else None, res[rows] if epi == 3 else None)
    assert np.array_equal(got[rows], want)
    cols = sorted(set(range(0, N, 256)) | set(range(255, N, 256)) | {N - 1})
    want_c = orc.gemm(Ap, Wp[cols], sA, sW[cols], epi, bias[cols] if epi else None,
                      res[:, cols] if epi == 3 else None)
    assert np.array_equal(got[:, cols], want_c)


@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_cfg2_m512_lm_head_shape_full(ie, orc, epi):
    """M = 512 activations x the 768 x 50257 LM-head
    weights (the 256x256-tile kernel, N % 256 = 81), the whole output against
    the oracle: int32 and Plain / Bias / Residual bit-exact, GELU 2e-6."""
    M, K, N = 512, 768, 50257
    A, W = problem(M, N, K, 512 + epi)
    r = rng(55 + epi)
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32))
        assert np.array_equal(got, orc.gemm_i32(Ap, Wp))
        return
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi,
                            dev(bias) if epi else None, dev(res) if epi == 3 else None))
    want = orc.gemm(Ap, Wp, sA, sW, epi, bias if epi else None, res if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7), np.abs(got - want).max()
    else:
        assert np.array_equal(got, want), np.abs(got - want).max()


# ------------------------------------------------------------------ wide (write-dominated) kernel
@pytest.mark.parametrize("M,N", [(17, 50000), (300, 50001), (700, 20000), (1024, 12800), (512, 49153)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_wide_kernel_shapes(ie, orc, epi, M, N):
    """Shapes the write-dominated kernel takes (K = 768, M <= 1024, wide N):
    one to four 256-row panels (700 rows: three panels on a 240-workgroup
    grid), ragged panels and column chunks, M = 17 (one row past the GEMV
    range); rows from both edges of every 32-row block and every panel, all
    columns; int32 and Plain / Bias / Residual bit-exact, GELU 2e-6.  The
    residual epilogue writes in place over the residual, as the engine calls
    it."""
    K = 768
    A, W = problem(M, N, K, 90 + epi + M)
    r = rng(91 + N)
    bias = r.standard_normal(N).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    rows = sorted({m for b in range(0, M, 32) for m in (b, b + 31) if m < M} | {M - 1})
    if epi == 4:
        got = host(ie.int8_gemm(dev(Ap), dev(Wp), epilogue=ie.EPI_I32))
        assert np.array_equal(got[rows], orc.gemm_i32(Ap[rows], Wp))
        return
    out = dev(res) if epi == 3 else None
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None, out, out=out))
    want = orc.gemm(Ap[rows], Wp, sA[rows], sW, epi, bias if epi else None, res[rows] if epi == 3 else None)
    if epi == 2:
        # device vs glibc tanhf: 2e-6 relative plus 1.2e-7 |v| (v = the
        # BiasOnly value), the bound of the drop-in test's GELU check
        v = orc.gemm(Ap[rows], Wp, sA[rows], sW, 1, bias)
        err = np.abs(got[rows].astype(np.float64) - want)
        assert (err <= 2e-6 * np.abs(want) + 1.2e-7 * np.abs(v)).all(), err.max()
    else:
        assert np.array_equal(got[rows], want), np.abs(got[rows] - want).max()


# ------------------------------------------------------------------ 256x256 tiles
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 1024), (3000, 5000, 512), (2304, 8192, 768),
                                   (8192, 3000, 256), (4096, 8448, 384), (4352, 4352, 640)])
def test_big_tile_kernel_exact(ie, orc, M, N, K):
    """Shapes routed to the 256x256-tile kernel (>= 128 tiles, K % 128 == 0),
    including ragged M and N; more tiles than CUs, so persistent workgroups
    take several tiles each (one whose next tile's first K stage lands in the
    other LDS slot: an odd number of K stages, K = 384 and 640); int32 exact
    on sampled rows plus a full column checksum."""
    import torch

    gen = torch.Generator(device="cuda").manual_seed(M + N + K)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device="cuda", generator=gen)
    B = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=gen)
    Ap, Bp = A.view(torch.int32), B.view(torch.int32)
    C = ie.int8_gemm(Ap, Bp, epilogue=ie.EPI_I32, path=ie.PATH_MFMA)
    torch.cuda.synchronize()
    colsum = A.to(torch.int64).sum(0).cpu().numpy()
    assert np.array_equal(C.to(torch.int64).sum(0).cpu().numpy(), B.cpu().numpy().astype(np.int64) @ colsum)
    rows = np.unique(np.clip(np.array([0, 1, 255, 256, M // 2, M - 257, M - 2, M - 1]), 0, M - 1))
    idx = torch.from_numpy(rows).cuda()
    want = orc.gemm_i32(Ap[idx].cpu().numpy(), Bp.cpu().numpy())
    assert np.array_equal(C[idx].cpu().numpy(), want)


@pytest.mark.parametrize("epi", [0, 4])
def test_big_tile_c_not_16_byte_aligned(ie, orc, epi):
    """N % 4 == 0 but C 4 bytes past a 16-byte boundary: the 256x256-tile
    kernel keeps the per-element stores (the quad-transposed 16-byte stores
    need aligned rows), same bits as an aligned C and the oracle."""
    import torch

    M, N, K = 2304, 4096, 768  # 9 x 16 tiles of 256 x 256
    A, W = problem(M, N, K, 60 + epi)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    dt = torch.int32 if epi == 4 else torch.float32
    buf = torch.zeros(M * N + 4, dtype=dt, device="cuda")
    C_off = buf[1:1 + M * N].view(M, N)
    assert C_off.data_ptr() % 16 == 4
    args = (dev(Ap), dev(Wp), dev(sA), dev(sW), epi) if epi != 4 else (dev(Ap), dev(Wp), None, None, epi)
    got = host(ie.int8_gemm(*args, out=C_off, path=ie.PATH_MFMA))
    aligned = host(ie.int8_gemm(*args, path=ie.PATH_MFMA))
    assert np.array_equal(got.view(np.int32), aligned.view(np.int32))
    rows = [0, 1, 255, 256, 1000, M - 1]
    if epi == 4:
        assert np.array_equal(got[rows], orc.gemm_i32(Ap[rows], Wp))
    else:
        assert np.array_equal(got[rows], orc.gemm(Ap[rows], Wp, sA[rows], sW, 0))


@pytest.mark.parametrize("M,N", [(2304, 4100), (2300, 4100), (2300, 4099)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_big_tile_epilogues(ie, orc, epi, M, N):
    """Every epilogue on the 256x256-tile kernel: N % 4 == 0 takes the
    quad-transposed 16-byte stores (full and ragged M), N % 4 != 0 the
    per-element stores; rows from every 256-row tile edge and the ragged end."""
    K = 768
    A, W = problem(M, N, K, 40 + epi)
    r = rng(41)
    bias = r.standard_normal(N).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    got = host(ie.int8_gemm(dev(Ap), dev(Wp), dev(sA), dev(sW), epi, dev(bias) if epi else None,
                            dev(res) if epi == 3 else None, path=ie.PATH_MFMA))
    rows = sorted({0, 1, 2, 3, 5, 8, 31, 127, 128, 255, 256, 1000, 2047, 2048, M - 5, M - 2, M - 1})
    want = orc.gemm(Ap[rows], Wp, sA[rows], sW, epi, bias if epi else None, res[rows] if epi == 3 else None)
    if epi == 2:
        assert np.allclose(got[rows], want, rtol=2e-6, atol=1e-7)
    else:
        assert np.array_equal(got[rows], want)

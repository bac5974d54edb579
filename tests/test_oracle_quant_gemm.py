"""Pins the CPU oracle's quantizer and INT8 GEMM (CPU only).

Each check compares the oracle with something other than its own formula:
libc's rand(), hand-derived known answers, numpy's int64 matmul, fp64 GEMM
within the reference's own tolerance (tests/test_int8_gemm.cu:17, 0.012*sqrt(K)),
and torch's tanh-approximate GELU.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

from conftest import pack_i8, rng, unpack_i8


# ---------------------------------------------------------------- generator
def test_glibc_rand_matches_libc(orc):
    libc = ctypes.CDLL(ctypes.util.find_library("c"))
    for seed in (42, 1, 12345):
        libc.srand(seed)
        want = [libc.rand() for _ in range(2000)]
        g = orc.GlibcRand(seed)
        got = [g.next() for _ in range(2000)]
        assert got == want


def test_reference_uniform_draw(orc):
    # (float)rand() / RAND_MAX * 2.0f - 1.0f, tests/test_int8_gemm.cu:25
    libc = ctypes.CDLL(ctypes.util.find_library("c"))
    libc.srand(42)
    raw = np.array([libc.rand() for _ in range(64)], dtype=np.int64)
    want = (raw.astype(np.float32) / np.float32(2147483647.0)) * np.float32(2.0) - np.float32(1.0)
    got = orc.GlibcRand(42).uniform(64)
    assert np.array_equal(got, want.astype(np.float32))
    assert got.min() >= -1.0 and got.max() <= 1.0
    a, b = orc.GlibcRand(42).uniform_pair(32)
    assert np.array_equal(a, got[0::2]) and np.array_equal(b, got[1::2])


# ---------------------------------------------------------------- quantizer
def test_quant_known_answers(orc):
    x = np.array([
        # row max 127 -> scale 1, inverse 1: q = rint(x), ties to even
        [127.0, -63.5, 62.5, 0.5, -0.5, 1.5, 2.5, -126.5],
        # row max 254 -> scale 2, inverse 0.5
        [254.0, 3.0, 5.0, -7.0, 0.0, -254.0, 1.0, -1.0],
        # all-zero row -> scale 1.0, q = 0
        [0.0] * 8,
        # negative maximum -> -127
        [-127.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
    ], dtype=np.float32)
    packed, scales = orc.quantize(x)
    assert scales.tolist() == [1.0, 2.0, 1.0, 1.0]
    q = unpack_i8(packed)
    assert q[0].tolist() == [127, -64, 62, 0, 0, 2, 2, -126]
    assert q[1].tolist() == [127, 2, 2, -4, 0, -127, 0, 0]
    assert q[2].tolist() == [0] * 8
    assert q[3].tolist() == [-127, 0, 0, 0, 0, 0, 0, 0]
    # little-endian packing: 127 | (-64 & 255) << 8 | 62 << 16 | 0 << 24
    assert packed[0, 0] == 0x003EC07F
    assert packed[3, 0] == 0x00000081


def test_quant_invariants_random(orc):
    r = rng(7)
    for rows, cols in [(1, 768), (16, 3072), (33, 516), (5, 4)]:
        x = (r.standard_normal((rows, cols)) * r.uniform(0.01, 100, (rows, 1))).astype(np.float32)
        packed, scales = orc.quantize(x)
        q = unpack_i8(packed).astype(np.int32)
        amax = np.abs(x).max(axis=1)
        assert np.array_equal(scales, (amax / np.float32(127.0)).astype(np.float32))
        # the largest-magnitude element maps to +-127; -128 never appears
        idx = np.abs(x).argmax(axis=1)
        assert np.all(np.abs(q[np.arange(rows), idx]) == 127)
        assert q.min() >= -127 and q.max() <= 127
        # reconstruction error at most half a step (plus float rounding of x*inv)
        err = np.abs(q * scales[:, None].astype(np.float64) - x)
        assert np.all(err <= scales[:, None] * (0.5 + 1e-5))
        # agrees with numpy's round-half-even of x * (1/scale)
        inv = (np.float32(1.0) / scales).astype(np.float32)
        ref = np.clip(np.rint(x * inv[:, None]), -128, 127).astype(np.int32)
        assert np.array_equal(q, ref)


def test_quant_rejects_bad_cols(orc):
    with pytest.raises(ValueError):
        orc.quantize(np.zeros((2, 6), dtype=np.float32))


# ---------------------------------------------------------------- int32 core
@pytest.mark.parametrize("M,N,K", [(1, 1, 4), (3, 5, 8), (16, 33, 64), (17, 7, 772), (4, 9, 0), (64, 64, 256)])
def test_gemm_i32_vs_numpy(orc, M, N, K):
    r = rng(M * 1000 + N * 10 + K)
    A = r.integers(-128, 128, (M, K), dtype=np.int64).astype(np.int8)
    B = r.integers(-128, 128, (N, K), dtype=np.int64).astype(np.int8)
    acc = orc.gemm_i32(pack_i8(A).reshape(M, K // 4), pack_i8(B).reshape(N, K // 4))
    want = A.astype(np.int64) @ B.astype(np.int64).T
    assert np.array_equal(acc.astype(np.int64), want)


def test_gemm_i32_closed_forms(orc):
    K = 64
    eye = np.eye(K, dtype=np.int8)
    B = rng(3).integers(-128, 128, (K, K), dtype=np.int64).astype(np.int8)
    acc = orc.gemm_i32(pack_i8(eye), pack_i8(B))
    assert np.array_equal(acc, B.T.astype(np.int32))  # I @ B^T^T
    lo = np.full((2, 4096), -128, dtype=np.int8)
    acc = orc.gemm_i32(pack_i8(lo), pack_i8(lo))
    assert np.all(acc == 4096 * 128 * 128)
    hi = np.full((1, 4096), 127, dtype=np.int8)
    assert orc.gemm_i32(pack_i8(hi), pack_i8(lo))[0, 0] == -4096 * 127 * 128


# ---------------------------------------------------------------- epilogues
def _reference_inputs(orc, M, N, K):
    """Exactly the reference test's inputs: srand(42), A then B, U(-1,1)."""
    g = orc.GlibcRand(42)
    A = g.uniform(M * K).reshape(M, K)
    B = g.uniform(K * N).reshape(K, N)
    return A, B


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (512, 512, 512), (512, 1024, 256), (1024, 1024, 1024)])
def test_plain_vs_fp64_reference_tolerance(orc, M, N, K):
    # tests/test_int8_gemm.cu:15-94: INT8 vs FP32 GEMM, max error < 0.012*sqrt(K)
    A, B = _reference_inputs(orc, M, N, K)
    Ap, sA = orc.quantize(A)
    Bp, sB = orc.quantize(np.ascontiguousarray(B.T))
    C = orc.gemm(Ap, Bp, sA, sB, 0)
    ref = orc.gemm_f64(A, B)
    err = np.abs(C - ref).max()
    assert err < 0.012 * np.sqrt(K), err
    # the same sum, rebuilt from the exact int32 core and the scales
    acc = orc.gemm_i32(Ap, Bp)
    assert np.array_equal(C, (acc.astype(np.float32) * sA[:, None]) * sB[None, :])


def test_bias_residual_vs_fp64(orc):
    M, N, K = 16, 768, 3072
    r = rng(11)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    res = r.standard_normal((M, N)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    exact = orc.gemm_f64(A, np.ascontiguousarray(W.T))
    tol = 0.012 * np.sqrt(K) * 0.02 * 4  # per-row scales of N(0,0.02) weights
    Cb = orc.gemm(Ap, Wp, sA, sW, 1, bias)
    assert np.abs(Cb - (exact + bias)).max() < tol
    Cr = orc.gemm(Ap, Wp, sA, sW, 3, bias, res)
    assert np.abs(Cr - (exact + bias + res)).max() < tol
    # bias enters exactly once: Plain + bias within one rounding of BiasOnly
    Cp = orc.gemm(Ap, Wp, sA, sW, 0)
    assert np.allclose(Cb, Cp + bias, rtol=1e-6, atol=1e-6)
    assert np.allclose(Cr, Cb + res, rtol=1e-6, atol=1e-6)


def test_gelu_vs_torch(orc):
    import torch

    M, N, K = 8, 3072, 768
    r = rng(12)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    bias = (r.standard_normal(N) * 2).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Wp, sW = orc.quantize(W)
    pre = orc.gemm(Ap, Wp, sA, sW, 1, bias)  # v = dequant + bias
    got = orc.gemm(Ap, Wp, sA, sW, 2, bias)
    want = torch.nn.functional.gelu(torch.from_numpy(pre).double(), approximate="tanh").numpy()
    assert np.allclose(got, want, rtol=2e-6, atol=2e-7)
    # GELU(0) = 0, GELU(v) ~ v for large v, ~0 for very negative v
    assert np.all(np.abs(got[pre > 6] - pre[pre > 6]) < 1e-4 * np.abs(pre[pre > 6]))
    assert np.all(np.abs(got[pre < -6]) < 1e-4)

"""CPU: the top-k sampler oracle (src/sampler.cu:16-45) pinned against brute
force, closed forms and the softmax distribution, and the library's host-side
draw (ie_top_k_draw) against the oracle, bit for bit."""
import ctypes
import math

import numpy as np
import pytest

from conftest import rng


def brute_topk(row, k):
    order = sorted(range(len(row)), key=lambda i: (-float(row[i]), i))[:k]
    return np.array([row[i] for i in order], dtype=np.float32), np.array(order, dtype=np.int32)


@pytest.mark.parametrize("seed", range(12))
def test_topk_matches_brute_force(orc, seed):
    r = rng(900 + seed)
    n = int(r.integers(1, 60))
    k = int(r.integers(1, n + 1))
    if seed % 3 == 0:
        row = r.integers(0, 4, n).astype(np.float32)  # many ties
    else:
        row = r.standard_normal(n).astype(np.float32)
    if seed % 4 == 1:
        row[r.integers(0, n, max(1, n // 5))] = -np.inf
    if seed % 5 == 2:
        row[::3] = np.where(np.arange(0, n, 3) % 2 == 0, np.float32(0.0), np.float32(-0.0))
    v, i = orc.topk(row[None], k)
    bv, bi = brute_topk(row, k)
    assert np.array_equal(i[0], bi)
    assert np.array_equal(v[0], bv)


def test_topk_large_row_against_numpy(orc):
    row = (rng(5).standard_normal(50257) * 3 - 80).astype(np.float32)
    v, i = orc.topk(row, 50)
    want = np.lexsort((np.arange(row.size), -row.astype(np.float64)))[:50]
    assert np.array_equal(i[0], want)
    assert np.array_equal(v[0], row[want])


def test_topk_k_equals_n_is_a_permutation(orc):
    row = rng(6).standard_normal(37).astype(np.float32)
    v, i = orc.topk(row, 37)
    assert sorted(i[0].tolist()) == list(range(37))
    assert np.all(np.diff(v[0]) <= 0)


def test_rand_unit_is_libc_rand(orc):
    libc = ctypes.CDLL("libc.so.6")
    for seed in (42, 43, 7):
        libc.srand(seed)
        a = libc.rand()
        b = libc.rand()
        assert orc.rand_unit(seed) == np.float32(a) / np.float32(2147483647)
        assert orc.rand_unit(seed, skip=1) == np.float32(b) / np.float32(2147483647)


def test_draw_closed_forms(orc):
    idx = np.array([7, 3, 9], dtype=np.int32)
    # k = 1 always returns the only index
    assert orc.top_k_draw(np.array([1.5], np.float32), idx[:1], 0.8, 0.999) == 7
    # a cold temperature puts all mass on the first entry
    assert orc.top_k_draw(np.array([2.0, 1.0, 0.0], np.float32), idx, 1e-3, 0.9) == 7
    # probabilities 3/4, 1/4 (exp(0) and exp(-ln 3)): the bound sits at 0.75
    vals = np.array([0.0, -math.log(3.0)], dtype=np.float32)
    assert orc.top_k_draw(vals, idx[:2], 1.0, 0.7499) == 7
    assert orc.top_k_draw(vals, idx[:2], 1.0, 0.7501) == 3
    # r = 1.0 (rand() == RAND_MAX rounds to 1.0f) falls through to idx[k-1]
    assert orc.top_k_draw(np.array([0.0, 0.0, 0.0], np.float32), idx, 1.0, 1.0) == 9


def test_draw_frequencies_follow_softmax(orc):
    vals = np.array([1.2, 0.9, 0.2, -0.4, -1.0], dtype=np.float32)
    idx = np.arange(5, dtype=np.int32)
    T, N = 0.8, 20000
    counts = np.zeros(5)
    for s in range(N):
        counts[orc.top_k_draw(vals, idx, T, orc.rand_unit(1000 + s))] += 1
    p = np.exp((vals.astype(np.float64) - vals[0]) / T)
    p /= p.sum()
    chi2 = float(((counts - N * p) ** 2 / (N * p)).sum())
    assert chi2 < 25.0  # 4 degrees of freedom: p(chi2 > 25) ~ 5e-5


def test_library_draw_matches_oracle(ie, orc):
    r = rng(77)
    seeds = iter(range(5000, 6000))
    ie.top_k_draw(np.zeros(1, np.float32), np.zeros(1, np.int32), 1.0, 1)  # last seed != any below
    for case in range(200):
        k = int(r.integers(1, 60))
        vals = np.sort(r.standard_normal(k).astype(np.float32) * 2)[::-1].copy()
        idx = r.permutation(50257)[:k].astype(np.int32)
        T = float(r.choice([0.3, 0.8, 1.0, 1.7]))
        seed = next(seeds)
        got = ie.top_k_draw(vals, idx, T, seed)
        assert got == orc.top_k_draw(vals, idx, T, orc.rand_unit(seed)), case


def test_library_draw_reseeds_only_on_a_new_seed(ie, orc):
    vals = np.linspace(0, -3, 40).astype(np.float32)
    idx = np.arange(40, dtype=np.int32)
    ie.top_k_draw(vals, idx, 1.0, 12345)
    # same seed again: the generator continues (the reference's last_seed rule)
    a = ie.top_k_draw(vals, idx, 1.0, 4242)
    b = ie.top_k_draw(vals, idx, 1.0, 4242)
    c = ie.top_k_draw(vals, idx, 1.0, 4242)
    for skip, got in enumerate((a, b, c)):
        assert got == orc.top_k_draw(vals, idx, 1.0, orc.rand_unit(4242, skip)), skip


def test_library_draw_rejects_bad_arguments(ie):
    with pytest.raises(ie.IeError):
        ie.top_k_draw(np.zeros(0, np.float32), np.zeros(0, np.int32), 1.0, 1)
    with pytest.raises(ie.IeError):
        ie.top_k_draw(np.zeros(2, np.float32), np.zeros(2, np.int32), 0.0, 1)
